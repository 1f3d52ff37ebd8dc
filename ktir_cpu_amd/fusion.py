"""Loop-level fusions: whole `scf.for` loops lowered to one kernel launch.

* K-loop matmul: a loop whose only loop-carried value is an accumulator tile
  updated by ``linalg.matmul ins(A_k, B_k) outs(acc)``, with A_k / B_k loaded
  from access tiles that move by a fixed element offset per iteration (the
  tiled GEMM of the reference's ``examples/triton-ktir/matmul_fwd_ktir.mlir:33-57``
  and ``notebooks/demo_gen_mlir.py:139-152``).  The reference runs one
  `np.matmul` per iteration (``dialects/linalg_ops.py:325-347``); here the
  loop becomes the K dimension of one batched matmul launch.
* Ordered indirect row read-modify-write: a loop of row gathers combined into
  row scatters (``tests/test_indirect_access.py:405-441`` collision order).
* Online-softmax attention: the flash-attention KV loop with loop-carried
  (m, l, acc) becomes one fused MFMA kernel.
"""

from __future__ import annotations

from typing import List, Optional

import numpy as np

from .affine import Box
from .executor import ATile, IATile, NeedEager, Tile, V16Copy

_SCALAR_OPS_PREFIX = ("arith.",)
_SKIP = {"ktdp.load", "arith.extf", "linalg.matmul", "scf.yield"}


def try_fuse_loop(ex, op, lb, st, trips, inits) -> Optional[List]:
    names = op.attributes.get("iter_args", [])
    if ex.collective:
        from .walker import _has_op
        if _has_op(op.regions[0].ops, "ktdp.inter_tile_reduce") or \
                _has_op(op.regions[0].ops, "ktdp.inter_tile_produce"):
            return None      # a ring reduce in the body needs the op-by-op walk
    if not _lx_fits(ex, op.regions[0].ops):
        return None          # let the op-by-op path raise the reference's LX overflow
    if len(names) == 1 and isinstance(inits[0], Tile):
        return _kloop_matmul(ex, op, lb, st, trips, inits[0])
    if not names:
        return _row_rmw(ex, op, lb, st, trips)
    if len(names) == 3:
        return _attention_loop(ex, op, lb, st, trips, inits)
    return None


def _lx_fits(ex, body) -> bool:
    """Upper bound of the LX bytes one iteration of `body` holds (every tile
    result live at once) against the capacity the reference enforces
    (grid.py:292-301)."""
    total = 0
    for o in body:
        for t in o.result_types:
            shape = getattr(t, "shape", None)
            if getattr(t, "kind", None) == "tensor" and shape and all(isinstance(x, int) for x in shape):
                n = 1
                for x in shape:
                    n *= x
                total += n * {"f16": 2, "bf16": 2, "f32": 4, "i64": 8}.get(t.elem, 4)
    return ex.lx_used + total <= ex.lx_capacity


def _kloop_matmul(ex, op, lb, st, trips, init: Tile):
    body = op.regions[0].ops
    acc_name = op.attributes["iter_args"][0]
    if not body or body[-1].op_type != "scf.yield" or len(body[-1].operands) != 1:
        return None
    by_res = {r: o for o in body for r in o.results}
    mm = by_res.get(body[-1].operands[0])
    if mm is None or mm.op_type != "linalg.matmul" or len(mm.operands) != 3 or mm.operands[2] != acc_name:
        return None
    chains = []
    for operand in mm.operands[:2]:
        o = by_res.get(operand)
        cast = None
        if o is not None and o.op_type == "arith.extf":
            cast = o
            o = by_res.get(o.operands[0])
        if o is None or o.op_type != "ktdp.load":
            return None
        chains.append((o, cast))
    allowed = {id(mm), id(body[-1])} | {id(c[0]) for c in chains} | {id(c[1]) for c in chains if c[1]}
    uses = {}
    for o in body:
        for n in o.operands:
            uses[n] = uses.get(n, 0) + 1
    for o in body:
        if id(o) in allowed:
            continue
        if o.op_type == "ktdp.construct_access_tile" or (o.op_type.startswith("arith.") and not o.regions):
            continue
        return None
    for ld, cast in chains:
        if uses.get(ld.results[0], 0) != 1 or (cast and uses.get(cast.results[0], 0) != 1):
            return None
    if uses.get(mm.results[0], 0) != 1:
        return None
    T = int(trips[0]) if len(trips) else 0
    if T < 1 or np.any(trips != T):
        return None
    # probe the access tiles at iterations 0, 1 and T-1
    probe_ops = [o for o in body if id(o) not in allowed]
    iv = op.attributes["iter_var"]

    def tiles_at(j):
        ex.push_scope()
        try:
            ex.set_value(iv, lb + j * st)
            for o in probe_ops:
                ex._exec(o)
            return [ex.get_value(ld.operands[0], peek=True) for ld, _ in chains]
        finally:
            ex.pop_scope()

    try:
        t0 = tiles_at(0)
        t1 = tiles_at(1) if T > 1 else t0
        tl = tiles_at(T - 1)
    except NeedEager:
        return None
    leaves, deltas, shapes = [], [], []
    for (ld, cast), a0, a1, al in zip(chains, t0, t1, tl):
        if not all(isinstance(x, ATile) for x in (a0, a1, al)):
            return None
        if not isinstance(a0.cs, Box) or a0.co is not None or len(a0.cs.extent) != 2:
            return None
        if not (np.array_equal(a0.view.base, a1.view.base) and np.array_equal(a0.view.base, al.view.base)):
            return None
        d = a1.origin - a0.origin
        if d.size and np.any(d != d.flat[0]):
            return None
        dk = int(d.flat[0]) if d.size else 0
        if not np.array_equal(al.origin, a0.origin + (T - 1) * dk):
            return None
        v = a0.view
        if v.space != "HBM":
            return None
        lo_off = sum(int(l) * int(s) for l, s in zip(a0.cs.lo, v.strides))
        shape = a0.cs.extent
        spec, alloc, rel = ex._hbm_leaf(v, a0.origin + lo_off, shape, v.strides)
        for j in range(T):
            ex.log(alloc, False, rel + j * dk, shape, v.strides)
        if cast is not None and v.dtype not in ("f16", "bf16", "f32"):
            return None
        leaves.append((spec, v.dtype))
        deltas.append(dk)
        shapes.append(shape)
    (M, K), (K2, N) = shapes
    if K != K2:
        return None
    dt = "f32" if any(c for _, c in chains) else leaves[0][1]
    from .program import Expr
    a_t = Tile(Expr("ld", dt, (M, K), attr=leaves[0][0]))
    b_t = Tile(Expr("ld", dt, (K, N), attr=leaves[1][0]))
    res = ex._matmul(a_t, b_t, init, ksteps=T, a_k=deltas[0], b_k=deltas[1], a_leaf=leaves[0], b_leaf=leaves[1],
                     name=op.results[0])
    return [res]


# ---------------------------------------------------------------------------
# ordered indirect row read-modify-write (gather + scatter-accumulate)
# ---------------------------------------------------------------------------

_RMW_OPS = {"arith.addf": "ADDF", "arith.subf": "SUBF", "arith.mulf": "MULF", "arith.maximumf": "MAXIMUMF",
            "arith.maxf": "MAXIMUMF", "arith.minimumf": "MINIMUMF", "arith.minf": "MINIMUMF",
            "arith.maxnumf": "MAXNUMF", "arith.minnumf": "MINNUMF"}


def _row_iat(iat_op):
    """(K, D, index expression) if `iat_op` is a row gather ``view[ind(idx[e + d0]), d1]``."""
    a = iat_op.attributes
    shape = tuple(a["shape"])
    subs = a["dim_subscripts"]
    vss = a["variables_space_set"]
    if len(shape) != 2 or a.get("variables_space_order") is not None or len(subs) != 2:
        return None
    if not isinstance(vss, Box) or not vss.is_concrete or tuple(vss.lo) != (0, 0) or tuple(vss.hi) != shape:
        return None
    s0, s1 = subs
    if s0["kind"] != "indirect" or len(s0["idx_exprs"]) != 1:
        return None
    if s1["kind"] != "direct_expr" or s1["subscript"] != ("dim", 1):
        return None
    return shape[0], shape[1], s0["idx_exprs"][0]


def _row_rmw(ex, op, lb, st, trips):
    from . import runtime as rt
    from .affine import evaluate
    from .executor import IATile
    body = op.regions[0].ops
    if not body or body[-1].op_type != "scf.yield" or body[-1].operands:
        return None
    by_res = {r: o for o in body for r in o.results}
    stores = [o for o in body if o.op_type == "ktdp.store"]
    if len(stores) != 1:
        return None
    store = stores[0]
    t_dst = store.operands[1]
    val = by_res.get(store.operands[0])
    if val is None or val.op_type not in _RMW_OPS or len(val.operands) != 2:
        return None
    loads = {}
    for k, name in enumerate(val.operands):
        o = by_res.get(name)
        cast = None
        if o is not None and o.op_type == "arith.extf":
            cast, o = o, by_res.get(o.operands[0])
        if o is None or o.op_type != "ktdp.load":
            return None
        loads[k] = (o, cast)
    dst_k = [k for k, (o, _) in loads.items() if o.operands[0] == t_dst]
    if len(dst_k) != 1 or loads[dst_k[0]][1] is not None:
        return None
    order = 0 if dst_k[0] == 0 else 1
    src_load, src_cast = loads[1 - dst_k[0]]
    dst_load = loads[dst_k[0]][0]
    iat_ops = {o.results[0]: o for o in body if o.op_type == "ktdp.construct_indirect_access_tile"}
    if t_dst not in iat_ops or src_load.operands[0] not in iat_ops or src_load.operands[0] == t_dst:
        return None
    chain = {id(store), id(val), id(src_load), id(dst_load), id(body[-1])} | \
        ({id(src_cast)} if src_cast is not None else set())
    for o in body:
        if id(o) in chain or o.op_type == "ktdp.construct_indirect_access_tile":
            continue
        if o.op_type.startswith("arith.") and not o.regions and o.op_type not in _RMW_OPS \
                and o.op_type != "arith.extf":
            continue
        return None
    rd, rs = _row_iat(iat_ops[t_dst]), _row_iat(iat_ops[src_load.operands[0]])
    if rd is None or rs is None or rd[:2] != rs[:2]:
        return None
    K, D = rd[:2]
    if K > 1024:
        return None
    L = ex.L
    if L == 0 or int(trips.sum()) == 0:
        return []
    iv = op.attributes["iter_var"]
    probe = [o for o in body if id(o) not in chain]

    def iats_at(j):
        jj = np.minimum(j, np.maximum(trips - 1, 0))
        ex.push_scope()
        try:
            ex.set_value(iv, lb + jj * st)
            for o in probe:
                ex._exec(o)
            return ex.get_value(t_dst, peek=True), ex.get_value(src_load.operands[0], peek=True)
        finally:
            ex.pop_scope()

    def pos_of(t: IATile, expr):
        iv_ = t.views[0]
        if len(iv_.shape) != 1 or t.ssa.get("__outer__"):
            raise NeedEager("index view")
        ibpe = rt.ELEM_BYTES[iv_.dtype]
        ia = ex._alloc_of(iv_.base * ibpe)
        ssa = lambda name: t.ssa[name]
        p0 = np.asarray(evaluate(expr, [np.zeros(L, np.int64), np.zeros(L, np.int64)], ssa=ssa), dtype=np.int64)
        p1 = np.asarray(evaluate(expr, [np.ones(L, np.int64), np.zeros(L, np.int64)], ssa=ssa), dtype=np.int64)
        pc = np.asarray(evaluate(expr, [np.zeros(L, np.int64), np.ones(L, np.int64)], ssa=ssa), dtype=np.int64)
        st_ = int(iv_.strides[0])
        if np.any((p1 - p0) * st_ != 1) or np.any(pc != p0):
            raise NeedEager("index positions not unit-stride")
        base = iv_.base - ia.addr // ibpe
        return ia, base + p0 * st_

    try:
        d0, s0 = iats_at(np.zeros(L, np.int64))
        d1, s1 = iats_at(np.ones(L, np.int64))
        dl, sl = iats_at(trips - 1)
        ia_d, pd0 = pos_of(d0, rd[2])
        ia_s, ps0 = pos_of(s0, rs[2])
        _, pd1 = pos_of(d1, rd[2])
        _, ps1 = pos_of(s1, rs[2])
        _, pdl = pos_of(dl, rd[2])
        _, psl = pos_of(sl, rs[2])
    except NeedEager:
        return None
    tm1 = np.maximum(trips - 1, 0)
    dd, ds = pd1 - pd0, ps1 - ps0
    if not (np.array_equal(pdl, pd0 + tm1 * dd) and np.array_equal(psl, ps0 + tm1 * ds)):
        return None
    lane = np.repeat(np.arange(L), trips)
    j = np.arange(int(trips.sum())) - np.repeat(np.cumsum(trips) - trips, trips)
    dst_pos = (pd0[lane] + j * dd[lane]).astype(np.int64)
    src_pos = (ps0[lane] + j * ds[lane]).astype(np.int64)
    vd, vs = d0.parent, s0.parent
    if vd.space != "HBM" or vs.space != "HBM":
        return None
    ad = ex._alloc_of(vd.base * rt.ELEM_BYTES[vd.dtype])
    as_ = ex._alloc_of(vs.base * rt.ELEM_BYTES[vs.dtype])
    if ad is as_ or rt.ELEM_BYTES[ad.dtype] != rt.ELEM_BYTES[vd.dtype] or \
            rt.ELEM_BYTES[as_.dtype] != rt.ELEM_BYTES[vs.dtype]:
        return None
    bd = vd.base - ad.addr // rt.ELEM_BYTES[vd.dtype]
    bs = vs.base - as_.addr // rt.ELEM_BYTES[vs.dtype]
    if np.any(bd != bd[0]) or np.any(bs != bs[0]):
        return None
    dt_dst = vd.dtype
    dt_src = vs.dtype
    # result dtype of the combine op (NumPy promotion as in the op-by-op path)
    src_dt_eff = "f32" if src_cast is not None else dt_src
    res_dt = dt_dst if dt_dst == src_dt_eff else ("bf16" if (dt_dst if order == 0 else src_dt_eff) == "bf16"
                                                   else "f32")
    ex.hazard_flush(ad)
    d = rt.RMW()
    n_inst = len(dst_pos)
    d.n_inst, d.K, d.D = n_inst, K, D
    keep = []
    pb, sb = ex.pool.upload(dst_pos), ex.pool.upload(src_pos)
    keep += [pb, sb]
    d.dst_pos, d.src_pos = pb.ptr, sb.ptr
    d.dst_idx_ptr, d.src_idx_ptr = ex.arena.ptr_of(ia_d), ex.arena.ptr_of(ia_s)
    d.dst_idx_dtype, d.src_idx_dtype = rt.DTYPE_CODE[ia_d.dtype], rt.DTYPE_CODE[ia_s.dtype]
    d.dst_idx_hi, d.src_idx_hi = ia_d.n_elems, ia_s.n_elems
    d.dst_ptr, d.src_ptr = ex.arena.ptr_of(ad), ex.arena.ptr_of(as_)
    d.dst_dtype, d.src_dtype = rt.DTYPE_CODE[dt_dst], rt.DTYPE_CODE[dt_src]
    d.dst_base, d.dst_row, d.dst_col, d.dst_hi = int(bd[0]), int(vd.strides[0]), int(vd.strides[1]), ad.n_elems
    d.src_base, d.src_row, d.src_col, d.src_hi = int(bs[0]), int(vs.strides[0]), int(vs.strides[1]), as_.n_elems
    d.op, d.order, d.dt = rt.op(_RMW_OPS[val.op_type]), order, rt.DTYPE_CODE[res_dt]
    n_rows = max(1, -(-(ad.n_elems - int(bd[0])) // max(int(vd.strides[0]), 1)))
    d.n_rows = n_rows
    # the chain heads and the successor slots: all -1 between calls (the
    # launch resets what it uses), so they are filled once here
    n_ent = max(1, n_inst * K)
    head = rt.DeviceBuffer(n_rows * 4)
    head.upload(np.full(n_rows, -1, np.int32))
    link = rt.DeviceBuffer(n_ent * 8)
    link.upload(np.full(2 * n_ent, -1, np.int32))
    records = ex.pool.temp(n_ent * 8)
    d.head, d.link, d.rows, d.srcs = head.ptr, link.ptr, records.ptr, 0
    keep += [head, link, records]
    grp = id(d)
    z = np.zeros(L, np.int64)
    ex.log(ad, True, z, (1,), (1,), whole=True, group=grp)
    ex.log(as_, False, z, (1,), (1,), whole=True, group=grp)
    ex.log(ia_d, False, z, (1,), (1,), whole=True, group=grp)
    if ia_s is not ia_d:
        ex.log(ia_s, False, z, (1,), (1,), whole=True, group=grp)
    ex.launch("rmw", d, keep)
    return []


# ---------------------------------------------------------------------------
# online-softmax attention loop (flash attention over KV tiles)
# ---------------------------------------------------------------------------

_EW_BIN = {"arith.addf", "arith.subf", "arith.mulf", "arith.divf", "arith.maximumf", "arith.minimumf"}
_EW_UN = {"math.exp"}
_COMM = {"arith.addf", "arith.mulf", "arith.maximumf", "arith.minimumf"}
_SWAP = {"EQ": "EQ", "NE": "NE", "SLT": "SGT", "SGT": "SLT", "SLE": "SGE", "SGE": "SLE",
         "ULTI": "UGTI", "UGTI": "ULTI", "ULEI": "UGEI", "UGEI": "ULEI"}
_NOT = {"EQ": "NE", "NE": "EQ", "SLT": "SGE", "SGE": "SLT", "SLE": "SGT", "SGT": "SLE",
        "ULTI": "UGEI", "UGEI": "ULTI", "ULEI": "UGTI", "UGTI": "ULEI"}


def _is_tensor(op) -> bool:
    t = op.result_types[0] if op.result_types else None
    return getattr(t, "kind", None) == "tensor"


class _Norm:
    """Elementwise normal form of loop-body values.

    Tensor-level arith/math ops and all-parallel ``linalg.generic`` ops whose
    bodies are built from the same ops normalise to one tree form, so the two
    spellings of the online-softmax update (whole-tensor ops as in the
    reference's ``notebooks/demo_gen_mlir.py:471-567`` and generics as in
    ``examples/triton-ktir/paged_attention.mlir:273-392``) match alike.
    ``("v", name)`` is an opaque value, ``("bc", t)`` broadcasts a row vector
    along the columns, ``("red", fn, t)`` reduces the columns of t,
    ``("mask", name)`` is a position-mask generic."""

    def __init__(self, body):
        self.by_res = {r: o for o in body for r in o.results}
        self.used = set()
        self.reduce_inits = []       # (combiner, init SSA name)
        self.masks = {}

    @staticmethod
    def mk(op, *args):
        if op in _COMM:
            args = tuple(sorted(args, key=repr))
        return (op,) + tuple(args)

    def __call__(self, name):
        o = self.by_res.get(name)
        if o is None:
            return ("v", name)
        t = o.op_type
        if t in _EW_BIN and len(o.operands) == 2 and _is_tensor(o):
            self.used.add(id(o))
            return self.mk(t, self(o.operands[0]), self(o.operands[1]))
        if t in _EW_UN and len(o.operands) == 1 and _is_tensor(o):
            self.used.add(id(o))
            return self.mk(t, self(o.operands[0]))
        if t == "linalg.reduce" and o.attributes.get("n_ins") == 1 and list(o.attributes.get("dimensions", [])) == [1] \
                and o.attributes.get("reduce_fn") in ("arith.maximumf", "arith.addf") and len(o.operands) == 2:
            self.used.add(id(o))
            self.reduce_inits.append((o.attributes["reduce_fn"], o.operands[1]))
            return ("red", o.attributes["reduce_fn"], self(o.operands[0]))
        if t == "linalg.generic":
            g = self._generic(o)
            if g is not None:
                self.used.add(id(o))
                return g
        return ("v", name)

    def _generic(self, o):
        a = o.attributes
        n_ins = a.get("n_ins", 0)
        maps = a.get("indexing_maps", [])
        if any(x != "parallel" for x in a.get("iterator_types") or []) or len(maps) != n_ins + 1:
            return None
        region = o.regions[0]
        args = [n for n, _ in region.args]
        if len(args) != n_ins + 1:
            return None
        nd = maps[-1].n_dims
        ident = tuple(("dim", i) for i in range(nd))
        if tuple(maps[-1].exprs) != ident:
            return None
        ops = region.ops
        if any(x.op_type == "linalg.index" for x in ops):
            if n_ins == 1 and tuple(maps[0].exprs) == ident and nd == 2:
                self.masks[o.results[0]] = o
                return ("mask", o.results[0])
            return None
        env = {}
        for i in range(n_ins):
            ex = tuple(maps[i].exprs)
            if ex == ident:
                env[args[i]] = self(o.operands[i])
            elif nd == 2 and ex == (("dim", 0),):
                env[args[i]] = ("bc", self(o.operands[i]))
            else:
                return None
        for x in ops:
            if x.op_type == "linalg.yield":
                return env.get(x.operands[0]) if len(x.operands) == 1 else None
            if any(n not in env for n in x.operands):
                return None
            if x.op_type in _EW_BIN and len(x.operands) == 2:
                env[x.results[0]] = self.mk(x.op_type, env[x.operands[0]], env[x.operands[1]])
            elif x.op_type in _EW_UN and len(x.operands) == 1:
                env[x.results[0]] = self.mk(x.op_type, env[x.operands[0]])
            else:
                return None
        return None


def _peel(by_res, name):
    """Follow extf / collapse_shape / transpose back to a ktdp.load."""
    ops, n_tr, ext = [], 0, False
    while True:
        o = by_res.get(name)
        if o is None:
            return None
        ops.append(o)
        t = o.op_type
        if t == "ktdp.load":
            return o, ops, n_tr, ext
        if t == "arith.extf":
            ext = True
        elif t == "tensor.collapse_shape":
            pass
        elif t == "linalg.transpose":
            if list(o.attributes.get("permutation", [])) != [1, 0]:
                return None
            n_tr += 1
        else:
            return None
        name = o.operands[0]


def _mask_lin(ex, mask_op, L):
    """Evaluate a causal-mask generic body on the host.

    Index values are kept as ``c[lane] + a * (row // g) + b * col``; the
    body must be ``select(cmpi(pred, kpos, qpos), s, neg)`` (either operand
    order of the compare and of the select) with kpos = c_k + col and
    qpos = c_q + row // g (g = 1 unless the row index is divided by a
    constant: the query-token position of grouped query heads, as in
    ``examples/triton-ktir/paged_attention.mlir:273-295``).
    Returns (pred, c_k, c_q, neg, g) or None."""
    region = mask_op.regions[0]
    sv = region.args[0][0]
    env = {}

    def val(n):
        if n in env:
            return env[n]
        v = ex.get_value(n, peek=True)
        if isinstance(v, Tile) or v is None:
            raise NeedEager("mask operand")
        arr = np.broadcast_to(np.asarray(v), (L,))
        if not np.issubdtype(arr.dtype, np.integer):
            raise NeedEager("mask operand")
        return (arr.astype(np.int64), 0, 0, 1)

    cmp = None
    try:
        for x in region.ops:
            t, r = x.op_type, (x.results[0] if x.results else None)
            if t == "linalg.index":
                env[r] = (np.zeros(L, np.int64), 1, 0, 1) if x.attributes.get("dim") == 0 \
                    else (np.zeros(L, np.int64), 0, 1, 1)
            elif t == "arith.constant" and isinstance(x.attributes.get("value"), int) \
                    and not isinstance(x.attributes.get("value"), bool):
                env[r] = (np.full(L, x.attributes["value"], np.int64), 0, 0, 1)
            elif t in ("arith.addi", "arith.subi"):
                a, b = val(x.operands[0]), val(x.operands[1])
                if a[1] and b[1] and a[3] != b[3]:
                    return None
                sg = 1 if t == "arith.addi" else -1
                env[r] = (a[0] + sg * b[0], a[1] + sg * b[1], a[2] + sg * b[2], a[3] if a[1] else b[3])
            elif t == "arith.muli":
                a, b = val(x.operands[0]), val(x.operands[1])
                if a[1] == 0 and a[2] == 0 and np.all(a[0] == a[0][0]):
                    a, b = b, a
                if b[1] != 0 or b[2] != 0 or not np.all(b[0] == b[0][0]):
                    return None
                k = int(b[0][0])
                env[r] = (a[0] * k, a[1] * k, a[2] * k, a[3])
            elif t in ("arith.divui", "arith.divsi", "arith.floordivsi"):
                a, b = val(x.operands[0]), val(x.operands[1])
                if b[1] != 0 or b[2] != 0 or not np.all(b[0] == b[0][0]) or int(b[0][0]) <= 0:
                    return None
                k = int(b[0][0])
                if a[1] == 0 and a[2] == 0:
                    if np.any(a[0] < 0) and t != "arith.floordivsi":
                        return None
                    env[r] = (a[0] // k, 0, 0, 1)
                elif a[2] == 0 and a[1] == 1 and not np.any(a[0]):
                    env[r] = (a[0], 1, 0, a[3] * k)     # (row // g) // k == row // (g k)
                else:
                    return None
            elif t in ("arith.index_cast", "arith.index_castui"):
                env[r] = val(x.operands[0])
            elif t == "arith.cmpi":
                from .walker import CMPI
                p = CMPI.get(x.attributes.get("predicate"))
                if p is None or cmp is not None:
                    return None
                a, b = val(x.operands[0]), val(x.operands[1])
                cmp = (r, p, a, b)
            elif t == "arith.select":
                if cmp is None or x.operands[0] != cmp[0]:
                    return None
                _, p, a, b = cmp
                if (a[1], a[2], b[1], b[2]) == (0, 1, 1, 0):
                    kp, qp = a, b
                elif (a[1], a[2], b[1], b[2]) == (1, 0, 0, 1):
                    kp, qp, p = b, a, _SWAP[p]
                else:
                    return None
                if x.operands[1] == sv:
                    neg_n = x.operands[2]
                elif x.operands[2] == sv:
                    neg_n, p = x.operands[1], _NOT[p]
                else:
                    return None
                nv = np.asarray(ex.get_value(neg_n, peek=True), dtype=np.float64).ravel()
                if nv.size == 0 or np.any(nv != nv[0]) and not np.all(np.isnan(nv)):
                    return None
                env[r] = ("sel", p, kp[0], qp[0], float(nv[0]), qp[3])
            elif t == "linalg.yield":
                y = env.get(x.operands[0]) if len(x.operands) == 1 else None
                if not isinstance(y, tuple) or y[0] != "sel":
                    return None
                return y[1:]
            else:
                return None
    except (NeedEager, KeyError):
        return None
    return None


def _splat_value(ex, name):
    v = ex.get_value(name, peek=True)
    if not isinstance(v, Tile) or v.e.kind != "const":
        return None
    return float(v.e.attr)


N_XCD = 8    # MI355X: workgroup i of a launch runs on XCD i % 8, each XCD with its own L2


def _xcd_order(trips, k_base, v_base, n_xcd=N_XCD):
    """Workgroup -> lane map for the attention launch.

    Lanes reading the same K/V stream (same bases: one attention head) go to
    the same XCD, so the KV tiles they share are fetched into that XCD's L2
    once; streams are spread over the XCDs by total trip count (longest
    first), and inside a stream lanes run longest first, so concurrently
    resident workgroups of one head sweep the same tiles together and the
    short ones fill the tail."""
    L = len(trips)
    if L == 0:
        return np.zeros(0, np.int32)
    _, grp = np.unique(np.stack([k_base, v_base], 1), axis=0, return_inverse=True)
    grp = grp.reshape(-1)
    work = np.bincount(grp, weights=trips.astype(np.float64) + 1.0)
    bins = [[] for _ in range(n_xcd)]
    load = np.zeros(n_xcd)
    for g in np.argsort(-work, kind="stable"):
        x = int(np.argmin(load))
        bins[x].append(int(g))
        load[x] += work[g]
    by_grp = {}
    for lane in np.lexsort((-trips, grp)):
        by_grp.setdefault(int(grp[lane]), []).append(int(lane))
    seqs = [[ln for g in b for ln in by_grp[g]] for b in bins]
    out = []
    pos = [0] * n_xcd
    while len(out) < L:
        for x in range(n_xcd):
            if pos[x] < len(seqs[x]):
                out.append(seqs[x][pos[x]])
                pos[x] += 1
    return np.asarray(out, np.int32)


def _pp_pairs(trips, k_base, v_base, kpos0, n_xcd=N_XCD):
    """Lane pairs for the two-group attention kernel (flat int32, -1 for a
    lane without a partner): lanes of one K/V stream (equal K/V bases and key
    positions) two by two in trip-count order, longest first, the streams
    spread over the XCDs by work as in _xcd_order."""
    L = len(trips)
    if L == 0:
        return np.zeros(0, np.int32)
    _, grp = np.unique(np.stack([k_base, v_base, kpos0], 1), axis=0, return_inverse=True)
    grp = grp.reshape(-1)
    by_grp = {}
    for lane in np.lexsort((-trips, grp)):
        by_grp.setdefault(int(grp[lane]), []).append(int(lane))
    prs = {g: [(ls[i], ls[i + 1] if i + 1 < len(ls) else -1) for i in range(0, len(ls), 2)]
           for g, ls in by_grp.items()}
    work = {g: sum(int(trips[a]) + 1 for a, _ in ps) for g, ps in prs.items()}
    bins = [[] for _ in range(n_xcd)]
    load = np.zeros(n_xcd)
    for g in sorted(work, key=lambda g: -work[g]):
        x = int(np.argmin(load))
        bins[x].append(g)
        load[x] += work[g]
    seqs = [[p for g in b for p in prs[g]] for b in bins]
    out, pos = [], [0] * n_xcd
    n = sum(len(q) for q in seqs)
    while len(out) < n:
        for x in range(n_xcd):
            if pos[x] < len(seqs[x]):
                out.append(seqs[x][pos[x]])
                pos[x] += 1
    return np.asarray(out, np.int32).reshape(-1)


def _attention_loop(ex, op, lb, st, trips, inits):
    """Fuse the online-softmax KV loop of flash attention into one launch
    (``ktir_launch_attention``).  The reference executes it op by op
    (``dialects/linalg_ops.py:325-347`` matmuls, ``:400-596`` generics and
    reductions, ``dialects/math_ops.py`` exp) once per core and iteration."""
    from . import runtime as rt
    from .program import LeafSpec, LaneOff, Expr
    body = op.regions[0].ops
    names = op.attributes["iter_args"]
    if not body or body[-1].op_type != "scf.yield" or len(body[-1].operands) != 3:
        return None
    nz = _Norm(body)
    by_res = nz.by_res
    ys = body[-1].operands
    ia = [i for i, y in enumerate(ys) if y in by_res and by_res[y].op_type == "linalg.matmul"]
    if len(ia) != 1:
        return None
    ia = ia[0]
    mm2 = by_res[ys[ia]]
    if len(mm2.operands) != 3 or mm2.attributes.get("n_ins") != 2:
        return None
    p_name, vf_name, accs_name = mm2.operands
    rest = [i for i in range(3) if i != ia]
    tm = None
    for im in rest:
        t = nz(ys[im])
        if t[0] == "arith.maximumf" and ("v", names[im]) in t[1:]:
            tm = t
            break
    if tm is None:
        return None
    il = rest[0] if im == rest[1] else rest[1]
    m_arg, l_arg, acc_arg = names[im], names[il], names[ia]
    red = tm[2] if tm[1] == ("v", m_arg) else tm[1]
    if red[0] != "red" or red[1] != "arith.maximumf":
        return None
    X = red[2]
    mk = nz.mk
    p_tree = mk("math.exp", mk("arith.subf", X, ("bc", tm)))
    alpha = mk("math.exp", mk("arith.subf", ("v", m_arg), tm))
    if nz(p_name) != p_tree or nz(accs_name) != mk("arith.mulf", ("v", acc_arg), ("bc", alpha)):
        return None
    if nz(ys[il]) != mk("arith.addf", mk("arith.mulf", ("v", l_arg), alpha), ("red", "arith.addf", p_tree)):
        return None
    mask_op = None
    s_tree = X
    if X[0] == "mask":
        mask_op = nz.masks[X[1]]
        s_tree = nz(mask_op.operands[0])
    scale_n = None
    if s_tree[0] == "v":
        qk = s_tree[1]
    elif s_tree[0] == "arith.mulf" and s_tree[1][0] == "v" and s_tree[2][0] == "v":
        a, b = s_tree[1][1], s_tree[2][1]
        if a in by_res and by_res[a].op_type == "linalg.matmul":
            qk, scale_n = a, b
        else:
            qk, scale_n = b, a
    else:
        return None
    mm1 = by_res.get(qk)
    if mm1 is None or mm1.op_type != "linalg.matmul" or len(mm1.operands) != 3 or mm1.attributes.get("n_ins") != 2:
        return None
    q_name, kt_name, s_init = mm1.operands
    if q_name in by_res:
        return None
    pk, pv = _peel(by_res, kt_name), _peel(by_res, vf_name)
    if pk is None or pv is None or pk[2] != 1 or pv[2] != 0 or not pk[3] or not pv[3]:
        return None
    matched = set(nz.used) | {id(mm1), id(mm2), id(body[-1])} | {id(o) for o in pk[1] + pv[1]}
    if mask_op is not None:
        matched.add(id(mask_op))
    uses = {}
    for o in body:
        for n in o.operands:
            uses.setdefault(n, []).append(o)
    for o in body:
        if id(o) in matched:
            continue
        if o.op_type in ("ktdp.construct_access_tile", "ktdp.construct_indirect_access_tile", "tensor.empty", "tensor.splat",
                         "arith.constant") \
                or (o.op_type.startswith("arith.") and not o.regions and not _is_tensor(o)):
            continue
        return None
    # every intermediate feeds only matched ops (no escaping values)
    for o in body:
        if id(o) in matched and o is not body[-1]:
            for r in o.results:
                if any(id(u) not in matched for u in uses.get(r, [])):
                    return None
    L = ex.L
    if L == 0:
        return None
    # initial state: m = -inf, acc = 0 and l = 0 (l may start at any constant
    # in the paged form: examples/triton-ktir/paged_attention.mlir:222 sets 1)
    def const_of(v):
        return float(v.e.attr) if isinstance(v, Tile) and v.e.kind == "const" else None
    l0 = const_of(inits[il])
    if const_of(inits[im]) != -np.inf or const_of(inits[ia]) != 0.0 or l0 is None:
        return None
    q = ex.get_value(q_name, peek=True)
    if not isinstance(q, Tile):
        return None
    probe = [o for o in body if id(o) not in matched]
    iv = op.attributes["iter_var"]
    k_ld, v_ld = pk[0], pv[0]

    def at(j):
        ex.push_scope()
        try:
            ex.set_value(iv, lb + j * st)
            for o in probe:
                ex._exec(o)
            out = {"k": ex.get_value(k_ld.operands[0], peek=True), "v": ex.get_value(v_ld.operands[0], peek=True)}
            out["inits"] = [(fn, _splat_value(ex, n)) for fn, n in nz.reduce_inits]
            out["s_init"] = _splat_value(ex, s_init)
            out["scale"] = _splat_value(ex, scale_n) if scale_n is not None else 1.0
            out["mask"] = _mask_lin(ex, mask_op, L) if mask_op is not None else None
            return out
        finally:
            ex.pop_scope()

    tm1 = np.maximum(trips - 1, 0)
    try:
        p0 = at(np.zeros(L, np.int64))
        p1 = at(np.ones(L, np.int64))
        pl = at(tm1)
    except NeedEager:
        return None
    for fn, v in p0["inits"]:
        if v != (-np.inf if fn == "arith.maximumf" else 0.0):
            return None
    if p0["s_init"] != 0.0 or p0["scale"] is None:
        return None
    if mask_op is not None:
        if p0["mask"] is None or p1["mask"] is None or pl["mask"] is None:
            return None
        pred, ck0, cq0, neg, row_div = p0["mask"]
        _, ck1, cq1, _, g1 = p1["mask"]
        _, ckl, cql, _, gl = pl["mask"]
        kstep = ck1 - ck0
        if np.any(kstep != kstep[0]) or not np.array_equal(cq0, cq1) or not np.array_equal(cq0, cql) \
                or not np.array_equal(ckl, ck0 + tm1 * kstep[0]) or not row_div == g1 == gl:
            return None
        kpos_step = int(kstep[0])
    else:
        pred, ck0, cq0, neg, kpos_step, row_div = "EQ", np.zeros(L, np.int64), np.zeros(L, np.int64), 0.0, 0, 1
    if isinstance(p0["k"], IATile) and isinstance(p0["v"], IATile):
        return _paged_attention(ex, trips, tm1, q, (p0, p1, pl), (pk, pv), l0, (im, il, ia),
                                (mask_op is not None, pred, ck0, cq0, neg, kpos_step, row_div))
    if l0 != 0.0 or row_div != 1:
        return None
    qe = q.e
    if not (qe.kind == "cast" and qe.dtype == "f32" and qe.attr in ("f16", "bf16") and qe.args[0].kind == "ld"
            and qe.args[0].attr.offsets is None):
        return None
    q_leaf = qe.args[0].attr
    AT = 128
    if tuple(q.shape) != (AT, AT) or len(q_leaf.strides) < 2 or q_leaf.strides[-1] != 1 \
            or any(s != 0 for s in q_leaf.strides[:-2]):
        return None
    dtype = q_leaf.dtype
    # K and V tiles: base offsets at iteration 0, uniform step, in bounds for every iteration run
    tiles = {}
    for key, ld in (("k", k_ld), ("v", v_ld)):
        a0, a1, al = p0[key], p1[key], pl[key]
        if not all(isinstance(x, ATile) for x in (a0, a1, al)):
            return None
        if not isinstance(a0.cs, Box) or a0.co is not None:
            return None
        if not (np.array_equal(a0.view.base, a1.view.base) and np.array_equal(a0.view.base, al.view.base)):
            return None
        d = a1.origin - a0.origin
        if np.any(d != d.flat[0]) or not np.array_equal(al.origin, a0.origin + tm1 * d.flat[0]):
            return None
        v = a0.view
        if v.dtype != dtype or v.space != "HBM":
            return None
        ext = tuple(a0.cs.extent)
        big = [i for i, e in enumerate(ext) if e != 1]
        if len(big) != 2 or ext[big[0]] != AT or ext[big[1]] != AT or v.strides[big[1]] != 1:
            return None
        lo_off = sum(int(l) * int(s) for l, s in zip(a0.cs.lo, v.strides))
        spec, alloc, rel = ex._hbm_leaf(v, a0.origin + lo_off, ext, v.strides)
        row, step = int(v.strides[big[0]]), int(d.flat[0])
        run = trips > 0
        lo = rel + np.minimum(0, tm1 * step)
        hi = rel + np.maximum(0, tm1 * step) + (AT - 1) * row + AT - 1
        if np.any(run & ((lo < 0) | (hi >= alloc.n_elems) | (rel % 8 != 0))) or row % 8 or step % 8 or row < AT:
            return None
        tiles[key] = (alloc, rel, row, step)
    q_off = q_leaf.lane.values(L)
    q_row = int(q_leaf.strides[-2])
    run = trips > 0
    if np.any(run & ((q_off < q_leaf.lo) | (q_off + (AT - 1) * q_row + AT - 1 >= q_leaf.hi) | (q_off % 8 != 0))) \
            or q_row % 8 or q_row < AT:
        return None
    # launch
    d = rt.ATTN()
    d.lanes, d.M, d.N, d.D = L, AT, AT, AT
    keep = []

    def up(arr):
        b = ex.pool.upload(np.ascontiguousarray(arr))
        keep.append(b)
        return b.ptr

    d.q_ptr = q_leaf.ptr
    d.k_ptr, d.v_ptr = ex.arena.ptr_of(tiles["k"][0]), ex.arena.ptr_of(tiles["v"][0])
    d.q_base = up(q_off.astype(np.int64))
    d.k_base, d.v_base = up(tiles["k"][1].astype(np.int64)), up(tiles["v"][1].astype(np.int64))
    d.q_row, d.k_row, d.v_row = q_row, tiles["k"][2], tiles["v"][2]
    d.k_step, d.v_step = tiles["k"][3], tiles["v"][3]
    d.trips = up(trips.astype(np.int32))
    if dtype == "bf16":
        # f16 copy of the V elements the loop reads (the kernel runs P @ V in
        # f16 when every one converts exactly), when that range is no larger
        # than the reads themselves
        _, vrel, vrow, vstep = tiles["v"]
        run = trips > 0
        vlo = vrel + np.minimum(0, tm1 * vstep)
        vhi = vrel + np.maximum(0, tm1 * vstep) + (AT - 1) * vrow + AT
        if np.any(run):
            lo_, hi_ = int(vlo[run].min()), int(vhi[run].max())
            if 0 < hi_ - lo_ <= int(trips[run].sum()) * AT * AT:
                v16 = ex.pool.temp((hi_ - lo_) * 2)
                flag = ex.pool.temp(4)
                keep += [v16, flag]
                d.v16_ptr, d.v16_flag, d.v16_lo, d.v16_n = v16.ptr, flag.ptr, lo_, hi_ - lo_
                valloc = tiles["v"][0]
                if any(a is valloc for a in ex.arena.allocs):
                    # replays may reuse the copy (executor.V16Copy says when)
                    ex.plan.v16[id(d)] = V16Copy(valloc, valloc.buf if valloc.buf is not None else ex.arena.buf)
    d.order = up(_xcd_order(trips, tiles["k"][1], tiles["v"][1]))
    pairs = _pp_pairs(trips, tiles["k"][1], tiles["v"][1], ck0.astype(np.int64))
    if len(pairs):
        d.pairs, d.n_pairs = up(pairs), len(pairs) // 2
    d.qpos0, d.kpos0 = up(cq0.astype(np.int64)), up(ck0.astype(np.int64))
    d.kpos_step = kpos_step
    d.scale, d.neg = p0["scale"], neg
    d.causal = 1 if mask_op is not None else 0
    d.pred = rt.K["KTIR_CMP_" + pred]
    d.dtype = rt.DTYPE_CODE[dtype]
    m_buf = ex.pool.temp(L * AT * 4)
    l_buf = ex.pool.temp(L * AT * 4)
    a_buf = ex.pool.temp(L * AT * AT * 4)
    d.m_out, d.l_out, d.acc_out = m_buf.ptr, l_buf.ptr, a_buf.ptr
    keep += [m_buf, l_buf, a_buf, q_leaf]
    tmax = max(int(trips.max()), 1)
    for key in ("k", "v"):
        alloc, rel, row, step = tiles[key]
        ex.log(alloc, False, rel, (tmax, AT, AT), (step, row, 1))
    ex.launch("attn", d, keep)
    ex.attn_pending = dict(desc=d, keep=keep, acc=a_buf, l=l_buf, lanes=L, level=len(ex.levels),
                           body_names=set(names),
                           reads={id(x) for x in (q_leaf.alloc, tiles["k"][0], tiles["v"][0]) if x is not None})
    vec = lambda b: Tile(Expr("ld", "f32", (AT,), attr=LeafSpec(b.ptr, "f32", LaneOff(0, AT), (1,), 0, L * AT,
                                                                  keep=(b,))))
    res = [None, None, None]
    res[im], res[il] = vec(m_buf), vec(l_buf)
    res[ia] = Tile(Expr("ld", "f32", (AT, AT), attr=LeafSpec(a_buf.ptr, "f32", LaneOff(0, AT * AT), (AT, 1), 0,
                                                               L * AT * AT, keep=(a_buf,))))
    return res


def _paged_attention(ex, trips, tm1, q, probes, peeled, l0, slots, mask):
    """Lower the online-softmax loop whose K and V tiles are pages of a
    cache read through a block table (indirect access tiles whose only
    indirect subscript is the page, as in the reference's
    ``examples/triton-ktir/paged_attention.mlir:239-262``) to one
    ``ktir_launch_paged_attention`` launch.  Checked on the host from the
    iterations 0, 1 and the last of every lane: each K / V tile is an N x D
    row-major block at a fixed lane offset plus page * page stride, the
    page's position in the table advances by one fixed step, and Q is one
    strided M x D tile.  Returns the loop results or None (op-by-op walk)."""
    from . import runtime as rt
    from .program import LeafSpec, LaneOff, Expr
    p0, p1, pl = probes
    im, il, ia = slots
    causal, pred, ck0, cq0, neg, kpos_step, row_div = mask
    L = ex.L
    qe = q.e
    if qe.kind == "cast" and qe.dtype == "f32" and qe.attr in ("f16", "bf16") and qe.args[0].kind == "ld":
        ql = qe.args[0].attr
    elif qe.kind == "ld" and qe.dtype == "f32":
        ql = qe.attr
    else:
        return None
    if len(q.shape) != 2 or ql.offsets is not None or ql.winner is not None or len(ql.strides) != 2 \
            or ql.strides[-1] != 1:
        return None
    M, D = (int(x) for x in q.shape)
    kv = {}
    for key, peel in (("k", peeled[0]), ("v", peeled[1])):
        coll = [o for o in peel[1] if o.op_type == "tensor.collapse_shape"]
        if len(coll) != 1 or tuple(getattr(coll[0].result_types[0], "shape", ())) [-1:] != (D,):
            return None
        N = int(coll[0].result_types[0].shape[0])
        parts = []
        for pr in (p0, p1, pl):
            at = pr[key]
            try:
                n, direct, ind = ex.iat_parts(at)
            except (ValueError, NotImplementedError):
                return None
            if n != N * D or len(ind) != 1:
                return None
            iv, pos, stride = ind[0]
            direct = np.broadcast_to(direct, (L, n))
            pos = np.broadcast_to(pos, (L, n))
            if np.any(pos != pos[:, :1]):
                return None
            row = int(direct[0, D] - direct[0, 0]) if N > 1 else D
            expect = direct[:, :1] + (np.arange(N)[:, None] * row + np.arange(D)[None, :]).reshape(1, -1)
            if not np.array_equal(direct, expect):
                return None
            ibpe = rt.ELEM_BYTES[iv.dtype]
            ibase = np.broadcast_to(np.asarray(iv.base, dtype=np.int64), (L,))
            try:
                ta = ex._alloc_of(ibase * ibpe)
                _, alloc, rel = ex._hbm_leaf(at.parent, np.zeros(L, np.int64), (n,), (1,))
            except NotImplementedError:
                return None
            parts.append((alloc, rel + direct[:, 0], row, int(stride), ta, ibase - ta.addr // ibpe + pos[:, 0],
                          iv.dtype, at.parent.dtype, N))
        x0, x1, xl = parts
        if any(x[0] is not x0[0] or x[4] is not x0[4] or x[2:4] != x0[2:4] or not np.array_equal(x[1], x0[1])
               for x in (x1, xl)):
            return None
        multi = trips > 1
        step = 0
        if np.any(multi):
            d_ = (x1[5] - x0[5])[multi]
            if np.any(d_ != d_[0]) or np.any((xl[5] != x0[5] + tm1 * int(d_[0]))[multi]):
                return None
            step = int(d_[0])
        kv[key] = x0[:5] + (x0[5], step) + x0[6:]
    k, v = kv["k"], kv["v"]
    if k[4] is not v[4] or not np.array_equal(k[5], v[5]) or k[6] != v[6] or k[7] != v[7] or k[8] != v[8] \
            or k[9] != v[9] or k[8] not in ("f16", "bf16", "f32") or k[7] not in ("i8", "i16", "i32", "i64"):
        return None
    N = k[9]
    lds = 4 * (M * (D + 8) + N * (D + 8) + N * D + M * N + 3 * M)
    if M * D > 8192 or lds > 160 * 1024 or D % 4:
        return None
    d = rt.PATTN()
    d.lanes, d.M, d.N, d.D = L, M, N, D
    keep = []

    def up(arr):
        b = ex.pool.upload(np.ascontiguousarray(arr))
        keep.append(b)
        return b.ptr

    d.q_ptr, d.q_base = ql.ptr, up(ql.lane.values(L).astype(np.int64))
    d.q_row, d.q_lo, d.q_hi = int(ql.strides[0]), int(ql.lo), int(ql.hi)
    d.q_dtype, d.kv_dtype = rt.DTYPE_CODE[ql.dtype], rt.DTYPE_CODE[k[8]]
    d.k_ptr, d.k_base, d.k_row, d.k_page = ex.arena.ptr_of(k[0]), up(k[1]), k[2], k[3]
    d.v_ptr, d.v_base, d.v_row, d.v_page = ex.arena.ptr_of(v[0]), up(v[1]), v[2], v[3]
    d.k_lo, d.k_hi, d.v_lo, d.v_hi = 0, k[0].n_elems, 0, v[0].n_elems
    d.tbl_ptr, d.tbl_pos, d.tbl_step = ex.arena.ptr_of(k[4]), up(k[5]), k[6]
    d.tbl_lo, d.tbl_hi, d.tbl_dtype = 0, k[4].n_elems, rt.DTYPE_CODE[k[7]]
    d.trips = up(trips.astype(np.int32))
    # lanes of one KV stream (equal K / V lane offsets: one KV head) on one XCD
    d.order = up(_xcd_order(trips, k[1], v[1]))
    d.qpos0, d.kpos0 = up(cq0.astype(np.int64)), up(ck0.astype(np.int64))
    d.kpos_step, d.row_div = kpos_step, row_div
    d.causal, d.pred = int(causal), rt.K["KTIR_CMP_" + pred]
    d.scale, d.neg, d.m0, d.l0 = p0["scale"], neg, -np.inf, l0
    m_buf, l_buf, a_buf = ex.pool.temp(L * M * 4), ex.pool.temp(L * M * 4), ex.pool.temp(L * M * D * 4)
    d.m_out, d.l_out, d.acc_out = m_buf.ptr, l_buf.ptr, a_buf.ptr
    keep += [m_buf, l_buf, a_buf, ql]
    zero = np.zeros(L, np.int64)
    for alloc in (k[0], v[0], k[4]):
        ex.log(alloc, False, zero, (1,), (1,), whole=True)
    ex.launch("pattn", d, keep)
    vec = lambda b: Tile(Expr("ld", "f32", (M,), attr=LeafSpec(b.ptr, "f32", LaneOff(0, M), (1,), 0, L * M,
                                                                 keep=(b,))))
    res = [None, None, None]
    res[im], res[il] = vec(m_buf), vec(l_buf)
    res[ia] = Tile(Expr("ld", "f32", (M, D), attr=LeafSpec(a_buf.ptr, "f32", LaneOff(0, M * D), (D, 1), 0,
                                                             L * M * D, keep=(a_buf,))))
    return res


def _plain_ld(e, ptr, inner):
    """`e` reads a whole attention state buffer at `ptr`: lane stride = one
    lane's block, the two inner strides `inner`, any leading dims of extent 1."""
    if e.kind != "ld" or e.attr.ptr != ptr or e.attr.offsets is not None or e.attr.winner is not None:
        return False
    sh, stv = tuple(e.shape), tuple(e.attr.strides)
    if len(sh) < 2 or any(x != 1 for x in sh[:-2]) or tuple(sh[-2:]) != (128, 128):
        return False
    return stv[-2:] == inner and e.attr.lane.arr is None and e.attr.lane.base == 0


def attention_epilogue(ex, e, dest) -> bool:
    """Fold ``store(cast(acc / l))`` of the loop results of the last fused
    attention launch into that launch (its kernel writes O directly), when
    nothing else still reads acc.  Same operations and roundings as the
    store's own program: f32 division, then rounding to the store type."""
    from . import runtime as rt
    from .walker import _reads
    pend = ex.attn_pending
    if pend is None or ex.eager or ex.L != pend["lanes"] or len(ex.levels) != pend["level"]:
        return False
    x = e
    if x.kind == "cast" and x.attr == "f32":
        x = x.args[0]
    if x.kind != "bin" or x.attr != rt.op("DIVF") or x.dtype != "f32" or len(x.args) != 2:
        return False
    acc_buf, l_buf = pend["acc"], pend["l"]
    a, b = x.args
    if not (_plain_ld(a, acc_buf.ptr, (128, 1)) and a.attr.lane.stride == 128 * 128
            and _plain_ld(b, l_buf.ptr, (1, 0)) and b.attr.lane.stride == 128):
        return False
    if dest.dtype not in ("f32", "bf16", "f16") or dest.offsets is not None or dest.winner is not None:
        return False
    # O is written while other workgroups still read Q, K and V
    if dest.alloc is not None and id(dest.alloc) in pend["reads"]:
        return False
    dsh = tuple(e.shape)
    dst = tuple(dest.strides)
    if len(dst) != len(dsh) or dst[-1] != 1 or any(s_ != 1 for s_ in dsh[:-2]):
        return False
    L = ex.L
    o_row = int(dst[-2])
    offs = dest.lane.values(L)
    if np.any(offs < dest.lo) or np.any(offs + 127 * o_row + 127 >= dest.hi) or np.any(offs % 8) or o_row % 8 \
            or o_row < 128:
        return False
    d = pend["desc"]
    # acc stays needed if any live value other than this store still reads it
    # (the loop's own iter_args are not visible after the loop)
    acc_live = False
    for fr in ex.frames:
        for name, v in fr.vals.items():
            if name in pend["body_names"] or not isinstance(v, Tile) or v.e is e:
                continue
            if any(n.attr.ptr == acc_buf.ptr for n in _walk_ld(v.e)):
                acc_live = True
    ob = ex.pool.upload(np.ascontiguousarray(offs.astype(np.int64)))
    pend["keep"].extend([ob, dest])
    d.o_ptr, d.o_base, d.o_row = dest.ptr, ob.ptr, o_row
    d.o_dtype = rt.DTYPE_CODE[dest.dtype]
    if not acc_live:
        d.acc_out = 0
    ex.attn_pending = None
    return True


def _walk_ld(e):
    from .program import walk
    return [n for n in walk(e) if n.kind == "ld"]


# ---------------------------------------------------------------------------
# matmul result stored straight from the MFMA kernel
# ---------------------------------------------------------------------------

def _ssa_index(ex):
    """Static facts of the running function's SSA values: how many operands
    name each value anywhere in the function, the block (op list) each value
    is defined in, and the blocks of its uses."""
    idx = getattr(ex, "_ssa", None)
    if idx is not None:
        return idx
    uses, use_blk, def_blk = {}, {}, {}

    def walk(ops):
        b = id(ops)
        for o in ops:
            for n in o.results:
                def_blk[n] = b
            for n in o.operands:
                uses[n] = uses.get(n, 0) + 1
                use_blk.setdefault(n, []).append((o, b))
            for r in o.regions:
                walk(r.ops)

    walk(ex.fn.operations)
    ex._ssa = (uses, use_blk, def_blk)
    return ex._ssa


def _sole_use(ssa, name, op_type):
    """The one op (of type `op_type`) that uses `name`, when that use is in
    the block defining `name` (so it runs once per definition)."""
    uses, use_blk, def_blk = ssa
    if uses.get(name, 0) != 1 or name not in def_blk:
        return None
    o, b = use_blk[name][0]
    return o if o.op_type == op_type and b == def_blk[name] else None


def mm_epilogue(ex, store_op, val, dest, alloc, shape) -> bool:
    """Fold ``store(truncf(C))`` (or ``store(C)``) of the last matmul launch's
    result C into that launch: its kernel then rounds the f32 sums to the
    store's dtype and writes the destination directly.  Taken only when the
    store (through at most one truncf) is the one use of C, both in C's own
    block, the matmul is the last launch recorded, and nothing live reads the
    destination.  Same roundings as the store's own program: the f32 result,
    then one rounding to the destination dtype."""
    from . import runtime as rt
    from .program import _fill_leaf
    from .walker import _reads
    pend = ex.mm_pending
    if pend is None or ex.eager or ex.L != pend["lanes"] or len(ex.levels) != pend["level"] \
            or len(ex.plan.launches) != pend["n"]:
        return False
    ssa = _ssa_index(ex)
    sname = store_op.operands[0]
    if _sole_use(ssa, sname, "ktdp.store") is not store_op:
        return False
    e = val.e
    cname = sname
    if e.kind == "cast":
        if e.attr != "f32" or e.dtype != dest.dtype:
            return False
        tr = _sole_use(ssa, pend["name"], "arith.truncf")
        if tr is None or tr.results[0] != sname:
            return False
        cname = pend["name"]
        e = e.args[0]
    elif e.dtype != dest.dtype:
        return False
    if cname != pend["name"]:
        return False
    M, N, L = pend["M"], pend["N"], ex.L
    buf = pend["buf"]
    if e.kind != "ld" or e.dtype != "f32" or e.attr.ptr != buf.ptr or e.attr.offsets is not None \
            or e.attr.winner is not None or tuple(e.shape) != (M, N) or tuple(e.attr.strides) != (N, 1) \
            or e.attr.lane.arr is not None or e.attr.lane.base != 0 or e.attr.lane.stride != M * N:
        return False
    d = pend["desc"]
    if d.accumulate == 1 or d.round_dt != rt.DTYPE_CODE["f32"]:
        return False
    # the kernel writes the destination while its workgroups still read the
    # operands: never into a tensor the product reads
    if id(alloc) in pend["reads"]:
        return False
    if dest.dtype not in ("f32", "f16", "bf16") or dest.offsets is not None or dest.winner is not None:
        return False
    if tuple(val.shape) != (M, N) or tuple(shape) != (M, N) or len(dest.strides) != 2 or dest.strides[1] != 1:
        return False
    row = int(dest.strides[0])
    offs = dest.lane.values(L)
    if row < N or np.any(offs < dest.lo) or np.any(offs + (M - 1) * row + N - 1 >= dest.hi):
        return False
    for fr in ex.frames:
        for v in fr.vals.values():
            if isinstance(v, Tile) and v is not val and _reads(v.e, alloc):
                return False
    _fill_leaf(d.c, dest, L, 2, pend["keep"])
    pend["keep"].append(dest)
    ex.mm_pending = None
    return True
