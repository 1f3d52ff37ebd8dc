"""Loop-level fusions: whole `scf.for` loops lowered to one kernel launch.

* K-loop matmul: a loop whose only loop-carried value is an accumulator tile
  updated by ``linalg.matmul ins(A_k, B_k) outs(acc)``, with A_k / B_k loaded
  from access tiles that move by a fixed element offset per iteration (the
  tiled GEMM of the reference's ``examples/triton-ktir/matmul_fwd_ktir.mlir:33-57``
  and ``notebooks/demo_gen_mlir.py:139-152``).  The reference runs one
  `np.matmul` per iteration (``dialects/linalg_ops.py:325-347``); here the
  loop becomes the K dimension of one batched matmul launch.
"""

from __future__ import annotations

from typing import List, Optional

import numpy as np

from .affine import Box
from .executor import ATile, NeedEager, Tile

_SCALAR_OPS_PREFIX = ("arith.",)
_SKIP = {"ktdp.load", "arith.extf", "linalg.matmul", "scf.yield"}


def try_fuse_loop(ex, op, lb, st, trips, inits) -> Optional[List]:
    names = op.attributes.get("iter_args", [])
    if not _lx_fits(ex, op.regions[0].ops):
        return None          # let the op-by-op path raise the reference's LX overflow
    if len(names) == 1 and isinstance(inits[0], Tile):
        return _kloop_matmul(ex, op, lb, st, trips, inits[0])
    if not names:
        return _row_rmw(ex, op, lb, st, trips)
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
    res = ex._matmul(a_t, b_t, init, ksteps=T, a_k=deltas[0], b_k=deltas[1], a_leaf=leaves[0], b_leaf=leaves[1])
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
    dst_t = ex.get_value(dst_load.results[0], peek=True) if False else None
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
    head = ex.pool.temp(n_rows * 4)
    scratch = [ex.pool.temp(max(1, n_inst * K) * 4) for _ in range(3)]
    owners = ex.pool.temp((4 + 4 * n_inst * K) * 4)
    d.head, d.link, d.rows, d.srcs = head.ptr, scratch[0].ptr, scratch[1].ptr, scratch[2].ptr
    d.owners = owners.ptr
    keep += [head, owners] + scratch
    grp = id(d)
    z = np.zeros(L, np.int64)
    ex.log(ad, True, z, (1,), (1,), whole=True, group=grp)
    ex.log(as_, False, z, (1,), (1,), whole=True, group=grp)
    ex.log(ia_d, False, z, (1,), (1,), whole=True, group=grp)
    ex.launch("rmw", d, keep)
    return []
