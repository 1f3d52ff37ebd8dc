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
    if len(names) == 1 and isinstance(inits[0], Tile):
        return _kloop_matmul(ex, op, lb, st, trips, inits[0])
    return None


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
