"""Lazy tile expressions and their compilation into fused gfx950 programs.

Every tile value of the executor is an :class:`Expr` DAG over one iteration
space (the tile's shape, per lane).  Leaves are strided or offset-list reads
of device memory: argument tensors in the HBM arena (``ktdp.load``) or
materialised temporaries.  Elementwise ops, casts, compares, selects,
broadcasts and transposes only build expressions; a ``ktdp.store`` or any
consumer that needs memory (matmul, a loop-carried value, a host read)
*materialises* the DAG: :func:`compile_program` turns it into one
``ktir_prog_t`` (include/ktir_hip.h) and the kernel evaluates it in a single
pass, reading each leaf straight from HBM.  Row reductions (``linalg.reduce``
over the innermost axis) stay lazy too and compile into row-mode programs
with LDS tree folds, so softmax-style chains become one kernel.

Reference semantics reproduced here: the per-op dtype rounding of NumPy tile
arithmetic (``dialects/_helpers.py:39-54``, ``ops/_helpers.py:50-60``) and the
pairwise-halving fold (``dialects/linalg_ops.py:86-133``).
"""

from __future__ import annotations

import ctypes as C
import struct
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import runtime as rt

FLOAT_DT = ("f16", "bf16", "f32")


def is_float(dt: str) -> bool:
    return dt in FLOAT_DT


class LaneOff:
    """Per-lane element offsets: affine ``base + lane*stride`` or an explicit array."""

    __slots__ = ("base", "stride", "arr")

    def __init__(self, base=0, stride=0, arr: Optional[np.ndarray] = None):
        self.base, self.stride, self.arr = int(base), int(stride), arr

    @staticmethod
    def from_array(a: np.ndarray) -> "LaneOff":
        a = np.asarray(a, dtype=np.int64)
        if a.size == 0:
            return LaneOff(0, 0)
        if a.size == 1:
            return LaneOff(int(a[0]), 0)
        d = np.diff(a)
        if np.all(d == d[0]):
            return LaneOff(int(a[0]), int(d[0]))
        return LaneOff(0, 0, a)

    def values(self, lanes: int) -> np.ndarray:
        if self.arr is not None:
            return self.arr
        return self.base + self.stride * np.arange(lanes, dtype=np.int64)

    def take(self, idx: np.ndarray) -> "LaneOff":
        if self.arr is None and self.stride == 0:
            return self
        if self.arr is None:
            return LaneOff.from_array(self.base + self.stride * idx.astype(np.int64))
        return LaneOff.from_array(self.arr[idx])

    def add(self, delta) -> "LaneOff":
        if np.isscalar(delta) or np.ndim(delta) == 0:
            if self.arr is not None:
                return LaneOff(0, 0, self.arr + int(delta))
            return LaneOff(self.base + int(delta), self.stride)
        return LaneOff.from_array(self.values(len(delta)) + np.asarray(delta, dtype=np.int64))


class LeafSpec:
    """A strided / offset-list view of device memory over an iteration space."""

    __slots__ = ("ptr", "dtype", "lane", "strides", "lo", "hi", "offsets", "offsets_ls", "winner",
                 "winner_base", "alloc", "keep", "__weakref__")

    def __init__(self, ptr, dtype, lane: LaneOff, strides, lo, hi, alloc=None, offsets=None, offsets_ls=0,
                 keep=()):
        self.ptr, self.dtype, self.lane = int(ptr), dtype, lane
        self.strides = tuple(int(s) for s in strides)
        self.lo, self.hi = int(lo), int(hi)
        self.alloc = alloc            # executor allocation record (arena tensors) or None (temporaries)
        self.offsets = offsets        # DeviceBuffer of int64 offsets or None
        self.offsets_ls = int(offsets_ls)
        self.winner = None
        self.winner_base = 0
        self.keep = tuple(keep)

    def with_strides(self, strides, lane=None) -> "LeafSpec":
        n = LeafSpec(self.ptr, self.dtype, self.lane if lane is None else lane, strides, self.lo, self.hi,
                     self.alloc, self.offsets, self.offsets_ls, self.keep)
        return n

    def take(self, idx) -> "LeafSpec":
        if self.offsets is not None:
            raise NotImplementedError("offset-list leaf cannot be re-laned")
        return self.with_strides(self.strides, self.lane.take(idx))


class Expr:
    """Node of a lazy tile expression.

    kind: 'ld' (attr LeafSpec), 'const' (attr python number, already rounded),
    'lane' (attr np.ndarray [lanes] of per-lane scalars), 'idx' (attr dim),
    'un'/'bin'/'cmpf'/'cmpi' (attr opcode or predicate), 'sel', 'fma',
    'cast' (attr source dtype), 'bitcast', 'fold' (attr combiner opcode; row
    level, reduces args[0] over its innermost axis), 'rowval' (element-level
    broadcast of a row-level expression along the innermost axis).
    `shape` is the tile shape; `rowc` is the innermost extent of the row space
    for row-level nodes, else None.
    """

    __slots__ = ("kind", "dtype", "shape", "args", "attr", "rowc", "_fold", "__weakref__")

    def __init__(self, kind, dtype, shape, args=(), attr=None, rowc=None):
        self.kind, self.dtype, self.shape = kind, dtype, tuple(shape)
        self.args = tuple(args)
        self.attr = attr
        self.rowc = rowc
        fr = rowc if kind == "fold" else None
        for a in self.args:
            if a._fold is not None:
                if fr is not None and a._fold != fr:
                    fr = -1
                else:
                    fr = a._fold if fr is None else fr
        self._fold = fr     # inner extent of the folds inside (None: no fold; -1: mixed)

    @property
    def has_fold(self) -> bool:
        return self._fold is not None

    def leaves(self) -> List[LeafSpec]:
        out, seen = [], set()
        for n in walk(self):
            if n.kind == "ld" and id(n.attr) not in seen:
                seen.add(id(n.attr))
                out.append(n.attr)
        return out


def walk(root: Expr):
    seen, stack, order = set(), [root], []
    while stack:
        n = stack.pop()
        if id(n) in seen:
            continue
        seen.add(id(n))
        order.append(n)
        stack.extend(n.args)
    return order


def topo(root: Expr) -> List[Expr]:
    seen, order = set(), []

    def visit(n):
        stack = [(n, False)]
        while stack:
            x, done = stack.pop()
            if done:
                order.append(x)
                continue
            if id(x) in seen:
                continue
            seen.add(id(x))
            stack.append((x, True))
            for a in reversed(x.args):
                if id(a) not in seen:
                    stack.append((a, False))

    visit(root)
    return order


# --------------------------------------------------------------------------
# value encoding helpers
# --------------------------------------------------------------------------

def round_host(v: float, dt: str) -> float:
    if dt == "f16":
        return float(np.float16(v))
    if dt == "bf16":
        b = np.array([v], dtype=np.float32).view(np.uint32)
        b = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        return float(b.view(np.float32)[0])
    if dt == "f32":
        return float(np.float32(v))
    return v


def imm_bits(v, dt: str) -> int:
    if is_float(dt):
        return struct.unpack("<i", struct.pack("<f", float(np.float32(round_host(float(v), dt)))))[0]
    if isinstance(v, (float, np.floating)):
        v = int(v)
    return int(np.int64(int(v)).astype(np.int32))


# --------------------------------------------------------------------------
# compilation
# --------------------------------------------------------------------------

class CompileError(Exception):
    """The DAG does not fit one program (registers, leaves, instructions)."""


class _Builder:
    def __init__(self, lanes: int, space: Tuple[int, ...], mode: int):
        self.lanes = lanes
        self.space = tuple(space)
        self.mode = mode
        self.instr: List[tuple] = []
        self.leaves: List[LeafSpec] = []
        self.leaf_slot: Dict[int, int] = {}
        self.lane_cols: List[np.ndarray] = []
        self.lane_slot: Dict[int, int] = {}
        self.free = list(range(rt.NREG - 1, -1, -1))

    def leaf(self, spec: LeafSpec) -> int:
        k = id(spec)
        if k not in self.leaf_slot:
            if len(self.leaves) >= rt.MAX_LEAVES:
                raise CompileError("too many leaves")
            self.leaf_slot[k] = len(self.leaves)
            self.leaves.append(spec)
        return self.leaf_slot[k]

    def lane_col(self, arr: np.ndarray) -> int:
        k = id(arr)
        if k not in self.lane_slot:
            self.lane_slot[k] = len(self.lane_cols)
            self.lane_cols.append(arr)
        return self.lane_slot[k]

    def alloc(self) -> int:
        if not self.free:
            raise CompileError("out of registers")
        return self.free.pop()

    def release(self, r: int):
        self.free.append(r)

    def emit(self, op, dst=0, a=0, b=0, c=0, dt="f32", aux=0, imm=0):
        if len(self.instr) >= rt.MAX_INSTR:
            raise CompileError("too many instructions")
        self.instr.append((op, dst, a, b, c, rt.DTYPE_CODE.get(dt, 2), aux, imm))
        return len(self.instr) - 1


_OPS = None


def _ops():
    global _OPS
    if _OPS is None:
        _OPS = {n: rt.op(n) for n in ("LD", "ST", "CONST", "LANE", "IDX", "RED", "FOLD", "ELEM", "ENDELEM",
                                      "CAST", "BITCAST", "SELECT", "FMA", "CMPF", "CMPI")}
    return _OPS


def _emit_one(b: _Builder, n: Expr, args: List[int], d: int, leaf_map=None):
    O = _ops()
    k = n.kind
    if k == "ld":
        spec = n.attr if leaf_map is None else leaf_map(n.attr)
        b.emit(O["LD"], d, dt=n.dtype, aux=b.leaf(spec))
    elif k == "const":
        b.emit(O["CONST"], d, dt=n.dtype, imm=imm_bits(n.attr, n.dtype))
    elif k == "lane":
        b.emit(O["LANE"], d, dt=n.dtype, aux=b.lane_col(n.attr))
    elif k == "idx":
        b.emit(O["IDX"], d, dt=n.dtype, aux=int(n.attr))
    elif k in ("un", "bin"):
        b.emit(int(n.attr), d, *(list(args) + [0, 0])[:2], dt=n.dtype)
    elif k == "cmpf":
        b.emit(O["CMPF"], d, args[0], args[1], dt="i1", aux=int(n.attr))
    elif k == "cmpi":
        b.emit(O["CMPI"], d, args[0], args[1], dt="i1", aux=int(n.attr))
    elif k == "sel":
        b.emit(O["SELECT"], d, args[0], args[1], args[2], dt=n.dtype)
    elif k == "fma":
        b.emit(O["FMA"], d, args[0], args[1], args[2], dt=n.dtype)
    elif k == "cast":
        b.emit(O["CAST"], d, args[0], dt=n.dtype, aux=rt.DTYPE_CODE[n.attr])
    elif k == "bitcast":
        b.emit(O["BITCAST"], d, args[0], dt=n.dtype)
    else:
        raise CompileError(f"cannot emit {k}")


def _emit_block(b: _Builder, nodes: List[Expr], regs: Dict[int, int], keep_ids: set, leaf_map=None):
    """Emit `nodes` (topological order).  Registers of nodes not in `keep_ids`
    are released after their last use inside this block; `regs` gains every
    emitted node.  Returns the registers still held by this block."""
    uses: Dict[int, int] = {}
    for n in nodes:
        for a in n.args:
            uses[id(a)] = uses.get(id(a), 0) + 1
    for k in keep_ids:
        uses[k] = uses.get(k, 0) + 1 << 20
    held: Dict[int, int] = {}
    for n in nodes:
        if id(n) in regs:
            continue
        if n.kind == "rowval":
            regs[id(n)] = regs[id(n.args[0])]
            continue
        args = [regs[id(a)] for a in n.args]
        for a in n.args:
            uses[id(a)] -= 1
            if uses[id(a)] == 0 and id(a) in held:
                b.release(held.pop(id(a)))
        d = b.alloc()
        _emit_one(b, n, args, d, leaf_map)
        regs[id(n)] = d
        if uses.get(id(n), 0) > 0:
            held[id(n)] = d
        else:
            b.release(d)
    return held


def compile_program(root: Expr, lanes: int, dest: LeafSpec) -> Tuple[rt.Prog, list]:
    """Compile `root` (stored through `dest`) into a ktir_prog_t.

    Returns (prog, keepalive).  Raises CompileError when the DAG does not fit
    one program; the caller then materialises a sub-expression first.
    """
    if root._fold == -1:
        raise CompileError("folds over different row spaces")
    O = _ops()
    if not root.has_fold:
        space = root.shape if root.shape else (1,)
        nodes = topo(root)
        lds = [n for n in nodes if n.kind == "ld"]
        if 0 < len(lds) <= 4 and len({id(n.attr) for n in lds}) == len(lds):
            try:
                return _compile_flat(root, nodes, lds, lanes, dest, space)
            except CompileError:
                pass
        b = _Builder(lanes, space, 0)
        regs: Dict[int, int] = {}
        _emit_block(b, nodes, regs, {id(root)})
        b.emit(O["ST"], 0, regs[id(root)], dt=root.dtype, aux=b.leaf(dest))
        return _finish(b, lanes, space)

    # ---- row mode: space = row dims + (C,) --------------------------------
    folds = [n for n in topo(root) if n.kind == "fold"]
    R = len(folds[0].args[0].shape)
    space = tuple(folds[0].args[0].shape)
    if any(tuple(f.args[0].shape) != space for f in folds):
        raise CompileError("folds over different row spaces")
    if len(root.shape) not in (R, R - 1):
        raise CompileError("root rank does not match the row space")
    row_root = len(root.shape) == R - 1
    b = _Builder(lanes, space, 1)
    row_specs: Dict[int, LeafSpec] = {}

    def row_leaf(spec: LeafSpec) -> LeafSpec:
        k = id(spec)
        if k not in row_specs:
            # a 1-D row space has one value per lane: a 0-d leaf (kept as
            # one element with strides (1,)) reads or writes that element
            base = () if R == 1 else tuple(spec.strides)
            row_specs[k] = spec.with_strides(base + (0,))
        return row_specs[k]

    def is_row(n: Expr) -> bool:
        return len(n.shape) == R - 1 and n.kind != "rowval"

    # emission units: (rows before fold k, element block of fold k)..., final rows, final block
    units = []
    for f in folds:
        sub = topo_stop(f.args[0])
        units.append(("rows", [n for n in sub if is_row(n) and n.kind != "fold"]))
        units.append(("elem", [n for n in sub if not is_row(n)], f))
    sub = topo_stop(root)
    units.append(("rows", [n for n in sub if is_row(n) and n.kind != "fold"]))
    if not row_root:
        units.append(("elem", [n for n in sub if not is_row(n)], None))
    needed_after = []
    acc: set = set()
    for u in reversed(units):
        needed_after.append(set(acc))
        for n in u[1]:
            for a in n.args:
                acc.add(id(a))
        if u[0] == "elem" and u[2] is not None:
            acc.add(id(u[2].args[0]))
    needed_after.reverse()
    if row_root:
        needed_after = [n | {id(root)} for n in needed_after]

    regs: Dict[int, int] = {}
    row_held: Dict[int, int] = {}
    for ui, u in enumerate(units):
        if u[0] == "rows":
            todo = [n for n in u[1] if id(n) not in regs]
            if todo:
                # row values a later unit reads stay held; the rest (constants,
                # intermediate steps of a scalar chain) free their registers
                # at their last use here
                keep = {id(n) for n in todo if id(n) in needed_after[ui]}
                held = _emit_block(b, todo, regs, keep, row_leaf)
                row_held.update(held)
        else:
            elem, f = u[1], u[2]
            start = b.emit(O["ELEM"])
            target = f.args[0] if f is not None else root
            held = _emit_block(b, elem, regs, {id(target)})
            if f is not None:
                b.emit(O["RED"], 0, regs[id(target)])
            else:
                b.emit(O["ST"], 0, regs[id(root)], dt=root.dtype, aux=b.leaf(dest))
            for r in set(held.values()):
                b.release(r)
            for n in elem:
                if n.kind != "rowval" or True:
                    regs.pop(id(n), None)
            end = b.emit(O["ENDELEM"])
            b.instr[start] = b.instr[start][:6] + (end,) + b.instr[start][7:]
            if f is not None:
                d = b.alloc()
                b.emit(O["FOLD"], d, dt=f.dtype, aux=int(f.attr))
                regs[id(f)] = d
                row_held[id(f)] = d
        # release row values no later unit reads
        for k in [k for k in row_held if k not in needed_after[ui]]:
            b.release(row_held.pop(k))
            regs.pop(k, None)
    if row_root:
        b.emit(O["ST"], 0, regs[id(root)], dt=root.dtype, aux=b.leaf(row_leaf(dest)))
    return _finish(b, lanes, space)


def _compile_flat(root, nodes, lds, lanes, dest, space):
    """Flat program whose leaf loads are prefetched into registers 0..n-1."""
    O = _ops()
    b = _Builder(lanes, space, 0)
    regs: Dict[int, int] = {}
    pf = []
    for n in lds:
        r = b.alloc()
        regs[id(n)] = r
        pf.append(b.leaf(n.attr))
    rest = [n for n in nodes if n.kind != "ld"]
    uses: Dict[int, int] = {}
    for n in nodes:
        for a in n.args:
            uses[id(a)] = uses.get(id(a), 0) + 1
    uses[id(root)] = uses.get(id(root), 0) + 1
    held = {id(n): regs[id(n)] for n in lds if uses.get(id(n), 0) > 0}
    for n in rest:
        args = [regs[id(a)] for a in n.args]
        for a in n.args:
            uses[id(a)] -= 1
            if uses[id(a)] == 0 and id(a) in held:
                b.release(held.pop(id(a)))
        d = b.alloc()
        _emit_one(b, n, args, d)
        regs[id(n)] = d
        if uses.get(id(n), 0) > 0:
            held[id(n)] = d
        else:
            b.release(d)
    b.emit(O["ST"], 0, regs[id(root)], dt=root.dtype, aux=b.leaf(dest))
    prog, keep = _finish(b, lanes, space)
    prog.n_pf = len(pf)
    for i, l in enumerate(pf):
        prog.pf_leaf[i] = l
    return prog, keep


def topo_stop(root: Expr) -> List[Expr]:
    """Topological order of `root`'s DAG without descending into fold inputs."""
    seen, order = set(), []
    stack = [(root, False)]
    while stack:
        x, done = stack.pop()
        if done:
            order.append(x)
            continue
        if id(x) in seen:
            continue
        seen.add(id(x))
        stack.append((x, True))
        if x.kind == "fold" and x is not root:
            continue
        for a in reversed(x.args):
            if id(a) not in seen:
                stack.append((a, False))
    return order


def _finish(b: _Builder, lanes: int, space) -> Tuple[rt.Prog, list]:
    if len(space) > rt.MAX_DIMS:
        raise CompileError("too many dims")
    p = rt.Prog()
    p.mode = b.mode
    p.ndim = len(space)
    p.lanes = lanes
    for i, s in enumerate(space):
        p.shape[i] = int(s)
    keep = []
    for i, L in enumerate(b.leaves):
        _fill_leaf(p.leaves[i], L, lanes, len(space), keep)
    p.n_leaves = len(b.leaves)
    for i, t in enumerate(b.instr):
        ins = p.instr[i]
        ins.op, ins.dst, ins.a, ins.b, ins.c, ins.dt, ins.aux, ins.imm = t
    p.n_instr = len(b.instr)
    if b.lane_cols:
        tab = np.stack([np.asarray(c, dtype=np.float64) for c in b.lane_cols], axis=1)
        buf = rt.DeviceBuffer(tab.nbytes)
        buf.upload(tab)
        keep.append(buf)
        p.lane_scalars = buf.ptr
        p.n_lane_scalars = tab.shape[1]
    return p, keep


def _fill_leaf(dst: rt.Leaf, L: LeafSpec, lanes: int, ndim: int, keep: list):
    dst.ptr = L.ptr
    st = list(L.strides)
    if len(st) != ndim:
        raise CompileError("leaf rank exceeds program rank")
    for i in range(ndim):
        dst.strides[i] = st[i]
    if L.lane.arr is not None:
        arr = np.ascontiguousarray(L.lane.arr, dtype=np.int64)
        if arr.size < lanes:
            raise CompileError("lane offsets shorter than lane count")
        buf = rt.DeviceBuffer(arr.nbytes)
        buf.upload(arr)
        keep.append(buf)
        dst.lane_base = buf.ptr
        dst.base, dst.lane_stride = 0, 0
        starts = arr
    else:
        dst.lane_base = 0
        dst.base, dst.lane_stride = L.lane.base, L.lane.stride
        starts = None
    if L.offsets is not None:
        dst.offsets = L.offsets.ptr
        dst.offsets_lane_stride = L.offsets_ls
        keep.append(L.offsets)
    dst.lo, dst.hi = L.lo, L.hi
    dst.dtype = rt.DTYPE_CODE[L.dtype]
    if L.winner is not None:
        dst.winner = L.winner.ptr
        dst.winner_base = L.winner_base
        keep.append(L.winner)
    # wide accesses: inner stride 1 and every 4- (8-) element vector start aligned
    flags = 0
    bpe = rt.ELEM_BYTES[L.dtype]
    for w, bit in ((4, rt.K["KTIR_LEAF_VEC"]), (8, rt.K["KTIR_LEAF_VEC8"])):
        ok = L.offsets is None and st[-1] == 1 and all(s % w == 0 for s in st[:-1]) and L.ptr % (w * bpe) == 0
        if ok:
            if starts is not None:
                ok = bool(np.all(starts % w == 0))
            else:
                ok = L.lane.base % w == 0 and L.lane.stride % w == 0
        if ok:
            flags |= bit
    dst.flags = flags
    keep.extend(L.keep)
