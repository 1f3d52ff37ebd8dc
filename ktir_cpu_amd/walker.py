"""Op handlers of the lockstep executor (one method per KTIR op).

Each handler mirrors the reference handler named in its docstring; scalar
(index / loop-bound / address) values are NumPy vectors with one entry per
lane, tile values are lazy :class:`program.Expr` DAGs evaluated on the GPU.
"""

from __future__ import annotations

import ctypes as C
import math
import operator
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

from . import runtime as rt
from .affine import AffineMap, AffineSet, Box, evaluate
from .executor import (Access, Alloc, Arena, ATile, DevScalar, DistATile, DistView, IATile, Instances, Lanes, NeedEager,
                       Plan, Pool, Tile, View, _launch, verify)
from .ir import IRFunction, Operation, Region
from .program import CompileError, Expr, LaneOff, LeafSpec, compile_program, is_float, round_host, topo

# ---------------------------------------------------------------------------
# op tables (semantics as the reference's: dialects/arith_ops.py:49-135,
# ops/math_ops.py:27-111, dialects/math_ops.py:28-59)
# ---------------------------------------------------------------------------

FLOAT_BIN = {"arith.addf": "ADDF", "arith.subf": "SUBF", "arith.mulf": "MULF", "arith.divf": "DIVF",
             "arith.remf": "REMF"}
MINMAX_F = {"arith.maxf": "MAXIMUMF", "arith.maximumf": "MAXIMUMF", "arith.maxnumf": "MAXNUMF",
            "arith.minf": "MINIMUMF", "arith.minimumf": "MINIMUMF", "arith.minnumf": "MINNUMF"}
INT_BIN = {"arith.addi": "ADDI", "arith.subi": "SUBI", "arith.muli": "MULI", "arith.divui": "FLOORDIVSI",
           "arith.divsi": "DIVSI", "arith.floordivsi": "FLOORDIVSI", "arith.remui": "FLOORREMSI",
           "arith.remsi": "REMSI", "arith.andi": "ANDI", "arith.ori": "ORI", "arith.xori": "XORI",
           "arith.shli": "SHLI", "arith.shrsi": "SHRSI", "arith.shrui": "SHRUI", "arith.minsi": "MINSI",
           "arith.maxsi": "MAXSI", "arith.minui": "MINSI", "arith.maxui": "MAXSI",
           "arith.ceildivsi": "CEILDIVSI", "arith.ceildivui": "CEILDIVSI"}
MATH_UN = {"math.exp": "EXP", "math.sqrt": "SQRT", "math.rsqrt": "RSQRT", "math.log": "LOG",
           "math.log2": "LOG2", "math.log1p": "LOG1P", "math.tanh": "TANH", "math.sin": "SIN",
           "math.cos": "COS", "math.erf": "ERF", "math.ceil": "CEIL", "math.floor": "FLOOR"}
COMBINERS = {"arith.addf": "ADDF", "arith.mulf": "MULF", "arith.maxf": "MAXIMUMF", "arith.maximumf": "MAXIMUMF",
             "arith.minf": "MINIMUMF", "arith.minimumf": "MINIMUMF", "arith.maxnumf": "MAXNUMF",
             "arith.minnumf": "MINNUMF", "arith.addi": "ADDI", "arith.muli": "MULI", "arith.maxsi": "MAXSI",
             "arith.minsi": "MINSI"}
COMBINER_IDENTITY = {"arith.addf": 0.0, "arith.addi": 0, "arith.mulf": 1.0, "arith.muli": 1,
                     "arith.maxf": float("-inf"), "arith.maximumf": float("-inf"),
                     "arith.minf": float("inf"), "arith.minimumf": float("inf")}
CMPF = {"false": "FALSE", "oeq": "OEQ", "ogt": "OGT", "oge": "OGE", "olt": "OLT", "ole": "OLE", "one": "ONE",
        "ord": "ORD", "ueq": "UEQ", "ugt": "UGT", "uge": "UGE", "ult": "ULT", "ule": "ULE", "une": "UNE",
        "uno": "UNO", "true": "TRUE"}
CMPI = {"eq": "EQ", "ne": "NE", "slt": "SLT", "sle": "SLE", "sgt": "SGT", "sge": "SGE", "ult": "ULTI",
        "ule": "ULEI", "ugt": "UGTI", "uge": "UGEI"}
NO_LX_CHARGE = {"arith.constant"}


def _np_floordiv(a, b):
    return np.floor_divide(a, np.where(b == 0, 1, b))


def _truncdiv(a, b):
    return np.trunc(np.asarray(a) / np.asarray(b)).astype(np.asarray(a).dtype)


SCALAR_INT = {"arith.addi": operator.add, "arith.subi": operator.sub, "arith.muli": operator.mul,
              "arith.divui": operator.floordiv, "arith.divsi": _truncdiv, "arith.floordivsi": operator.floordiv,
              "arith.remui": operator.mod, "arith.remsi": lambda a, b: a - _truncdiv(a, b) * b,
              "arith.andi": operator.and_, "arith.ori": operator.or_, "arith.xori": operator.xor,
              "arith.shli": operator.lshift, "arith.shrsi": operator.rshift,
              "arith.minsi": np.minimum, "arith.maxsi": np.maximum, "arith.minui": np.minimum,
              "arith.maxui": np.maximum,
              "arith.ceildivsi": lambda a, b: np.ceil(a / b).astype(np.int64),
              "arith.ceildivui": lambda a, b: np.ceil(a / b).astype(np.int64)}
SCALAR_FLOAT = {"arith.addf": operator.add, "arith.subf": operator.sub, "arith.mulf": operator.mul,
                "arith.divf": operator.truediv, "arith.remf": operator.mod}
SCALAR_MINMAX = {"arith.maxf": np.maximum, "arith.maximumf": np.maximum, "arith.maxnumf": np.fmax,
                 "arith.minf": np.minimum, "arith.minimumf": np.minimum, "arith.minnumf": np.fmin}


def _erf_np(x):
    a = np.abs(x)
    t = 1.0 / (1.0 + 0.3275911 * a)
    poly = t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027 + t * 1.061405429))))
    return np.sign(x) * (1.0 - poly * np.exp(-a * a))


SCALAR_MATH = {"math.exp": np.exp, "math.sqrt": np.sqrt, "math.rsqrt": lambda x: 1.0 / np.sqrt(x),
               "math.log": np.log, "math.log2": np.log2, "math.log1p": np.log1p, "math.tanh": np.tanh,
               "math.sin": np.sin, "math.cos": np.cos, "math.erf": _erf_np, "math.ceil": np.ceil,
               "math.floor": np.floor}

NP_DTYPE = {"f16": np.float16, "f32": np.float32, "bf16": np.float32, "i1": np.bool_, "i32": np.int32,
            "index": np.int32, "i64": np.int64}


def _canon(dt: str) -> str:
    return {"index": "i32", "si32": "i32", "si64": "i64", "ui32": "i32", "fp16": "f16"}.get(dt, dt)


def _elem_of(t) -> Optional[str]:
    if t is None:
        return None
    return _canon(getattr(t, "elem", None) or getattr(t, "name", None) or "")


def _is_scalar(v) -> bool:
    return isinstance(v, np.ndarray)


def _narrow_scalar(v, target, op_name) -> np.ndarray:
    """A scalar float cast (reference ops/arith_ops.py:38-87): a value that
    is already of the target type is kept; a finite value that becomes
    infinite raises OverflowError."""
    a = np.asarray(v)
    if a.dtype == target:
        return a
    with np.errstate(over="ignore"):
        r = a.astype(target)
    bad = np.isinf(r) & np.isfinite(a.astype(np.float64))
    if np.any(bad):
        raise OverflowError(f"{op_name}: {a[bad].flat[0]} overflows {np.dtype(target).name}")
    return r


def _scalar_kind(v) -> Optional[str]:
    """The NumPy float type of a scalar operand ("f16" / "f32"), or None for
    one that acts as a Python number (a constant, a float64 value, a
    reduction's Python float) and takes the other operand's type."""
    if isinstance(v, DevScalar):
        return None if v.weak else v.dtype
    dt = np.asarray(v).dtype
    return {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32"}.get(dt)


class _Yield:
    __slots__ = ("values",)

    def __init__(self, values):
        self.values = values


def _unwrap(res):
    if not isinstance(res, _Yield):
        return res
    if not res.values:
        return None
    return res.values[0] if len(res.values) == 1 else tuple(res.values)


def _uniform(a: np.ndarray, what: str):
    if a.size and np.any(a != a.flat[0]):
        raise NeedEager(f"{what} differs between lanes")
    return a.flat[0] if a.size else 0


# ---------------------------------------------------------------------------
# expression builders
# ---------------------------------------------------------------------------

def E_const(v, dt, shape) -> Expr:
    return Expr("const", dt, shape, attr=v)


def E_scalar(v: np.ndarray, dt: str, shape) -> Expr:
    """A per-lane scalar broadcast over a tile shape."""
    if v.size and np.all(v == v.flat[0]):
        x = v.flat[0]
        return E_const(x.item() if hasattr(x, "item") else x, dt, shape)
    return Expr("lane", dt, shape, attr=np.asarray(v, dtype=np.float64))


def _strides_injective(shape, strides) -> bool:
    """Whether distinct positions of a box of `shape` over `strides` always
    reach distinct elements (sufficient test: every stride, smallest first,
    exceeds the span of the smaller ones).  A store through a box that fails
    it can write one element twice, and then the later position in
    row-major order must win, as in the reference's fancy-index write."""
    span = 0
    for s, n in sorted((abs(int(s)), int(n)) for s, n in zip(strides, shape) if int(n) > 1):
        if s <= span:
            return False
        span += s * (n - 1)
    return True


def _collapse_dims(e: Expr, dest: LeafSpec, max_dims: int):
    """Rewrite a fold-free expression stored through `dest` over fewer
    dimensions: dims of extent 1 are dropped (their index is 0), then
    adjacent dims d, d + 1 merge where every leaf (and `dest`) has
    stride[d] == stride[d + 1] * extent[d + 1] and no linalg.index reads
    either.  Gather leaves (offset lists) are laid out over the flattened
    positions, so they keep contiguous strides.  Returns (e, dest) of rank
    <= max_dims, or None."""
    shape = tuple(e.shape)
    nodes = topo(e)
    if any(n.kind in ("fold", "rowval") for n in nodes):
        return None
    specs = [n.attr for n in nodes if n.kind == "ld"] + [dest]
    if any(len(sp.strides) != len(shape) for sp in specs):
        return None
    if any(sp.offsets is not None and tuple(sp.strides) != _cstrides(shape) for sp in specs):
        return None
    idx_dims = {int(n.attr) for n in nodes if n.kind == "idx"}
    # groups of old dims that become one new dim
    groups = [[d] for d in range(len(shape)) if shape[d] != 1]
    if not groups:
        groups = [[len(shape) - 1]]
    k = 0
    while len(groups) > max_dims and k < len(groups) - 1:
        a, b = groups[k], groups[k + 1]
        ok = not (set(a) | set(b)) & idx_dims
        for sp in specs:
            if ok and int(sp.strides[a[-1]]) != int(sp.strides[b[-1]]) * _prod([shape[d] for d in b]):
                ok = False
        if ok:
            groups[k:k + 2] = [a + b]
        else:
            k += 1
    if len(groups) > max_dims:
        return None
    nshape = tuple(_prod([shape[d] for d in g]) for g in groups)
    pos = {g[0]: i for i, g in enumerate(groups)}

    def lf(spec):
        if spec.offsets is not None:
            return spec.with_strides(_cstrides(nshape))
        return spec.with_strides(tuple(int(spec.strides[g[-1]]) for g in groups))

    def idxf(d):
        if d in pos:
            return Expr("idx", "i32", nshape, attr=pos[d])
        return E_const(0, "i32", nshape)

    memo = {}

    def rebuild(x):
        k2 = id(x)
        if k2 in memo:
            return memo[k2]
        if x.kind == "ld":
            r = Expr("ld", x.dtype, nshape, attr=lf(x.attr))
        elif x.kind == "idx":
            r = idxf(int(x.attr))
        elif x.kind in ("const", "lane"):
            r = Expr(x.kind, x.dtype, nshape, attr=x.attr)
        else:
            r = Expr(x.kind, x.dtype, nshape, [rebuild(a) for a in x.args], x.attr)
        memo[k2] = r
        return r

    return rebuild(e), lf(dest)


def _map_leaf_idx(e: Expr, shape, leaf_fn, idx_fn, memo=None) -> Expr:
    """Rebuild `e` over a new iteration space.  leaf_fn(spec) -> spec maps
    strided leaves; idx_fn(dim) -> Expr builds the new index of an old dim."""
    if memo is None:
        memo = {}
    k = id(e)
    if k in memo:
        return memo[k]
    if e.kind == "fold" or e.kind == "rowval":
        raise CompileError("view transform over a row reduction")
    if e.kind == "ld":
        spec = e.attr
        if spec.offsets is not None:
            raise CompileError("view transform over a gather")
        r = Expr("ld", e.dtype, shape, attr=leaf_fn(spec))
    elif e.kind == "idx":
        r = idx_fn(int(e.attr))
    elif e.kind in ("const", "lane"):
        r = Expr(e.kind, e.dtype, shape, attr=e.attr)
    else:
        r = Expr(e.kind, e.dtype, shape, [_map_leaf_idx(a, shape, leaf_fn, idx_fn, memo) for a in e.args], e.attr)
    memo[k] = r
    return r


def remap_lanes(e: Expr, idx: np.ndarray, memo=None) -> Expr:
    if memo is None:
        memo = {}
    k = id(e)
    if k in memo:
        return memo[k]
    if e.kind == "ld":
        spec = e.attr
        if spec.offsets is not None:
            if spec.offsets_ls == 0 and spec.lane.arr is None and spec.lane.stride == 0:
                r = e
            else:
                raise CompileError("gather leaf cannot change lanes")
        else:
            r = Expr("ld", e.dtype, e.shape, attr=spec.take(idx))
    elif e.kind == "lane":
        r = Expr("lane", e.dtype, e.shape, attr=e.attr[idx])
    elif e.kind in ("const", "idx"):
        r = e
    else:
        r = Expr(e.kind, e.dtype, e.shape, [remap_lanes(a, idx, memo) for a in e.args], e.attr, e.rowc)
    memo[k] = r
    return r


def _mm_quads(la, lb, L: int, M: int, N: int) -> Optional[np.ndarray]:
    """Group the lanes of a 128 x 128 matmul 2 x 2 into 256 x 256 blocks:
    {top-left, top-right, bottom-left, bottom-right} with the right lane's B
    N columns after the left's (same A) and the bottom lane's A M rows below
    the top's (same B).  None unless every lane falls in exactly one group."""
    if L < 4 or L % 4 or la.strides[-1] != 1 or lb.strides[-1] != 1:
        return None
    ao, bo = la.lane.values(L).astype(np.int64), lb.lane.values(L).astype(np.int64)
    dn, dm = N * 1, M * int(la.strides[-2])
    where = {}
    for i in range(L):
        where.setdefault((int(ao[i]), int(bo[i])), []).append(i)
    used = np.zeros(L, bool)
    out = []
    for i in np.lexsort((bo, ao)):
        if used[i]:
            continue
        a, b = int(ao[i]), int(bo[i])
        grp = [i]
        for key in ((a, b + dn), (a + dm, b), (a + dm, b + dn)):
            cand = [j for j in where.get(key, []) if not used[j] and j not in grp]
            if not cand:
                return None
            grp.append(cand[0])
        for j in grp:
            used[j] = True
        out.extend(grp)
    return _xcd_blocks(np.asarray(out, dtype=np.int32).reshape(-1, 4), ao, bo).ravel()


# workgroups one XCD runs at once (MI355X: 256 CUs in 8 XCDs, one 256 x 256
# matmul workgroup per CU)
_XCD_SLOTS, _N_XCD = 32, 8


def _xcd_blocks(q: np.ndarray, ao: np.ndarray, bo: np.ndarray) -> np.ndarray:
    """Order the 2 x 2 groups `q` (rows {tl, tr, bl, br}) so that the 32
    workgroups an XCD runs together cover a 4 x 8 block of the result grid:
    the kernel gives XCD x the x-th eighth of the list, so each XCD streams
    4 rows of A blocks and 8 columns of B blocks per round instead of 1 x 32.
    Unchanged unless the groups form a full grid that such blocks tile."""
    n = len(q)
    if n % (_XCD_SLOTS * _N_XCD):
        return q
    ra = np.unique(ao[q[:, 0]], return_inverse=True)[1]
    cb = np.unique(bo[q[:, 0]], return_inverse=True)[1]
    nm, nn = int(ra.max()) + 1, int(cb.max()) + 1
    if nm * nn != n or nm % 4 or nn % 8:
        return q
    grid = np.full((nm, nn), -1, np.int64)
    grid[ra, cb] = np.arange(n)
    if np.any(grid < 0):
        return q
    order = grid.reshape(nm // 4, 4, nn // 8, 8).transpose(0, 2, 1, 3).ravel()
    return q[order]


class _Future:
    """ktdp.inter_tile_produce result (reference ir_types.py:481-530): every
    lane's yielded partial(s), its group index and the sets."""

    __slots__ = ("partials", "gid", "producer_set", "groups_set")

    def __init__(self, partials, gid, producer_set, groups_set):
        self.partials, self.gid = partials, gid
        self.producer_set, self.groups_set = producer_set, groups_set

    def take(self, idx):
        return _Future(None if self.partials is None else tuple(take_value(p, idx) for p in self.partials),
                       self.gid[idx], self.producer_set, self.groups_set)


def take_value(v, idx: np.ndarray):
    if isinstance(v, np.ndarray):
        return v[idx]
    if isinstance(v, Tile):
        return Tile(remap_lanes(v.e, idx))
    if isinstance(v, DevScalar):
        return DevScalar(Tile(remap_lanes(v.t.e, idx)), v.weak)
    if isinstance(v, (View, ATile, IATile, DistView, DistATile, _Future)):
        return v.take(idx)
    if isinstance(v, tuple):
        return tuple(take_value(x, idx) for x in v)
    return v


# ---------------------------------------------------------------------------
# the executor
# ---------------------------------------------------------------------------

class _Frame:
    __slots__ = ("vals", "level")

    def __init__(self, level):
        self.vals: Dict[str, Any] = {}
        self.level = level


class _Level:
    __slots__ = ("lanes", "parent_idx", "cache")

    def __init__(self, lanes: Lanes, parent_idx: Optional[np.ndarray]):
        self.lanes = lanes
        self.parent_idx = parent_idx
        self.cache: Dict[int, np.ndarray] = {}


class Executor:
    def __init__(self, fn: IRFunction, arena: Arena, args: Dict[str, Any], pool: Pool, *, sequential: bool,
                 lx_size_mb: int = 2, allow_expand: bool = True, latency=None, lx=None):
        self.fn = fn
        # every core's LX scratchpad on the device (executor.LXSpace), or None
        # when the function addresses no LX memory
        self.lx = lx
        # cores meet at ktdp.inter_tile_reduce: every core must run in lockstep
        self.collective = _has_op(fn.operations, "ktdp.inter_tile_reduce")
        self.had_reduce = False
        # latency model: lanes charged by the op being recorded (None: all),
        # and the ring bytes a reduce moved per core
        self._lat_mask: Optional[np.ndarray] = None
        self._lat_comm = 0
        # latency model (ktir_cpu_amd.latency.LatencyTracker) charged op by op, or None
        self.lat = latency
        self._lat_mem: Optional[np.ndarray] = None
        self.arena = arena
        self.args = args
        self.pool = pool
        self.sequential = sequential
        self.eager = sequential
        self.attn_pending = None     # last fused attention launch whose epilogue may still fold in
        self.mm_pending = None       # last matmul launch whose result store may still fold in
        self.allow_expand = allow_expand and not sequential
        self.plan = Plan(pool)
        self.plan.mode = "sequential" if sequential else "lockstep"
        nx, ny, nz = fn.grid
        self.grid = (nx, ny, nz)
        self.n_cores = nx * ny * nz
        self.insts = Instances(self.n_cores)
        self.accesses: List[Access] = []
        self.stored: set = set()     # id() of every allocation a launch stores into
        self.lx_capacity = lx_size_mb * 1024 * 1024
        self.use_counts = _use_counts(fn.operations)
        self._linalg_shape: List[Tuple[int, ...]] = []

    # -- driver -------------------------------------------------------------
    def run(self):
        plan = self._run_grid()
        # a device copy of an input stays valid across replays only if no
        # launch of the plan stores into the input
        for c in plan.v16.values():
            c.ok = id(c.alloc) not in self.stored
        return plan

    def _run_grid(self):
        if self.sequential:
            for c in range(self.n_cores):
                lanes = Lanes(np.array([c], dtype=np.int64), np.array([c], dtype=np.int64))
                self._run_body(lanes)
        else:
            if self.lat is not None:
                # the latency model reads device data op by op: launch as walked
                self._go_eager()
            lanes = Lanes(np.arange(self.n_cores, dtype=np.int64), np.arange(self.n_cores, dtype=np.int64))
            self._run_body(lanes)
            why = verify(self.accesses, self.insts)
            if why is not None:
                if self.had_reduce:
                    raise NotImplementedError(f"cross-core dependence through memory after "
                                              f"ktdp.inter_tile_reduce: {why}")
                raise NeedEager(why)
        return self.plan

    def _run_body(self, lanes: Lanes):
        self.levels = [_Level(lanes, None)]
        self.frames = [_Frame(0)]
        self.lx_used = 0
        self.refcount: Dict[int, int] = {}
        self.uncharged: set = set()
        for name, v in self.args.items():
            if isinstance(v, np.ndarray) and v.ndim == 0:
                v = np.full(lanes.n, v.item())
            elif not isinstance(v, np.ndarray):
                v = np.full(lanes.n, v)
            self.set_value("%" + name, v)
        self._run(self.fn.operations)

    @property
    def lanes(self) -> Lanes:
        return self.levels[-1].lanes

    @property
    def L(self) -> int:
        return self.levels[-1].lanes.n

    # -- launches -------------------------------------------------------------
    def launch(self, kind, desc, keep=()):
        self.plan.add(kind, desc, keep)
        if self.eager:
            _launch(rt.lib(), kind, desc)

    # -- scopes and values (reference grid.py:210-350) -------------------------
    def push_scope(self):
        self.frames.append(_Frame(len(self.levels) - 1))
        self._scope_lx = getattr(self, "_scope_lx", [])
        self._scope_lx.append(self.lx_used)

    def pop_scope(self):
        fr = self.frames.pop()
        for v in fr.vals.values():
            if isinstance(v, Tile):
                self._release(v)
        self._scope_lx.pop()

    def _idx_to(self, level: int) -> np.ndarray:
        cur = self.levels[-1]
        if level in cur.cache:
            return cur.cache[level]
        idx = np.arange(cur.lanes.n, dtype=np.int64)
        for lv in range(len(self.levels) - 1, level, -1):
            idx = self.levels[lv].parent_idx[idx]
        cur.cache[level] = idx
        return idx

    def set_value(self, name, value, charge=True):
        fr = self.frames[-1]
        old = fr.vals.get(name)
        if isinstance(old, Tile):
            self._release(old)
        fr.vals[name] = value
        if isinstance(value, Tile):
            vid = id(value)
            if (not charge) or vid in self.uncharged:
                self.uncharged.add(vid)
                self.refcount[vid] = self.refcount.get(vid, 0) + 1
                return
            if self.refcount.get(vid, 0) == 0:
                sz = value.nbytes()
                if self.lx_used + sz > self.lx_capacity:
                    core = int(self.lanes.cores[0]) if self.L else 0
                    raise MemoryError(
                        f"LX scratchpad overflow on core {core}: requested {sz} bytes, available "
                        f"{self.lx_capacity - self.lx_used} bytes (capacity {self.lx_capacity} bytes)")
                self.lx_used += sz
            self.refcount[vid] = self.refcount.get(vid, 0) + 1

    def _release(self, t: Tile):
        vid = id(t)
        if vid not in self.refcount:
            return
        unch = vid in self.uncharged
        self.refcount[vid] -= 1
        if self.refcount[vid] == 0:
            del self.refcount[vid]
            self.uncharged.discard(vid)
            if not unch:
                self.lx_used -= t.nbytes()

    def get_value(self, name, peek=False, dev=False):
        """The value of SSA name `name` on the current lanes.  A scalar that
        lives on the device (DevScalar) is returned as it is only to callers
        that keep it there (`dev`); any other caller gets its per-lane host
        values."""
        for fr in reversed(self.frames):
            if name in fr.vals:
                v = fr.vals[name]
                if (not peek and isinstance(v, Tile) and self.use_counts.get(name, 0) == 1
                        and fr is self.frames[-1]):
                    del fr.vals[name]
                    self._release(v)
                if fr.level != len(self.levels) - 1:
                    v = take_value(v, self._idx_to(fr.level))
                if isinstance(v, DevScalar) and not dev:
                    v = self.host_scalar(v)
                return v
        raise KeyError(f"Value '{name}' not found")

    def host_scalar(self, v: DevScalar) -> np.ndarray:
        """Per-lane host values of a device scalar, as the NumPy scalar type
        the reference holds.  Reading device data needs the work recorded so
        far to have run: a lockstep walk starts again core by core (or, where
        cores meet at a ring reduce, launches from here on as it walks)."""
        if not self.eager:
            if not self.collective:
                raise NeedEager("a scalar read from tile data is used on the host")
            self._go_eager()
        data = self.read_tile(v.t).reshape(self.L)
        if v.weak:
            return data.astype(np.float64)
        return data.astype(np.float16 if v.dtype == "f16" else np.float32)

    def has_value(self, name) -> bool:
        return any(name in fr.vals for fr in self.frames)

    # -- execution ------------------------------------------------------------
    def _run(self, ops):
        res = None
        for op in ops:
            res = self._exec(op)
        return res

    def _exec(self, op: Operation):
        h = getattr(self, "h_" + op.op_type.replace(".", "_"), None)
        t = op.op_type
        lat_ops = None
        if self.lat is not None:
            # operands as they were before the op (reference interpreter.py:209-217)
            lat_ops = [self.get_value(n, peek=True, dev=True) if self.has_value(n) else None for n in op.operands]
            self._lat_mem = None
        if h is not None:
            res = h(op)
        elif t in FLOAT_BIN:
            res = self.float_binop(op, FLOAT_BIN[t])
        elif t in MINMAX_F:
            res = self.minmax(op)
        elif t in INT_BIN:
            res = self.int_binop(op)
        elif t in MATH_UN:
            res = self.math_unary(op)
        else:
            raise ValueError(f"Unknown operation: {t}")
        if op.results and res is not None:
            vals = res if isinstance(res, tuple) else (res,)
            if len(vals) != len(op.results):
                raise RuntimeError(f"{t}: expected {len(op.results)} result(s), got {len(vals)}")
            charge = t not in NO_LX_CHARGE
            for n, v in zip(op.results, vals):
                self.set_value(n, v, charge=charge)
        if self.lat is not None:
            self._lat_record(t, res, lat_ops)
        return res

    # -- latency model (reference latency.py:289-432) -------------------------
    def _lat_record(self, t: str, res, operands):
        """Charge op `t` to every active core: HBM bytes of a load / store at
        stick granularity, M/N/K of a matmul, else the element count of the
        result (or of the first tile operand)."""
        from . import latency
        cat = latency.category_of(t)
        cores = self.lanes.cores
        sel = np.arange(len(cores)) if self._lat_mask is None else np.flatnonzero(self._lat_mask)
        cores = cores[sel]
        if cat == latency.LC.MEMORY:
            sticks = self._lat_mem[sel] if self._lat_mem is not None else np.zeros(len(cores), np.int64)
            for c, k in zip(cores, sticks):
                self.lat.record_op(int(c), t, nbytes=int(k) * latency.STICK_BYTES)
            return
        if cat == latency.LC.COMM:
            for c in cores:
                self.lat.record_op(int(c), t, nbytes=int(self._lat_comm))
            return
        if cat == latency.LC.COMPUTE_MATMUL:
            tiles = [v for v in (operands or []) if isinstance(v, Tile)]
            mnk = (1, 1, 1)
            if len(tiles) >= 2:
                a, b = tiles[0].shape, tiles[1].shape
                mnk = (a[0] if len(a) >= 2 else 1, b[1] if len(b) >= 2 else 1, a[1] if len(a) >= 2 else a[0])
            for c in cores:
                self.lat.record_op(int(c), t, mnk=mnk)
            return
        n = 1
        if isinstance(res, Tile):
            n = _prod(res.shape)
        else:
            for v in operands or []:
                if isinstance(v, Tile):
                    n = _prod(v.shape)
                    break
        for c in cores:
            self.lat.record_op(int(c), t, n_elems=n)

    def _lat_box(self, rel: np.ndarray, shape, strides, bpe: int):
        """Per-lane unique sticks of a strided box access (element offsets
        relative to a stick-aligned allocation)."""
        if self.lat is None:
            return
        from .latency import unique_sticks_rows, unique_sticks_elems
        shape = tuple(int(x) for x in shape) or (1,)
        strides = tuple(int(x) for x in strides) or (1,)
        rel = np.asarray(rel, dtype=np.int64).reshape(-1)
        outer = np.zeros(1, np.int64)
        for ext, st in zip(shape[:-1], strides[:-1]):
            outer = (outer[:, None] + np.arange(ext, dtype=np.int64)[None, :] * st).reshape(-1)
        if strides[-1] == 1:
            self._lat_mem = np.array([unique_sticks_rows((r + outer) * bpe, shape[-1] * bpe) for r in rel], np.int64)
        else:
            full = (outer[:, None] + np.arange(shape[-1], dtype=np.int64)[None, :] * strides[-1]).reshape(-1)
            self._lat_mem = np.array([unique_sticks_elems((r + full) * bpe) for r in rel], np.int64)

    def _lat_elems(self, rel: np.ndarray, offs: np.ndarray, bpe: int, extra: Optional[np.ndarray] = None):
        """Per-lane unique sticks of single-element accesses at `offs` (plus `extra` sticks)."""
        if self.lat is None:
            return
        from .latency import unique_sticks_elems
        rel = np.asarray(rel, dtype=np.int64).reshape(-1)
        offs = np.asarray(offs, dtype=np.int64)
        if offs.ndim == 1:
            offs = np.broadcast_to(offs, (len(rel), offs.size))
        k = np.array([unique_sticks_elems((r + o) * bpe) for r, o in zip(rel, offs)], np.int64)
        self._lat_mem = k if extra is None else k + extra

    # -- memory helpers -------------------------------------------------------
    def _alloc_of(self, byte_addr: np.ndarray) -> Alloc:
        a0 = self.arena.find(int(byte_addr.flat[0]))
        if byte_addr.size > 1:
            lo, hi = a0.addr, a0.addr + a0.nbytes
            if np.any((byte_addr < lo) | (byte_addr >= max(hi, lo + 1))):
                for x in np.unique(byte_addr):
                    if self.arena.find(int(x)) is not a0:
                        raise NotImplementedError("access tile spans several argument tensors across lanes")
        return a0

    def _hbm_leaf(self, view: View, origin: np.ndarray, shape, strides,
                  offs: Optional[np.ndarray] = None) -> Tuple[LeafSpec, Alloc, np.ndarray]:
        bpe = rt.ELEM_BYTES[view.dtype]
        if view.space != "HBM":
            return self._lx_leaf(view, origin, shape, strides, offs)
        elem = view.base.astype(np.int64) + origin.astype(np.int64)
        a = self._alloc_of(elem * bpe)
        if rt.ELEM_BYTES[a.dtype] != bpe:
            raise NotImplementedError(f"view dtype {view.dtype} over a {a.dtype} tensor")
        rel = elem - a.addr // bpe
        spec = LeafSpec(self.arena.ptr_of(a), view.dtype, LaneOff.from_array(rel), strides, 0, a.n_elems, alloc=a)
        return spec, a, rel

    def _lx_leaf(self, view: View, origin: np.ndarray, shape, strides, offs: Optional[np.ndarray] = None,
                 span: Optional[Tuple[np.ndarray, np.ndarray]] = None):
        """A leaf over the addressed core's LX: element `core * (bytes per
        core / bpe) + pointer + origin` of the LX space.  Refuses an access
        that leaves the core's scratchpad (`offs`: the element offsets of an
        offset-list access shared by all lanes; `span`: per-lane [lo, hi)
        element offsets, lanes with an empty span access nothing)."""
        lx = self.lx
        bpe = rt.ELEM_BYTES[view.dtype]
        if lx is None or view.core is None:
            raise NotImplementedError("LX memory view without an LX space")
        if lx.bytes_per_core % bpe:
            raise NotImplementedError("LX size is not a multiple of the element size")
        start = view.base.astype(np.int64) + origin.astype(np.int64)
        if span is not None:
            live = span[1] > span[0]
            lo_e, hi_e = (start + span[0])[live], (start + span[1])[live]
        elif offs is not None and len(offs):
            lo_e, hi_e = start + int(np.min(offs)), start + int(np.max(offs)) + 1
        else:
            ext = sum((int(n) - 1) * abs(int(st)) for n, st in zip(shape, strides) if int(n) > 0)
            neg = sum((int(n) - 1) * int(st) for n, st in zip(shape, strides) if int(st) < 0 and int(n) > 0)
            lo_e, hi_e = start + neg, start + neg + ext + 1
        if np.any(lo_e < 0) or np.any(hi_e * bpe > lx.bytes_per_core):
            raise NotImplementedError(f"LX access outside the {lx.bytes_per_core}-byte scratchpad")
        core = np.broadcast_to(np.asarray(view.core, dtype=np.int64), start.shape)
        rel = core * (lx.bytes_per_core // bpe) + start
        spec = LeafSpec(lx.buf.ptr, view.dtype, LaneOff.from_array(rel), strides, 0, lx.alloc.nbytes // bpe,
                        alloc=lx.alloc)
        return spec, lx.alloc, rel

    def _log_mem(self, alloc, store, rel, shape, strides, dtype, mask=None):
        """Log an access in the allocation's units: elements for a tensor,
        bytes for the LX space (whose views may differ in dtype)."""
        if self.lx is not None and alloc is self.lx.alloc:
            bpe = rt.ELEM_BYTES[dtype]
            rel = np.asarray(rel, dtype=np.int64) * bpe
            shape = tuple(shape) + (bpe,)
            strides = tuple(int(s) * bpe for s in strides) + (1,)
        self.log(alloc, store, rel, shape, strides, mask=mask)

    def log(self, alloc, store, base, shape, strides, whole=False, group=None, mask=None):
        if store and alloc is not None:
            self.stored.add(id(alloc))
        if self.sequential:
            return
        inst = self.lanes.inst.copy()
        base = np.broadcast_to(np.asarray(base, dtype=np.int64), inst.shape)
        if mask is not None:
            inst, base = inst[mask], base[mask]
        self.accesses.append(Access(alloc, store, inst, np.ascontiguousarray(base),
                                    tuple(shape), tuple(strides), whole, group))

    def materialize(self, t: Tile, dest: Optional[LeafSpec] = None) -> Tile:
        """Evaluate `t` into a fresh contiguous temporary (or into `dest`)."""
        e = t.e
        shape = e.shape if e.shape else (1,)
        if dest is None and e.kind == "ld" and e.attr.alloc is None and e.attr.offsets is None \
                and _contiguous(e.attr.strides, shape) and e.attr.lane.arr is None \
                and e.attr.lane.stride == _prod(shape):
            return t
        L = self.L
        if dest is None:
            n = _prod(shape)
            buf = self.pool.temp(max(1, L * n * rt.ELEM_BYTES[_store_dt(e.dtype)]))
            dest = LeafSpec(buf.ptr, _store_dt(e.dtype), LaneOff(0, n), _cstrides(shape), 0, L * n, keep=(buf,))
            out = Tile(Expr("ld", _store_dt(e.dtype), e.shape, attr=dest))
        else:
            out = None
        self._emit_store(e, dest)
        return out

    def _emit_store(self, e: Expr, dest: LeafSpec, depth=0):
        if len(e.shape) > rt.MAX_DIMS and not e.has_fold:
            c = _collapse_dims(e, dest, rt.MAX_DIMS)
            if c is None:
                raise NotImplementedError(f"a tile expression of rank {len(e.shape)} whose dims do not collapse "
                                          f"to {rt.MAX_DIMS}")
            e, dest = c
        if depth == 0 and self._pattn_finalise(e, dest):
            return
        try:
            prog, keep = compile_program(e, self.L, dest)
        except CompileError:
            if depth > 12:
                raise
            e2 = self._split(e)
            return self._emit_store(e2, dest, depth + 1)
        self.launch("prog", prog, keep + [dest])

    def _pattn_finalise(self, e: Expr, dest: LeafSpec) -> bool:
        """The store right after a paged attention launch of
        cast(acc / l) -- the division and cast that end the reference's
        unified attention kernel (examples/triton-ktir/paged_attention.mlir) --
        runs in that launch's epilogue instead of a launch of its own.  Only
        the exact form: the launch's own acc and l buffers, row-major over the
        stored shape, an output with unit inner stride whose rows are groups
        of evenly spaced rows, no overlap with anything the launch reads."""
        if self.eager or not self.plan.launches:
            return False
        kind, d, keep = self.plan.launches[-1]
        if kind != "pattn" or d.out_ptr or not isinstance(keep, list) or d.lanes != self.L:
            return False
        if e.kind != "cast" or e.attr != "f32" or e.dtype not in ("f16", "bf16", "f32"):
            return False
        dv = e.args[0]
        if dv.kind != "bin" or dv.attr != rt.op("DIVF") or dv.dtype != "f32":
            return False
        a, b = dv.args
        if a.kind != "ld" or b.kind != "ld":
            return False
        A, B = a.attr, b.attr
        M, D = int(d.M), int(d.D)
        shape = tuple(int(x) for x in e.shape)
        if not shape or shape[-1] != D or _prod(shape[:-1]) != M or len(shape) > 3:
            return False
        rows = shape[:-1]
        if A.ptr != d.acc_out or A.dtype != "f32" or A.offsets is not None or A.lane.arr is not None \
                or A.lane.base != 0 or A.lane.stride != M * D or A.strides != _cstrides(shape):
            return False
        if B.ptr != d.l_out or B.dtype != "f32" or B.offsets is not None or B.lane.arr is not None \
                or B.lane.base != 0 or B.lane.stride != M or B.strides != _cstrides(rows) + (0,):
            return False
        if dest.dtype != e.dtype or dest.offsets is not None or dest.winner or dest.strides[-1] != 1:
            return False
        if len(rows) == 1:
            grp, gstride, row = M, 0, dest.strides[0]
        else:
            grp, gstride, row = rows[1], dest.strides[0], dest.strides[1]
        es = rt.ELEM_BYTES[dest.dtype]
        lo_b, hi_b = dest.ptr + dest.lo * es, dest.ptr + dest.hi * es
        width = {c: rt.ELEM_BYTES[n] for n, c in rt.DTYPE_CODE.items() if n in rt.ELEM_BYTES}
        reads = [(d.q_ptr, d.q_lo, d.q_hi, width[d.q_dtype]), (d.k_ptr, d.k_lo, d.k_hi, width[d.kv_dtype]),
                 (d.v_ptr, d.v_lo, d.v_hi, width[d.kv_dtype]), (d.tbl_ptr, d.tbl_lo, d.tbl_hi, width[d.tbl_dtype])]
        if any(p + l * w < hi_b and lo_b < p + h * w for p, l, h, w in reads):
            return False
        base = self.pool.upload(np.ascontiguousarray(dest.lane.values(self.L).astype(np.int64)))
        keep += [base, dest]
        d.out_ptr, d.out_base = dest.ptr, base.ptr
        d.out_grp, d.out_gstride, d.out_row, d.out_lo, d.out_hi = grp, gstride, row, dest.lo, dest.hi
        d.out_dtype = rt.DTYPE_CODE[dest.dtype]
        return True

    def _split(self, e: Expr) -> Expr:
        """Materialise the largest non-trivial subtree of `e` and return the
        rebuilt expression (used when `e` does not fit one program)."""
        nodes = topo(e)
        sizes = {}
        for n in nodes:
            sizes[id(n)] = 1 + sum(sizes[id(a)] for a in n.args)
        cands = [n for n in nodes if n is not e and n.kind not in ("ld", "const", "lane", "idx", "rowval")]
        if e.has_fold:
            folds = [n for n in nodes if n.kind == "fold"]
            cands = folds[:1] + [n for n in cands if not n.has_fold]
        if not cands:
            raise CompileError("cannot split expression")
        best = max(cands, key=lambda n: sizes[id(n)]) if not e.has_fold else cands[0]
        # a sub-expression that cannot compile either splits again; bound the
        # nesting (materialize starts a fresh _emit_store for it)
        self._split_depth = getattr(self, "_split_depth", 0) + 1
        try:
            if self._split_depth > 16:
                raise NotImplementedError(f"a tile expression that no split fits into one program "
                                          f"(shape {tuple(e.shape)})")
            leaf = self.materialize(Tile(best)).e
        finally:
            self._split_depth -= 1
        return _replace(e, best, leaf)

    def hazard_flush(self, alloc: Alloc, keep: Optional[Tile] = None):
        """Materialise every live lazy value that reads `alloc` before it is
        overwritten (loads observe HBM at the time of the load)."""
        for fr in self.frames:
            for name, v in list(fr.vals.items()):
                if isinstance(v, Tile) and v is not keep and _reads(v.e, alloc):
                    if fr.level != len(self.levels) - 1:
                        raise NeedEager("store would race a lazy outer-scope load")
                    fr.vals[name] = self._swap_tile(v, self.materialize(v))

    def _swap_tile(self, old: Tile, new: Tile) -> Tile:
        if new is old:
            return old
        vid, nid = id(old), id(new)
        if vid in self.refcount:
            self.refcount[nid] = self.refcount.pop(vid)
            if vid in self.uncharged:
                self.uncharged.discard(vid)
                self.uncharged.add(nid)
        return new

    # ======================================================================
    # ktdp (reference dialects/ktdp_ops.py:53-260)
    # ======================================================================
    def h_ktdp_get_compute_tile_id(self, op):
        nx, ny, _ = self.grid
        c = self.lanes.cores
        pos = (c % nx, (c // nx) % ny, c // (nx * ny))
        n = max(1, len(op.results))
        return pos[0].astype(np.int64) if n == 1 else tuple(pos[d].astype(np.int64) for d in range(n))

    def h_ktdp_construct_memory_view(self, op):
        a = op.attributes
        ptr = self.get_value(op.operands[0])
        shape = tuple(int(_uniform(self.get_value(s), "view size")) if isinstance(s, str) else int(s)
                      for s in a["shape"])
        strides = tuple(int(_uniform(self.get_value(s), "view stride")) if isinstance(s, str) else int(s)
                        for s in a["strides"])
        cs = a.get("coordinate_set")
        if isinstance(cs, Box) and not cs.is_concrete:
            cs = cs.specialize(tuple(int(_uniform(self.get_value(s), "view size"))
                                     for s in a["shape"] if isinstance(s, str)))
        core = None
        if a["memory_space"] == "LX":
            ct = a.get("lx_core_id")
            if ct is not None and not 0 <= int(ct) < self.n_cores:
                raise IndexError(f"ct_id {ct} names no core of the {self.n_cores}-core grid")
            core = self.lanes.cores.astype(np.int64) if ct is None else np.full(self.L, int(ct), np.int64)
        return View(np.asarray(ptr, dtype=np.int64), shape, strides, _canon(a["dtype"]), a["memory_space"], cs,
                    core)

    def h_ktdp_construct_distributed_memory_view(self, op):
        """Reference dialects/ktdp_ops.py:109-140 with ir_types.py:176-265:
        a dynamic global dim takes the partitions' extent max(hi); a
        declared dim must equal it; every partition has a coordinate set and
        the view's dtype."""
        parts = [self.get_value(n) for n in op.operands]
        for i, p in enumerate(parts):
            if not isinstance(p, View):
                raise ValueError(f"construct_distributed_memory_view: operand {i} is {type(p).__name__}, "
                                 f"expected a memory view")
            if p.cs is None:
                raise ValueError(f"DistributedMemRef partition {i} must have a coordinate_set")
        a = op.attributes
        if "shape" not in a or "dtype" not in a:
            raise ValueError("construct_distributed_memory_view: missing required attributes 'shape'/'dtype'")
        shape = list(a["shape"])
        dtype = _canon(a["dtype"])
        for axis in range(len(shape)):
            his = [p.cs.hi[axis] for p in parts if isinstance(p.cs, Box)]
            ext = max(his) if his else None
            if shape[axis] is None:
                if ext is None:
                    raise ValueError("construct_distributed_memory_view: dynamic axis with no box partition")
                shape[axis] = ext
            elif ext is not None and shape[axis] != ext:
                raise ValueError(f"construct_distributed_memory_view: declared dim {shape[axis]} on axis {axis} "
                                 f"does not match the partition extent {ext}")
        for i, p in enumerate(parts):
            if p.dtype != dtype:
                raise ValueError(f"DistributedMemRef partition {i} dtype {p.dtype!r} does not match view dtype "
                                 f"{dtype!r}")
        return DistView(parts, tuple(shape), dtype)

    def h_ktdp_construct_access_tile(self, op):
        parent = self.get_value(op.operands[0])
        idx = [np.asarray(self.get_value(o), dtype=np.int64) for o in op.operands[1:]]
        a = op.attributes
        cs = a["coordinate_set"]
        if isinstance(cs, Box) and not cs.is_concrete:
            raise NotImplementedError("construct_access_tile: symbolic access_tile_set is not supported")
        base = a["base_map"].eval(idx)
        if isinstance(parent, DistView):
            x = tuple(np.broadcast_to(np.asarray(c, dtype=np.int64), (self.L,)).copy() for c in base)
            if len(x) != len(parent.shape):
                raise ValueError("construct_access_tile: index rank does not match the distributed view")
            return DistATile(parent, x, tuple(a["shape"]), cs)
        off = np.zeros(self.L, dtype=np.int64)
        for c, s in zip(base, parent.strides):
            off = off + np.asarray(c, dtype=np.int64) * int(s)
        return ATile(parent, off, tuple(a["shape"]), cs, a.get("coordinate_order"))

    def h_ktdp_construct_indirect_access_tile(self, op):
        parent = self.get_value(op.operands[0])
        views = [self.get_value(n) for n in op.operands[1:]]
        ivars = op.attributes["intermediate_vars"]
        ssa: Dict[str, np.ndarray] = {}
        shape = tuple(op.attributes["shape"])
        vss = op.attributes["variables_space_set"]

        def collect(e):
            tag = e[0]
            if tag == "ssa":
                ssa[e[1]] = np.asarray(self.get_value(e[1]), dtype=np.int64)
            elif tag in ("add", "sub", "mul"):
                collect(e[1])
                collect(e[2])
            elif tag in ("neg", "floordiv", "ceildiv", "mod"):
                collect(e[1])

        for s in op.attributes["dim_subscripts"]:
            for e in s.get("idx_exprs", []) + ([s["subscript"]] if "subscript" in s else []):
                collect(e)
        outer = {}
        for i, v in enumerate(ivars):
            if self.has_value("%" + v):
                pts = vss.enumerate(shape)
                if any(p[i] != 0 for p in pts):
                    raise ValueError(
                        f"construct_indirect_access_tile: intermediate variable %{v} (index {i}) is an "
                        f"outer SSA value but its dimension in variables_space_set has a non-zero range.")
                outer[i] = np.asarray(self.get_value("%" + v), dtype=np.int64)
        t = IATile(parent, shape, op.attributes["dim_subscripts"], views, vss,
                   op.attributes.get("variables_space_order"), ssa)
        t.ssa["__outer__"] = outer
        return t

    def h_ktdp_load(self, op):
        at = self.get_value(op.operands[0])
        rs = op.attributes.get("_result_shape")
        if isinstance(at, IATile):
            return self.indirect_load(at, rs if rs is not None else at.shape)
        if isinstance(at, DistATile):
            return self.distributed_load(at, tuple(rs) if rs is not None else tuple(at.shape))
        v = at.view
        cs, co = at.cs, at.co
        if isinstance(cs, Box) and co is None and _strides_injective(cs.extent, v.strides):
            lo_off = sum(int(l) * int(s) for l, s in zip(cs.lo, v.strides))
            shape = cs.extent
            spec, alloc, rel = self._hbm_leaf(v, at.origin + lo_off, shape, v.strides)
            self._log_mem(alloc, False, rel, shape, v.strides, v.dtype)
            self._lat_box(rel, shape, v.strides, rt.ELEM_BYTES[v.dtype])
            return Tile(Expr("ld", v.dtype, shape, attr=spec))
        coords = cs.enumerate(at.shape)
        if co is not None:
            coords = [co.eval(p) for p in coords]
        out_shape = tuple(rs) if rs is not None else tuple(at.shape)
        return self._coord_load(v, at.origin, coords, out_shape)

    def _coord_load(self, v: View, origin, coords, out_shape):
        st = np.asarray(v.strides, dtype=np.int64)
        offs = (np.asarray(coords, dtype=np.int64).reshape(len(coords), len(st)) @ st) if len(coords) else \
            np.zeros(0, np.int64)
        if len(offs) != _prod(out_shape):
            raise ValueError(f"cannot reshape {len(offs)} loaded elements into {out_shape}")
        spec, alloc, rel = self._hbm_leaf(v, origin, out_shape, _cstrides(out_shape), offs=offs)
        self._lat_elems(rel, offs, rt.ELEM_BYTES[v.dtype])
        buf = self.pool.upload(offs)
        spec.offsets, spec.offsets_ls = buf, 0
        spec.strides = _cstrides(out_shape) if out_shape else (1,)
        self._log_mem(alloc, False, rel + (offs.min() if len(offs) else 0),
                      (int(np.ptp(offs)) + 1 if len(offs) else 1,), (1,), v.dtype)
        return Tile(Expr("ld", v.dtype, out_shape, attr=spec))

    def h_ktdp_store(self, op):
        val = self.get_value(op.operands[0])
        if not isinstance(val, Tile):
            raise TypeError(f"ktdp.store expects a Tile, got {type(val)}")
        at = self.get_value(op.operands[1])
        if isinstance(at, IATile):
            self.indirect_store(val, at)
            return None
        if isinstance(at, DistATile):
            self.distributed_store(val, at)
            return None
        v = at.view
        cs, co = at.cs, at.co
        if isinstance(cs, Box) and co is None and _strides_injective(cs.extent, v.strides):
            lo_off = sum(int(l) * int(s) for l, s in zip(cs.lo, v.strides))
            shape = cs.extent
            spec, alloc, rel = self._hbm_leaf(v, at.origin + lo_off, shape, v.strides)
            from .fusion import mm_epilogue
            if not mm_epilogue(self, op, val, spec, alloc, shape):
                self._store_expr(val, spec, alloc, shape)
            self._log_mem(alloc, True, rel, shape, v.strides, v.dtype)
            self._lat_box(rel, shape, v.strides, rt.ELEM_BYTES[v.dtype])
            return None
        coords = cs.enumerate(at.shape)
        if co is not None:
            coords = [co.eval(p) for p in coords]
        st = np.asarray(v.strides, dtype=np.int64)
        offs = np.asarray(coords, dtype=np.int64).reshape(len(coords), len(st)) @ st
        n = _prod(val.shape)
        if len(offs) != n:
            raise ValueError("ktdp.store: tile size does not match the access tile's points")
        spec, alloc, rel = self._hbm_leaf(v, at.origin, val.shape, _cstrides(val.shape), offs=offs)
        self._lat_elems(rel, offs, rt.ELEM_BYTES[v.dtype])
        spec.offsets, spec.offsets_ls = self.pool.upload(offs), 0
        if len(np.unique(offs)) != len(offs):
            self._winners(spec, n)
        self._store_expr(val, spec, alloc, val.shape)
        self._log_mem(alloc, True, rel + (offs.min() if len(offs) else 0),
                      (int(np.ptp(offs)) + 1 if len(offs) else 1,), (1,), v.dtype)
        return None

    def _store_expr(self, val: Tile, dest: LeafSpec, alloc: Alloc, shape):
        if tuple(val.shape) != tuple(shape) and _prod(val.shape) == _prod(shape):
            val = self.reshape(val, tuple(shape))
        elif tuple(val.shape) != tuple(shape):
            val = self.broadcast_to(val, tuple(shape))
        self.hazard_flush(alloc, keep=val)
        e = val.e
        if _reads(e, alloc) and not _same_access(e, dest, alloc):
            e = self.materialize(Tile(e)).e
        if e.dtype != dest.dtype and not (is_float(e.dtype) and is_float(dest.dtype)):
            e = Expr("cast", dest.dtype, e.shape, [e], e.dtype)
        from .fusion import attention_epilogue
        if attention_epilogue(self, e, dest):
            return
        self.materialize(Tile(e), dest=dest)

    def _winners(self, spec: LeafSpec, n: int):
        """Last-writer-wins table for a scatter whose offsets may repeat."""
        a = spec.alloc
        tb = self.pool.temp(a.n_elems * 4)
        leaf = rt.Leaf()
        from .program import _fill_leaf
        keep = []
        _fill_leaf(leaf, spec, self.L, len(spec.strides), keep)
        self.launch("winners", (leaf, self.L, n, tb.ptr), keep + [tb])
        spec.winner = tb
        spec.winner_base = 0

    # -- indirect access (reference ops/memory_ops.py:224-576, 868-964) --------
    # -- distributed views (reference ops/memory_ops.py:986-1259) ------------
    _ABSENT = 1 << 60      # offset-list entry that lies past every window: read 0, write dropped

    def _dist_routes(self, at: DistATile):
        """Per partition i, for every lane: C_i = B_i & (x + A) and the
        partition origin p_i = min(B_i) (reference memory_ops.py:986-1098).
        Returns [(view, kind, lane mask, data, p_i)] with kind "box" (data =
        per-lane lo/hi arrays) or "pts" (data = the partition's points)."""
        dist, x, A, L = at.dist, at.x, at.cs, self.L
        nd = len(dist.shape)
        if isinstance(A, Box) and not A.is_concrete:
            raise NotImplementedError("construct_access_tile: symbolic access_tile_set is not supported")
        routes, any_hit = [], np.zeros(L, dtype=bool)
        for part in dist.parts:
            B = part.cs
            if isinstance(B, Box) and isinstance(A, Box):
                lo = [np.maximum(B.lo[d], x[d] + A.lo[d]) for d in range(nd)]
                hi = [np.minimum(B.hi[d], x[d] + A.hi[d]) for d in range(nd)]
                m = np.ones(L, dtype=bool)
                for l, h in zip(lo, hi):
                    m &= h > l
                routes.append((part, "box", m, (lo, hi), tuple(B.lo)))
            else:
                pts = np.asarray(B.enumerate() if isinstance(B, Box) else B.enumerate(dist.shape),
                                 dtype=np.int64).reshape(-1, nd)
                if not len(pts):
                    continue
                rel = pts[None, :, :] - np.stack(x, axis=1)[:, None, :]            # lane x point x dim
                if A is None:
                    inside = np.all((rel >= 0) & (rel < np.asarray(at.shape, dtype=np.int64)), axis=2)
                else:
                    inside = A.mask([rel[:, :, d] for d in range(nd)])
                m = inside.any(axis=1)
                routes.append((part, "pts", m, (pts, inside), tuple(int(v) for v in pts.min(axis=0))))
            any_hit |= routes[-1][2]
        if not np.all(any_hit):
            c = int(self.lanes.cores[int(np.flatnonzero(~any_hit)[0])])
            xs = tuple(int(v[int(np.flatnonzero(~any_hit)[0])]) for v in x)
            raise ValueError(f"distributed_tile_access: no partition covers access region global_base={xs} "
                             f"shape={tuple(at.shape)} (core {c})")
        return routes

    def _dist_single(self, at: DistATile, routes, shape):
        """The common case as one strided leaf: every lane's access lies
        whole inside one partition, the tile starts at the access origin,
        and the partitions reached share strides and memory space.  Returns
        (leaf, alloc, rel, strides) or None."""
        A = at.cs
        if not isinstance(A, Box) or any(l != 0 for l in A.lo) or tuple(A.hi) != tuple(shape):
            return None
        L, nd = self.L, len(shape)
        pick = np.full(L, -1, dtype=np.int64)
        for k, (part, kind, m, data, p_i) in enumerate(routes):
            if not m.any():
                continue
            if kind != "box":
                return None
            lo, hi = data
            full = m.copy()
            for d in range(nd):
                full &= (lo[d] == at.x[d]) & (hi[d] == at.x[d] + A.hi[d])
            if np.any(m != full) or np.any(pick[m] >= 0):
                return None
            pick[m] = k
        used = [routes[k][0] for k in np.unique(pick)]
        v0 = used[0]
        if any(v.strides != v0.strides or v.space != v0.space for v in used):
            return None
        base = np.zeros(L, dtype=np.int64)
        core = None if v0.core is None else np.zeros(L, dtype=np.int64)
        for k in np.unique(pick):
            part, _, _, _, p_i = routes[k]
            sel = pick == k
            off = np.zeros(int(sel.sum()), dtype=np.int64)
            for d in range(nd):
                off += (at.x[d][sel] - p_i[d]) * part.strides[d]
            base[sel] = part.base[sel] + off
            if core is not None:
                core[sel] = part.core[sel]
        view = View(base, tuple(shape), v0.strides, v0.dtype, v0.space, None, core)
        try:
            spec, alloc, rel = self._hbm_leaf(view, np.zeros(L, dtype=np.int64), shape, v0.strides)
        except NotImplementedError:
            return None
        return spec, alloc, rel, v0.strides

    def _dist_offsets(self, at: DistATile, route, shape):
        """Offset lists of one partition: for every lane and every position
        n of the tile, the element offset inside the partition (from its
        pointer) of global point x + n when that point lies in C_i, else
        absent; plus the per-lane lowest/highest offset used."""
        part, kind, m, data, p_i = route
        L, nd, N = self.L, len(shape), _prod(shape)
        cst = np.asarray(_cstrides(shape), dtype=np.int64)
        pst = np.asarray(part.strides, dtype=np.int64)
        pos = np.full((L, N), self._ABSENT, dtype=np.int64)
        src = np.full((L, N), self._ABSENT, dtype=np.int64)
        lo_o = np.zeros(L, dtype=np.int64)
        hi_o = np.zeros(L, dtype=np.int64)
        for l in np.flatnonzero(m):
            xl = np.array([int(v[l]) for v in at.x], dtype=np.int64)
            if kind == "box":
                lo, hi = data
                g = np.indices(tuple(int(hi[d][l] - lo[d][l]) for d in range(nd))).reshape(nd, -1).T
                g = g + np.array([int(lo[d][l]) for d in range(nd)], dtype=np.int64)
            else:
                pts, inside = data
                g = pts[inside[l]]
            rel = g - xl
            if np.any(rel < 0) or np.any(rel >= np.asarray(shape, dtype=np.int64)):
                raise ValueError("distributed access: a covered point falls outside the result tile")
            n = rel @ cst
            o = (g - np.asarray(p_i, dtype=np.int64)) @ pst
            pos[l, n] = n
            src[l, n] = o
            if len(np.unique(o)) != len(o):
                raise NotImplementedError("distributed partition whose strides alias elements")
            lo_o[l], hi_o[l] = int(o.min()), int(o.max()) + 1
        return pos, src, lo_o, hi_o

    def _dist_leaf(self, route, src, lo_o, hi_o, shape):
        part, _, m, _, _ = route
        L = self.L
        if part.space == "HBM":
            spec, alloc, rel = self._hbm_leaf(part, np.zeros(L, dtype=np.int64), shape, _cstrides(shape))
        else:
            spec, alloc, rel = self._lx_leaf(part, np.zeros(L, dtype=np.int64), shape, _cstrides(shape),
                                             span=(lo_o, hi_o))
        spec.offsets, spec.offsets_ls = self.pool.upload(src), _prod(shape)
        spec.strides = _cstrides(shape)
        return spec, alloc, rel

    def distributed_load(self, at: DistATile, shape):
        """Reference memory_ops.py:1127-1196: a zero tile; each partition's
        C_i, read at C_i - p_i, lands at C_i - x."""
        shape = tuple(int(d) for d in shape)
        dtype = at.dist.dtype
        routes = self._dist_routes(at)
        one = self._dist_single(at, routes, shape)
        if one is not None:
            spec, alloc, rel, strides = one
            self._log_mem(alloc, False, rel, shape, strides, dtype)
            self._lat_box(rel, shape, strides, rt.ELEM_BYTES[dtype])
            return Tile(Expr("ld", dtype, shape, attr=spec))
        L, N = self.L, _prod(shape)
        out = self.materialize(Tile(E_const(0, _store_dt(dtype), shape)))
        dst = out.e.attr
        for route in routes:
            part, _, m, _, _ = route
            if not m.any():
                continue
            pos, src, lo_o, hi_o = self._dist_offsets(at, route, shape)
            spec, alloc, rel = self._dist_leaf(route, src, lo_o, hi_o, shape)
            dest = LeafSpec(dst.ptr, dst.dtype, dst.lane, dst.strides, dst.lo, dst.hi,
                            offsets=self.pool.upload(pos), offsets_ls=N, keep=dst.keep)
            self._emit_store(Expr("ld", dtype, shape, attr=spec), dest)
            self._log_mem(alloc, False, rel + lo_o, (int(np.max(hi_o - lo_o)),), (1,), dtype, mask=m)
        return Tile(Expr("ld", dst.dtype, shape, attr=dst))

    def distributed_store(self, val: Tile, at: DistATile):
        """Reference memory_ops.py:1199-1259: only C_i is written in each
        partition, from the tile's positions C_i - x."""
        shape = tuple(int(d) for d in at.shape)
        dtype = at.dist.dtype
        if tuple(val.shape) != shape:
            if _prod(val.shape) != _prod(shape):
                raise ValueError(f"ktdp.store: tile shape {tuple(val.shape)} does not match the access tile "
                                 f"{shape}")
            val = self.reshape(val, shape)
        routes = self._dist_routes(at)
        one = self._dist_single(at, routes, shape)
        if one is not None:
            spec, alloc, rel, strides = one
            self._store_expr(val, spec, alloc, shape)
            self._log_mem(alloc, True, rel, shape, strides, dtype)
            self._lat_box(rel, shape, strides, rt.ELEM_BYTES[dtype])
            return
        live = [r for r in routes if r[2].any()]
        if len(live) > 1:
            val = self.materialize(val)
        for route in live:
            _, _, m, _, _ = route
            pos, src, lo_o, hi_o = self._dist_offsets(at, route, shape)
            spec, alloc, rel = self._dist_leaf(route, src, lo_o, hi_o, shape)
            self._store_expr(val, spec, alloc, shape)
            self._log_mem(alloc, True, rel + lo_o, (int(np.max(hi_o - lo_o)),), (1,), dtype, mask=m)

    def iat_parts(self, at: IATile):
        """Host part of an indirect access tile: (n points, direct element
        offsets [1 or lanes, n], [(index view, element positions in it
        [1 or lanes, n], parent stride)] per indirect dimension), points in
        the order of the variables space (reference ops/memory_ops.py:491-576)."""
        if at.vso is not None and not at.vso.is_permutation():
            raise ValueError("variables_space_order must permute its input dimensions")
        if at.parent.space != "HBM" or any(v.space != "HBM" for v in at.views):
            raise NotImplementedError("indirect access tile over LX memory")
        pts = at.vss.enumerate(at.shape)
        if at.vso is not None:
            pts = sorted(pts, key=lambda p: at.vso.eval(p))
        P = np.asarray(pts, dtype=np.int64).reshape(len(pts), len(at.shape))
        n = len(P)
        outer = at.ssa.get("__outer__", {})
        cols = []
        for k in range(P.shape[1]):
            if k in outer:
                cols.append(outer[k][:, None] + np.zeros((1, n), np.int64))
            else:
                cols.append(P[:, k][None, :])

        def ssa(name):
            return at.ssa[name][:, None]

        pst = at.parent.strides
        direct = np.zeros((1, n), dtype=np.int64)
        ind = []
        for d, sub in enumerate(at.subs):
            if sub["kind"] == "direct":
                direct = direct + cols[sub["var_index"]] * pst[d]
            elif sub["kind"] == "direct_expr":
                direct = direct + np.asarray(evaluate(sub["subscript"], cols, ssa=ssa), dtype=np.int64) * pst[d]
            else:
                iv = at.views[sub["index_view_idx"]]
                pos = np.zeros((1, n), dtype=np.int64)
                for ex, s in zip(sub["idx_exprs"], iv.strides):
                    pos = pos + np.asarray(evaluate(ex, cols, ssa=ssa), dtype=np.int64) * int(s)
                ind.append((iv, pos, pst[d]))
        if len(ind) > 4:
            raise NotImplementedError("more than 4 indirect dimensions")
        return n, direct, ind

    def _iat_offsets(self, at: IATile) -> Tuple[rt.DeviceBuffer, int, LeafSpec, Alloc]:
        n, direct, ind = self.iat_parts(at)
        L = self.L
        d = rt.IAT()
        d.lanes, d.n = L, n
        direct = np.broadcast_to(direct, (direct.shape[0], n)).astype(np.int64)
        dbuf = self.pool.upload(direct)
        d.dir, d.dir_ls = dbuf.ptr, (n if direct.shape[0] > 1 else 0)
        keep = [dbuf]
        d.n_ind = len(ind)
        for k, (iv, pos, stride) in enumerate(ind):
            ibpe = rt.ELEM_BYTES[iv.dtype]
            base = iv.base.astype(np.int64)
            ia = self._alloc_of(base * ibpe)
            self.log(ia, False, np.zeros(L, np.int64), (1,), (1,), whole=True)
            pos = np.broadcast_to(pos, (pos.shape[0], n)).astype(np.int64)
            pb = self.pool.upload(pos)
            keep.append(pb)
            lane_rel = base - ia.addr // ibpe
            lb = self.pool.upload(lane_rel)
            keep.append(lb)
            d.idx_ptr[k] = self.arena.ptr_of(ia)
            d.idx_dtype[k] = rt.DTYPE_CODE[iv.dtype]
            d.idx_lo[k], d.idx_hi[k] = 0, ia.n_elems
            d.pos[k], d.pos_ls[k] = pb.ptr, (n if pos.shape[0] > 1 else 0)
            d.pos_lane[k] = lb.ptr
            d.stride[k] = int(stride)
        out = self.pool.temp(max(1, L * n * 8))
        d.out = out.ptr
        self.launch("iat", d, keep + [out])
        spec, alloc, rel = self._hbm_leaf(at.parent, np.zeros(L, np.int64), (n,), (1,))
        spec.offsets, spec.offsets_ls = out, n
        spec.keep = spec.keep + (out,)
        if self.lat is not None:
            # index-tensor sticks from the positions read, data sticks from the
            # offsets the GPU computed (the run is eager, so they exist now)
            from .latency import unique_sticks_elems
            idx_k = np.zeros(L, np.int64)
            for iv, pos, _ in ind:
                ibpe = rt.ELEM_BYTES[iv.dtype]
                ia = self._alloc_of(iv.base.astype(np.int64) * ibpe)
                lane_rel = iv.base.astype(np.int64) - ia.addr // ibpe
                p = np.broadcast_to(pos, (L, n))
                idx_k += np.array([unique_sticks_elems((lr + pp) * ibpe) for lr, pp in zip(lane_rel, p)], np.int64)
            rt.sync()
            raw = out.buf.download(L * n * 8)
            offs = np.frombuffer(raw.tobytes(), dtype=np.int64).reshape(L, n)
            self._lat_iat = (rel, offs, rt.ELEM_BYTES[at.parent.dtype], idx_k)
        return out, n, spec, alloc

    def indirect_load(self, at: IATile, result_shape):
        _, n, spec, alloc = self._iat_offsets(at)
        self.log(alloc, False, np.zeros(self.L, np.int64), (1,), (1,), whole=True)
        if self.lat is not None:
            rel, offs, bpe, idx_k = self._lat_iat
            self._lat_elems(rel, offs, bpe, extra=idx_k)
        shape = tuple(result_shape)
        if _prod(shape) != n:
            raise ValueError(f"cannot reshape {n} gathered elements into {shape}")
        spec.strides = _cstrides(shape) if shape else (1,)
        return Tile(Expr("ld", at.parent.dtype, shape, attr=spec))

    def indirect_store(self, val: Tile, at: IATile):
        if tuple(val.shape) != tuple(at.shape):
            raise ValueError(f"indirect_store: source tile shape {tuple(val.shape)} does not match "
                             f"IAT shape {tuple(at.shape)}")
        _, n, spec, alloc = self._iat_offsets(at)
        spec.strides = _cstrides(val.shape) if val.shape else (1,)
        if self.lat is not None:
            rel, offs, bpe, idx_k = self._lat_iat
            lat_mem = (rel, offs, bpe, idx_k)
        self._winners(spec, n)
        self.log(alloc, True, np.zeros(self.L, np.int64), (1,), (1,), whole=True)
        self._store_expr(val, spec, alloc, val.shape)
        if self.lat is not None:
            rel, offs, bpe, idx_k = lat_mem
            self._lat_elems(rel, offs, bpe, extra=idx_k)

    # ======================================================================
    # arith / math (reference dialects/arith_ops.py, ops/arith_ops.py, ops/math_ops.py)
    # ======================================================================
    def h_arith_constant(self, op):
        a = op.attributes
        v = a.get("value", 0)
        if a.get("is_tensor"):
            dt = _canon(a.get("dtype", "f16"))
            shape = tuple(a["shape"])
            if a.get("dense_list"):
                arr = np.array(v, dtype=NP_DTYPE.get(dt, np.float32)).reshape(shape)
                return self._host_tile(np.broadcast_to(arr, (self.L,) + shape), dt)
            return Tile(E_const(_round_val(v, dt), dt, shape))
        if isinstance(v, bool):
            return np.full(self.L, v, dtype=bool)
        if isinstance(v, int):
            return np.full(self.L, v, dtype=np.int64)
        return np.full(self.L, v, dtype=np.float64)

    def _host_tile(self, arr: np.ndarray, dt: str) -> Tile:
        """A tile whose per-lane contents are known on the host."""
        shape = arr.shape[1:]
        store = {"bf16": np.uint16}.get(dt, NP_DTYPE.get(dt, np.float32))
        if dt == "bf16":
            from .program import round_host as _r
            f = np.asarray(arr, dtype=np.float32)
            b = f.view(np.uint32)
            b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
            data = b
        else:
            data = np.asarray(arr, dtype=store)
        buf = self.pool.upload(np.ascontiguousarray(data).reshape(-1))
        n = _prod(shape)
        spec = LeafSpec(buf.ptr, dt if dt != "index" else "i32", LaneOff(0, n), _cstrides(shape) if shape else (1,),
                        0, self.L * n, keep=(buf,))
        return Tile(Expr("ld", spec.dtype, shape, attr=spec))

    def _operand(self, v, dt: str, shape, float_scalar=True) -> Expr:
        """Tile operand expression, broadcasting scalars (rounded to f16 like
        the reference's `np.float16(scalar)` coercion when float_scalar)."""
        if isinstance(v, Tile):
            return self.broadcast_to(v, shape).e if tuple(v.shape) != tuple(shape) else v.e
        if isinstance(v, DevScalar):
            if is_float(dt):
                # registers hold f32: the f16 value needs no widening cast
                t = self._cast_tile(v.t, "f16") if float_scalar else v.t
                return self._ds_broadcast(t, shape).e
            v = self.host_scalar(v)
        arr = np.asarray(v)
        if float_scalar and is_float(dt):
            arr = arr.astype(np.float64)
            arr = np.asarray(arr, dtype=np.float16).astype(np.float64)
            return E_scalar(arr, "f32", shape)
        if is_float(dt):
            return E_scalar(arr.astype(np.float64), "f32", shape)
        return E_scalar(arr.astype(np.int64), "i32", shape)

    def float_binop(self, op, code):
        a, b = self.get_value(op.operands[0], dev=True), self.get_value(op.operands[1], dev=True)
        if not isinstance(a, Tile) and not isinstance(b, Tile):
            if isinstance(a, DevScalar) or isinstance(b, DevScalar):
                # both scalars rounded to f16, an f16 result (dialects/_helpers.py:47-50)
                ea, eb = self._scalar_operand(a, "f16"), self._scalar_operand(b, "f16")
                return DevScalar(Tile(Expr("bin", "f16", (1,), [ea, eb], rt.op(code))))
            fn = SCALAR_FLOAT[op.op_type]
            with np.errstate(all="ignore"):
                return np.asarray(fn(np.asarray(a, dtype=np.float16), np.asarray(b, dtype=np.float16)),
                                  dtype=np.float16)
        ref = a if isinstance(a, Tile) else b
        shape = _bshape(a, b)
        dt = _res_float_dt(a, b)
        ea = self._operand(a, ref.dtype, shape)
        eb = self._operand(b, ref.dtype, shape)
        return Tile(Expr("bin", dt, shape, [ea, eb], rt.op(code)))

    def minmax(self, op):
        a, b = self.get_value(op.operands[0], dev=True), self.get_value(op.operands[1], dev=True)
        f = SCALAR_MINMAX[op.op_type]
        if not isinstance(a, Tile) and not isinstance(b, Tile):
            if isinstance(a, DevScalar) or isinstance(b, DevScalar):
                # NumPy's promotion of two scalars: a NumPy float scalar keeps
                # its type against a Python float, the wider of two NumPy types wins
                kinds = [_scalar_kind(x) for x in (a, b)]
                if kinds == [None, None]:
                    a, b = (self.host_scalar(x) if isinstance(x, DevScalar) else x for x in (a, b))
                    return f(a, b)
                dt = "f32" if "f32" in kinds else "f16"
                ea, eb = self._scalar_operand(a, dt), self._scalar_operand(b, dt)
                return DevScalar(Tile(Expr("bin", dt, (1,), [ea, eb], rt.op(MINMAX_F[op.op_type]))))
            return f(a, b)
        ref = a if isinstance(a, Tile) else b
        shape = _bshape(a, b)
        dt = _res_float_dt(a, b) if isinstance(a, Tile) and isinstance(b, Tile) else ref.dtype
        ea = self._operand(a, ref.dtype, shape, float_scalar=False)
        eb = self._operand(b, ref.dtype, shape, float_scalar=False)
        return Tile(Expr("bin", dt, shape, [ea, eb], rt.op(MINMAX_F[op.op_type])))

    def int_binop(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        if not isinstance(a, Tile) and not isinstance(b, Tile):
            t = op.op_type
            a, b = np.asarray(a), np.asarray(b)
            if t == "arith.shrui":
                return (a.astype(np.int32).view(np.uint32) >> b.astype(np.uint32)).astype(np.int64)
            with np.errstate(all="ignore"):
                if t in ("arith.divui", "arith.floordivsi"):
                    r = _np_floordiv(a.astype(np.int64), b.astype(np.int64))
                elif t == "arith.remui":
                    r = np.mod(a.astype(np.int64), np.where(b == 0, 1, b).astype(np.int64))
                else:
                    r = SCALAR_INT[t](a, b)
            return np.asarray(r)
        ref = a if isinstance(a, Tile) else b
        shape = _bshape(a, b)
        ea = self._operand(a, ref.dtype, shape, float_scalar=False)
        eb = self._operand(b, ref.dtype, shape, float_scalar=False)
        return Tile(Expr("bin", ref.dtype, shape, [ea, eb], rt.op(INT_BIN[op.op_type])))

    def math_unary(self, op):
        v = self.get_value(op.operands[0], dev=True)
        if isinstance(v, DevScalar):
            if not v.weak:
                # a NumPy float scalar keeps its type (ops/_helpers.py:59-60)
                return DevScalar(Tile(Expr("un", v.dtype, v.t.shape, [v.t.e], rt.op(MATH_UN[op.op_type]))))
            v = self.host_scalar(v)      # a Python float: float64 math
        if not isinstance(v, Tile):
            x = np.asarray(v)
            if not np.issubdtype(x.dtype, np.floating):
                x = x.astype(np.float64)
            with np.errstate(all="ignore"):
                return np.asarray(SCALAR_MATH[op.op_type](x)).astype(x.dtype)
        return Tile(Expr("un", v.dtype, v.shape, [v.e], rt.op(MATH_UN[op.op_type])))

    def h_arith_negf(self, op):
        v = self.get_value(op.operands[0], dev=True)
        if isinstance(v, DevScalar):
            return DevScalar(Tile(Expr("un", v.dtype, v.t.shape, [v.t.e], rt.op("NEGF"))), v.weak)
        return Tile(Expr("un", v.dtype, v.shape, [v.e], rt.op("NEGF"))) if isinstance(v, Tile) else -v

    def h_arith_absf(self, op):
        v = self.get_value(op.operands[0], dev=True)
        if isinstance(v, DevScalar):
            return DevScalar(Tile(Expr("un", v.dtype, v.t.shape, [v.t.e], rt.op("ABSF"))), v.weak)
        return Tile(Expr("un", v.dtype, v.shape, [v.e], rt.op("ABSF"))) if isinstance(v, Tile) else np.abs(v)

    h_math_absf = h_arith_absf

    def h_math_absi(self, op):
        v = self.get_value(op.operands[0])
        return Tile(Expr("un", v.dtype, v.shape, [v.e], rt.op("ABSI"))) if isinstance(v, Tile) else np.abs(v)

    def h_math_powf(self, op):
        b, e = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        if isinstance(b, Tile):
            ee = self._operand(e, "f32", b.shape, float_scalar=False)
            return Tile(Expr("bin", b.dtype, b.shape, [b.e, ee], rt.op("POWF")))
        return np.asarray(np.power(np.asarray(b, dtype=np.float64), np.asarray(e, dtype=np.float64)))

    def h_math_fma(self, op):
        a, b, c = (self.get_value(o) for o in op.operands[:3])
        if isinstance(a, Tile):
            sh = a.shape
            return Tile(Expr("fma", a.dtype, sh, [a.e, self._operand(b, a.dtype, sh, False),
                                                  self._operand(c, a.dtype, sh, False)]))
        return np.asarray(a, dtype=np.float64) * b + c

    def h_arith_cmpi(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        p = op.attributes["predicate"]
        if p not in CMPI:
            raise NotImplementedError(f"arith.cmpi: unsupported predicate '{p}'")
        if not isinstance(a, Tile) and not isinstance(b, Tile):
            fns = {"slt": np.less, "ult": np.less, "sle": np.less_equal, "ule": np.less_equal,
                   "sgt": np.greater, "ugt": np.greater, "sge": np.greater_equal, "uge": np.greater_equal,
                   "eq": np.equal, "ne": np.not_equal}
            return fns[p](a, b)
        shape = _bshape(a, b)
        ref = a if isinstance(a, Tile) else b
        ea = self._operand(a, ref.dtype, shape, False)
        eb = self._operand(b, ref.dtype, shape, False)
        return Tile(Expr("cmpi", "i1", shape, [ea, eb], rt.cmp(CMPI[p])))

    def h_arith_cmpf(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        p = op.attributes["predicate"]
        if p not in CMPF:
            raise NotImplementedError(f"arith.cmpf: unsupported predicate '{p}'")
        if not isinstance(a, Tile) and not isinstance(b, Tile):
            l, r = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
            nan = np.isnan(l) | np.isnan(r)
            with np.errstate(all="ignore"):
                tab = {"false": np.zeros_like(nan), "oeq": l == r, "one": (l != r) & ~nan, "olt": l < r,
                       "ole": l <= r, "ogt": l > r, "oge": l >= r, "ueq": (l == r) | nan, "une": l != r,
                       "ult": (l < r) | nan, "ule": (l <= r) | nan, "ugt": (l > r) | nan, "uge": (l >= r) | nan,
                       "ord": ~nan, "uno": nan, "true": np.ones_like(nan)}
            return tab[p]
        shape = _bshape(a, b)
        ref = a if isinstance(a, Tile) else b
        ea = self._operand(a, ref.dtype, shape, False)
        eb = self._operand(b, ref.dtype, shape, False)
        return Tile(Expr("cmpf", "i1", shape, [ea, eb], rt.cmp(CMPF[p])))

    def h_arith_select(self, op):
        c, t, f = (self.get_value(o) for o in op.operands[:3])
        if not any(isinstance(x, Tile) for x in (c, t, f)):
            return np.where(np.asarray(c, dtype=bool), t, f)
        ref = t if isinstance(t, Tile) else (f if isinstance(f, Tile) else None)
        if ref is None:
            dt = "f16"
            shape = c.shape
        else:
            dt, shape = ref.dtype, tuple(np.broadcast_shapes(*(x.shape for x in (c, t, f) if isinstance(x, Tile))))
        ec = self._operand(c, "i1", shape, False) if isinstance(c, Tile) else E_scalar(
            np.asarray(c, dtype=np.int64), "i32", shape)
        et = self._operand(t, dt, shape, False)
        ef = self._operand(f, dt, shape, False)
        return Tile(Expr("sel", dt, shape, [ec, et, ef]))

    def _cast_tile(self, v: Tile, dt: str) -> Tile:
        if v.dtype == dt:
            return v
        return Tile(Expr("cast", dt, v.shape, [v.e], v.dtype))

    def h_arith_extf(self, op):
        v = self.get_value(op.operands[0], dev=True)
        if isinstance(v, DevScalar):
            # from f16 or f32: exact, never overflows
            return DevScalar(self._cast_tile(v.t, "f32"))
        if isinstance(v, Tile):
            return self._cast_tile(v, "f32")
        return _narrow_scalar(v, np.float32, "extf")

    def h_arith_truncf(self, op):
        dt = _elem_of(op.result_type) or "f16"
        dt = "bf16" if dt == "bf16" else "f16"
        v = self.get_value(op.operands[0], dev=True)
        if isinstance(v, DevScalar):
            if dt == "bf16":
                return DevScalar(self._cast_tile(self._cast_tile(v.t, "bf16"), "f32"))
            if v.dtype == "f16" and not v.weak:
                return v
            # an f32 value that f16 cannot hold raises: read it on the host
            v = self.host_scalar(v)
        if isinstance(v, Tile):
            return self._cast_tile(v, dt)
        if dt == "bf16":
            return np.asarray([round_host(float(x), "bf16") for x in np.asarray(v).ravel()], dtype=np.float32)
        return _narrow_scalar(v, np.float16, "truncf")

    def h_arith_extsi(self, op):
        v = self.get_value(op.operands[0])
        return self._cast_tile(v, "i64") if isinstance(v, Tile) else np.asarray(v, dtype=np.int64)

    h_arith_extui = h_arith_extsi

    def h_arith_trunci(self, op):
        v = self.get_value(op.operands[0])
        return self._cast_tile(v, "i32") if isinstance(v, Tile) else np.asarray(v, dtype=np.int64)

    def h_arith_fptosi(self, op):
        v = self.get_value(op.operands[0])
        if isinstance(v, Tile):
            return self._cast_tile(v, "i32")
        return np.trunc(np.asarray(v, dtype=np.float64)).astype(np.int64)

    h_arith_fptoui = h_arith_fptosi

    def h_arith_sitofp(self, op):
        v = self.get_value(op.operands[0])
        dt = _elem_of(op.result_type) or "f32"
        if isinstance(v, Tile):
            return self._cast_tile(v, dt)
        return np.asarray(v).astype(NP_DTYPE.get(dt, np.float32))

    def h_arith_uitofp(self, op):
        v = self.get_value(op.operands[0])
        return self._cast_tile(v, "f32") if isinstance(v, Tile) else np.asarray(v, dtype=np.float64)

    def h_arith_index_cast(self, op):
        v = self.get_value(op.operands[0])
        if isinstance(v, Tile):
            raise NeedEager("index_cast of a tile")
        return np.asarray(v).astype(np.int64)

    h_arith_index_castui = h_arith_index_cast

    def h_arith_bitcast(self, op):
        v = self.get_value(op.operands[0])
        dst = op.attributes.get("dst_type", "f32")
        if isinstance(v, Tile):
            if dst not in ("f32", "i32", "si32"):
                raise NotImplementedError(f"arith.bitcast: unsupported dst_type '{dst}' for Tile")
            return Tile(Expr("bitcast", "f32" if dst == "f32" else "i32", v.shape, [v.e]))
        arr = np.asarray(v)
        if dst == "f32":
            return arr.astype(np.int64).astype(np.int32).view(np.float32).astype(np.float64)
        if dst in ("i32", "si32"):
            return arr.astype(np.float32).view(np.int32).astype(np.int64)
        raise NotImplementedError(f"arith.bitcast: unsupported dst_type '{dst}' for scalar")

    def h_arith_shrui(self, op):
        return self.int_binop(op)

    # ======================================================================
    # tensor (reference dialects/tensor_ops.py)
    # ======================================================================
    def h_tensor_empty(self, op):
        shape = tuple(op.attributes.get("shape", (1,)))
        dt = _canon(op.attributes.get("dtype", "f16"))
        return Tile(E_const(0, dt, shape))

    def h_tensor_splat(self, op):
        s = self.get_value(op.operands[0], dev=True)
        if isinstance(s, Tile):
            # the reference splats the tile's first element
            if not is_float(s.dtype):
                raise NeedEager("tensor.splat of an integer tile element")
            s = DevScalar(self._element(s, []))
        shape = tuple(op.attributes.get("shape", ()))
        dt = _canon(op.attributes.get("dtype", "f16"))
        if not shape:
            shape = (1,)
        if isinstance(s, DevScalar):
            if is_float(dt) or dt == "i32":
                # np.full: one conversion of the scalar to the tile's type
                return self._cast_tile(self._ds_broadcast(s.t, shape), dt)
            s = self.host_scalar(s)
        arr = np.asarray(s)
        if np.issubdtype(arr.dtype, np.integer) and arr.dtype != np.bool_:
            return Tile(E_scalar(arr.astype(np.int64), "i32", shape))
        vals = np.array([_round_val(float(x), dt) for x in np.asarray(arr, dtype=np.float64).ravel()])
        return Tile(E_scalar(vals, dt, shape))

    def h_tensor_extract(self, op):
        src = self.get_value(op.operands[0], dev=True)
        idx = [self.get_value(o) for o in op.operands[1:]]
        if not isinstance(src, Tile):
            return src
        if is_float(src.dtype):
            # the element stays on the device; only a host use reads it
            return DevScalar(self._element(src, idx))
        if not self.eager and self.collective:
            self._go_eager()
        if not self.eager:
            raise NeedEager("tensor.extract reads tile data on the host")
        data = self.read_tile(src)
        if not idx:
            v = data.reshape(self.L, -1)[:, 0]
        else:
            ii = tuple(np.asarray(i, dtype=np.int64) for i in idx)
            v = data[(np.arange(self.L),) + ii]
        if src.dtype in ("f16",):
            return v.astype(np.float16)
        if src.dtype in ("f32", "bf16"):
            return v.astype(np.float32)
        return v.astype(np.int64) if src.dtype != "i1" else v.astype(bool)

    def _go_eager(self):
        """Run what the walk has recorded so far and launch the rest as it
        is walked, all lanes still together: the walk may then read tile
        data on the host.  Used where the cores cannot run one after another
        (they meet at a ring reduce)."""
        L = rt.lib()
        for kind, desc, _ in self.plan.launches:
            _launch(L, kind, desc)
        self.eager = True
        self.plan.ran_during_walk = True
        self.plan.replayable = False
        self.attn_pending = None
        self.mm_pending = None

    def _element(self, src: Tile, idx) -> Tile:
        """Element `idx` of every lane's `src` (per-lane host indices; a
        negative index counts from the end, as in NumPy; none: the first
        element) as a tile of shape () or (1,), in f16 for an f16 tile and
        f32 otherwise (reference dialects/tensor_ops.py:88-102)."""
        shape = tuple(src.shape)
        L = self.L
        if idx and len(idx) != len(shape):
            raise IndexError(f"tensor.extract: {len(idx)} indices for a rank-{len(shape)} tensor")
        ii = []
        for k, n in enumerate(shape):
            a = np.broadcast_to(np.asarray(idx[k] if idx else 0, dtype=np.int64), (L,))
            if np.any((a < -n) | (a >= n)):
                raise IndexError(f"tensor.extract: index out of range for dimension {k} of size {n}")
            ii.append(np.where(a < 0, a + n, a))
        ones = (1,) * len(shape)
        if shape == ones:
            t = src
        elif all(L == 0 or np.all(a == a[0]) for a in ii):
            t = Tile(self._slice_expr(src, [int(a[0]) if L else 0 for a in ii], ones, ones))
        else:
            m = src if src.e.kind == "ld" and src.e.attr.offsets is None else self.materialize(src)
            spec = m.e.attr
            delta = sum(a * int(st) for a, st in zip(ii, spec.strides))
            t = Tile(Expr("ld", m.dtype, ones, attr=spec.with_strides(spec.strides, spec.lane.add(delta))))
        if len(t.shape) > 1:
            t = self.reshape(t, (1,))
        return self._cast_tile(t, "f16" if src.dtype == "f16" else "f32")

    def _ds_broadcast(self, t: Tile, shape) -> Tile:
        """A device scalar's tile broadcast over `shape`.  A per-row fold
        value spread along the row it folded stays one fused row program
        (the 'rowval' form linalg.broadcast uses); anything else with a fold
        in it is evaluated first."""
        shape = tuple(shape)
        e = t.e
        if e.has_fold and len(shape) >= 1 and tuple(t.shape) == shape[:-1] and e._fold == shape[-1]:
            return Tile(Expr("rowval", e.dtype, shape, [e]))
        return self.broadcast_to(t, shape)

    def _scalar_operand(self, v, dt: str) -> Expr:
        """A scalar operand of a device-scalar op: a (1,)-shaped expression
        holding `v` converted to `dt`."""
        if isinstance(v, DevScalar):
            # rounded to dt; registers hold f32, so no widening cast after it
            return self.broadcast_to(self._cast_tile(v.t, dt), (1,)).e
        arr = np.broadcast_to(np.asarray(v, dtype=np.float64), (self.L,))
        return E_scalar(arr.astype(NP_DTYPE[dt]).astype(np.float64), "f32", (1,))

    def read_tile(self, t: Tile) -> np.ndarray:
        m = self.materialize(t)
        spec = m.e.attr
        n = _prod(t.shape) if t.shape else 1
        rt.sync()
        stdt = rt.STORAGE[spec.dtype]
        raw = rt.DeviceBuffer.download(_Wrap(spec.ptr), self.L * n * np.dtype(stdt).itemsize)
        arr = np.frombuffer(raw.tobytes(), dtype=stdt).copy()
        if spec.dtype == "bf16":
            arr = (arr.astype(np.uint32) << 16).view(np.float32)
        return arr.reshape((self.L,) + tuple(t.shape))

    def reshape(self, t: Tile, shape) -> Tile:
        shape = tuple(shape)
        if tuple(t.shape) == shape:
            return t
        e = t.e
        if not e.has_fold and all(n.kind != "idx" for n in topo(e)):
            try:
                def lf(spec):
                    st = _reshape_strides(spec.strides, t.shape, shape)
                    if st is None:
                        raise CompileError("reshape")
                    return spec.with_strides(st)
                return Tile(_map_leaf_idx(e, shape, lf, None))
            except CompileError:
                pass
        m = self.materialize(t)
        spec = m.e.attr
        return Tile(Expr("ld", m.dtype, shape, attr=spec.with_strides(_cstrides(shape) if shape else (1,))))

    def _h_reshape(self, op):
        src = self.get_value(op.operands[0])
        ts = op.attributes.get("target_shape")
        if ts is None:
            raise ValueError(f"{op.op_type}: missing 'target_shape' attribute")
        if not isinstance(src, Tile):
            return src
        return self.reshape(src, tuple(ts))

    h_tensor_expand_shape = _h_reshape
    h_tensor_collapse_shape = _h_reshape
    h_tensor_reshape = _h_reshape

    def h_tensor_from_elements(self, op):
        shape = tuple(op.attributes["shape"])
        dt = _canon(op.attributes["dtype"])
        cols = []
        for n in op.operands:
            v = self.get_value(n)
            if isinstance(v, Tile):
                raise NeedEager("tensor.from_elements of a tile")
            cols.append(np.asarray(v, dtype=np.float64))
        arr = np.stack(cols, axis=1).reshape((self.L,) + shape)
        if is_float(dt):
            arr = np.vectorize(lambda x: _round_val(x, dt))(arr)
        return self._host_tile(arr, dt)

    def _slice_params(self, op, first_dyn):
        a = op.attributes
        K = -(1 << 63)
        dyn = iter(op.operands[first_dyn:])

        def res(lst):
            return [int(_uniform(self.get_value(next(dyn)), "slice parameter")) if v == K else int(v) for v in lst]

        return res(a["static_offsets"]), res(a["static_sizes"]), res(a["static_strides"])

    def _slice_expr(self, src: Tile, offs, sizes, steps) -> Expr:
        shape = tuple(sizes)

        def lf(spec):
            delta = sum(o * s for o, s in zip(offs, spec.strides))
            return spec.with_strides(tuple(s * st for s, st in zip(spec.strides, steps)), spec.lane.add(delta))

        def idxf(d):
            base = Expr("idx", "i32", shape, attr=d)
            if steps[d] != 1:
                base = Expr("bin", "i32", shape, [base, E_const(steps[d], "i32", shape)], rt.op("MULI"))
            if offs[d]:
                base = Expr("bin", "i32", shape, [base, E_const(offs[d], "i32", shape)], rt.op("ADDI"))
            return base

        try:
            return _map_leaf_idx(src.e, shape, lf, idxf)
        except CompileError:
            m = self.materialize(src)
            return _map_leaf_idx(m.e, shape, lf, idxf)

    def h_tensor_extract_slice(self, op):
        src = self.get_value(op.operands[0])
        offs, sizes, steps = self._slice_params(op, 1)
        rs = tuple(op.attributes["result_shape"])
        e = self._slice_expr(src, offs, sizes, steps)
        t = Tile(e)
        return self.reshape(t, rs) if tuple(sizes) != rs else t

    def h_tensor_insert_slice(self, op):
        src = self.get_value(op.operands[0])
        dst = self.get_value(op.operands[1])
        offs, sizes, steps = self._slice_params(op, 2)
        out = self.materialize(Tile(self._cast_tile(dst, dst.dtype).e), None)
        out = Tile(out.e) if out is not dst else self._copy(dst)
        spec = out.e.attr
        delta = sum(o * s for o, s in zip(offs, spec.strides))
        sub = spec.with_strides(tuple(s * st for s, st in zip(spec.strides, steps)), spec.lane.add(delta))
        sv = self.reshape(src, tuple(sizes)) if tuple(src.shape) != tuple(sizes) else src
        e = sv.e if sv.dtype == spec.dtype else Expr("cast", spec.dtype, sv.shape, [sv.e], sv.dtype)
        self.materialize(Tile(e), dest=sub)
        return out

    def _copy(self, t: Tile) -> Tile:
        e = t.e
        wrapped = Expr("bitcast", e.dtype, e.shape, [e]) if e.kind == "ld" else e
        return self.materialize(Tile(wrapped))

    def h_tensor_generate(self, op):
        shape = tuple(op.attributes["shape"])
        dt = _canon(op.attributes["dtype"])
        region = op.regions[0]
        self.push_scope()
        for d, (n, _) in enumerate(region.args):
            self.set_value(n, Tile(Expr("idx", "i32", shape, attr=d)))
        res = self._run(region.ops)
        if isinstance(res, _Yield):
            res = res.values[0]
        self.pop_scope()
        if isinstance(res, Tile):
            return self._cast_tile(self.broadcast_to(res, shape), dt)
        return Tile(E_scalar(np.asarray(res), dt if is_float(dt) else "i32", shape))

    # ======================================================================
    # linalg (reference dialects/linalg_ops.py)
    # ======================================================================
    def broadcast_to(self, t: Tile, shape) -> Tile:
        """NumPy broadcasting of a tile to `shape`."""
        shape = tuple(shape)
        src = tuple(t.shape)
        if src == shape:
            return t
        nd = len(shape)
        pad = nd - len(src)
        if pad < 0:
            raise ValueError(f"cannot broadcast {src} to {shape}")
        full = (1,) * pad + src
        for s, d in zip(full, shape):
            if s != d and s != 1:
                raise ValueError(f"cannot broadcast {src} to {shape}")

        def lf(spec):
            st = (0,) * pad + tuple(spec.strides)
            return spec.with_strides(tuple(0 if full[i] == 1 and shape[i] != 1 else st[i] for i in range(nd)))

        def idxf(d):
            nd_ = d + pad
            if full[nd_] == 1 and shape[nd_] != 1:
                return E_const(0, "i32", shape)
            return Expr("idx", "i32", shape, attr=nd_)

        e = t.e
        if e.has_fold:
            e = self.materialize(t).e
        try:
            return Tile(_map_leaf_idx(e, shape, lf, idxf))
        except CompileError:
            return Tile(_map_leaf_idx(self.materialize(t).e, shape, lf, idxf))

    def h_linalg_broadcast(self, op):
        inp = self.get_value(op.operands[0])
        out = self.get_value(op.operands[1])
        dims = sorted(op.attributes.get("dimensions", []))
        oshape = tuple(out.shape)
        e = inp.e
        if e.has_fold and dims == [len(oshape) - 1] and tuple(inp.shape) == oshape[:-1] and e._fold == oshape[-1]:
            return Tile(Expr("rowval", e.dtype, oshape, [e]))
        if e.has_fold:
            e = self.materialize(inp).e
        keep = [d for d in range(len(oshape)) if d not in dims]

        def lf(spec):
            st = [0] * len(oshape)
            for k, d in enumerate(keep):
                st[d] = spec.strides[k]
            return spec.with_strides(tuple(st))

        def idxf(d):
            return Expr("idx", "i32", oshape, attr=keep[d])

        try:
            return Tile(_map_leaf_idx(e, oshape, lf, idxf))
        except CompileError:
            return Tile(_map_leaf_idx(self.materialize(Tile(e)).e, oshape, lf, idxf))

    def transpose(self, t: Tile, perm) -> Tile:
        perm = list(perm)
        shape = tuple(t.shape[i] for i in perm)
        inv = [perm.index(d) for d in range(len(perm))]

        def lf(spec):
            return spec.with_strides(tuple(spec.strides[p] for p in perm))

        def idxf(d):
            return Expr("idx", "i32", shape, attr=inv[d])

        e = t.e if not t.e.has_fold else self.materialize(t).e
        try:
            return Tile(_map_leaf_idx(e, shape, lf, idxf))
        except CompileError:
            return Tile(_map_leaf_idx(self.materialize(Tile(e)).e, shape, lf, idxf))

    def h_linalg_transpose(self, op):
        inp = self.get_value(op.operands[0])
        perm = op.attributes.get("permutation")
        if perm is None:
            raise ValueError("linalg.transpose: missing permutation attribute")
        return self.transpose(inp, perm)

    def h_linalg_fill(self, op):
        s = self.get_value(op.operands[0], dev=True)
        out = self.get_value(op.operands[1])
        if isinstance(s, DevScalar):
            if is_float(out.dtype) or out.dtype == "i32":
                return self._cast_tile(self._ds_broadcast(s.t, out.shape), out.dtype)
            s = self.host_scalar(s)
        vals = np.asarray(s, dtype=np.float64)
        if is_float(out.dtype):
            vals = np.array([_round_val(float(x), out.dtype) for x in vals.ravel()])
            return Tile(E_scalar(vals, out.dtype, out.shape))
        return Tile(E_scalar(vals.astype(np.int64), out.dtype, out.shape))

    def h_linalg_add(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        return Tile(Expr("bin", a.dtype, a.shape, [a.e, self.broadcast_to(b, a.shape).e],
                         rt.op("ADDF" if is_float(a.dtype) else "ADDI")))

    def h_linalg_max(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        return Tile(Expr("bin", a.dtype, a.shape, [a.e, self.broadcast_to(b, a.shape).e],
                         rt.op("MAXIMUMF" if is_float(a.dtype) else "MAXSI")))

    def _combiner(self, region: Region) -> Optional[str]:
        ops = [o for o in region.ops if o.op_type not in ("linalg.yield", "scf.yield", "tensor.yield")]
        names = [n for n, _ in region.args]
        if len(ops) == 1 and len(names) == 2 and sorted(ops[0].operands[:2]) == sorted(names[:2]):
            return ops[0].op_type
        return None

    def fold(self, t: Tile, dim: int, region: Region) -> Tile:
        """Pairwise-halving fold of `t` along `dim` (reference linalg_ops.py:86-133)."""
        comb = self._combiner(region)
        if comb is None or comb not in COMBINERS:
            return self._fold_generic(t, dim, region)
        nd = len(t.shape)
        if dim != nd - 1:
            perm = [d for d in range(nd) if d != dim] + [dim]
            t = self.transpose(t, perm)
        n = t.shape[-1]
        if nd > rt.MAX_DIMS:
            # a row space of more dims than a program has: fold a contiguous
            # (rows, n) copy, then give the rows their shape back
            lead = tuple(t.shape[:-1])
            flat = self.reshape(self.materialize(t), (_prod(lead), n))
            return self.reshape(self.fold(flat, 1, region), lead)
        if self.lat is not None:
            # the reference runs the combiner once per halving level on the
            # two halves (linalg_ops.py:114-131): charge those runs
            other, m = _prod(t.shape[:-1]), n
            while m > 1:
                half = m // 2
                for c in self.lanes.cores:
                    self.lat.record_op(int(c), comb, n_elems=other * half)
                m = half + (m % 2)
        if n > rt.MAX_ROW:
            # a row longer than the row kernels fold in LDS: the first halving
            # levels of the same pairwise fold run as elementwise programs on
            # the two halves (an odd last element carried), the rest as a row
            # program; the combiner runs are already charged above
            lat, self.lat = self.lat, None
            try:
                while n > rt.MAX_ROW:
                    half = n // 2
                    comb_t = self._combine(region, self._take_range(t, nd - 1, 0, half),
                                           self._take_range(t, nd - 1, half, 2 * half))
                    if n % 2:
                        comb_t = self._concat(comb_t, self._take_range(t, nd - 1, 2 * half, n), nd - 1)
                    t = comb_t
                    n = t.shape[-1]
            finally:
                self.lat = lat
        e = t.e
        if e.has_fold and (e._fold != n or len(_fold_space(e)) != len(t.shape)):
            e = self.materialize(t).e
        return Tile(Expr("fold", t.dtype, t.shape[:-1], [e], rt.op(COMBINERS[comb]), rowc=n))

    def _fold_generic(self, t: Tile, dim: int, region: Region) -> Tile:
        """Fold with an arbitrary combiner region: run the region on the two
        halves log2(n) times, exactly like the reference."""
        acc = t
        n = t.shape[dim]
        while n > 1:
            half = n // 2
            left = self._take_range(acc, dim, 0, half)
            right = self._take_range(acc, dim, half, 2 * half)
            comb = self._combine(region, left, right)
            if n % 2:
                tail = self._take_range(acc, dim, 2 * half, n)
                comb = self._concat(comb, tail, dim)
            acc = comb
            n = acc.shape[dim]
        return acc

    def _take_range(self, t: Tile, dim, lo, hi) -> Tile:
        offs = [0] * len(t.shape)
        offs[dim] = lo
        sizes = list(t.shape)
        sizes[dim] = hi - lo
        return Tile(self._slice_expr(self.materialize(t), offs, sizes, [1] * len(sizes)))

    def _concat(self, a: Tile, b: Tile, dim) -> Tile:
        shape = list(a.shape)
        shape[dim] += b.shape[dim]
        n = _prod(shape)
        buf = self.pool.temp(max(1, self.L * n * rt.ELEM_BYTES[_store_dt(a.dtype)]))
        cs = _cstrides(tuple(shape))
        base = LeafSpec(buf.ptr, _store_dt(a.dtype), LaneOff(0, n), cs, 0, self.L * n, keep=(buf,))
        self.materialize(a, dest=base.with_strides(cs))
        off = a.shape[dim] * cs[dim]
        self.materialize(b, dest=base.with_strides(cs, LaneOff(off, n)))
        return Tile(Expr("ld", base.dtype, tuple(shape), attr=base))

    def _combine(self, region: Region, lhs, rhs):
        self.push_scope()
        try:
            names = [n for n, _ in region.args]
            if names:
                self.set_value(names[0], lhs)
            if len(names) > 1:
                self.set_value(names[1], rhs)
            res = self._run(region.ops)
        finally:
            self.pop_scope()
        return res.values[0] if isinstance(res, _Yield) else res

    def h_linalg_reduce(self, op):
        tile = self.get_value(op.operands[0])
        region = op.regions[0]
        dims = op.attributes.get("dimensions")
        outs = op.attributes.get("outs") or []
        outs_var = outs[0] if outs else None
        outs_tile = self.get_value(outs_var) if outs_var else None
        if not isinstance(tile, Tile):
            result = tile
        else:
            if dims is None:
                flat = self.reshape(tile, (_prod(tile.shape),))
                red = self.fold(flat, 0, region)
                reduced_all = True
            else:
                red = tile
                for d in sorted(dims, reverse=True):
                    red = self.fold(red, d, region)
                reduced_all = len(red.shape) == 0
            if isinstance(outs_tile, Tile):
                o = outs_tile
                if tuple(o.shape) != tuple(red.shape):
                    if reduced_all and o.shape and _prod(o.shape) == 1:
                        # a full reduction combined with a one-element outs of
                        # rank >= 1 broadcasts to that shape: the reference
                        # then holds a tile, not a scalar
                        red = self.reshape(red, o.shape)
                        reduced_all = False
                    elif _prod(o.shape) == _prod(red.shape):
                        o = self.reshape(o, red.shape)
                red = self._combine(region, red, o)
            if reduced_all and is_float(tile.dtype):
                # the reference's Python float: the reduced value, held exactly
                result = DevScalar(self._cast_tile(red, "f16" if red.dtype == "f16" else "f32"), weak=True)
            elif reduced_all:
                if not self.eager:
                    raise NeedEager("reduction to a scalar")
                v = self.read_tile(red).reshape(self.L)
                result = v.astype(np.float16 if tile.dtype == "f16" else np.float32) if is_float(tile.dtype) \
                    else v.astype(np.int64)
            else:
                result = red
        if outs_var and result is not None:
            self.set_value(outs_var, result)
        return result

    def _mm_leaf(self, t: Tile) -> Tuple[LeafSpec, str]:
        """A leaf for a matmul operand, reading through exact f16/bf16->f32 casts."""
        e = t.e
        if e.kind == "cast" and e.dtype == "f32" and e.attr in ("f16", "bf16") and e.args[0].kind == "ld" \
                and e.args[0].attr.offsets is None:
            return e.args[0].attr, e.args[0].attr.dtype
        if e.kind == "ld" and e.attr.offsets is None:
            return e.attr, e.dtype
        m = self.materialize(t)
        return m.e.attr, m.dtype

    def _matmul(self, a: Tile, b: Tile, acc: Optional[Tile], ksteps=1, a_k=0, b_k=0, a_leaf=None, b_leaf=None,
                name=None):
        if len(a.shape) != 2 or len(b.shape) != 2:
            raise NotImplementedError("linalg.matmul on tiles of rank != 2")
        M, K = a.shape
        N = b.shape[1]
        la, dta = a_leaf or self._mm_leaf(a)
        lb, dtb = b_leaf or self._mm_leaf(b)
        res_dt = a.dtype
        out_dt = acc.dtype if acc is not None else res_dt
        L = self.L
        d = rt.MM()
        d.lanes, d.M, d.N, d.K, d.ksteps = L, M, N, K, ksteps
        keep = []
        from .program import _fill_leaf
        _fill_leaf(d.a, la.with_strides(tuple(la.strides[-2:])), L, 2, keep)
        _fill_leaf(d.b, lb.with_strides(tuple(lb.strides[-2:])), L, 2, keep)
        # the product is rounded to a's dtype (np.matmul(a, b).astype(a.dtype))
        d.a.dtype = rt.DTYPE_CODE[dta]
        d.b.dtype = rt.DTYPE_CODE[dtb]
        d.a_kstep, d.b_kstep = a_k, b_k
        # bounds / alignment of every lane's operand reads, for the MFMA path
        for leaf, spec, rows, cols, ks in ((d.a, la, M, K, a_k), (d.b, lb, K, N, b_k)):
            st0, st1 = spec.strides[-2], spec.strides[-1]
            offs = spec.lane.values(L)
            if st0 >= 0 and st1 == 1 and ks >= 0 and len(offs):
                ext = (rows - 1) * st0 + (cols - 1) + (ksteps - 1) * ks
                if offs.min() >= spec.lo and offs.max() + ext < spec.hi and np.all(offs % 8 == 0):
                    leaf.flags |= rt.K["KTIR_LEAF_CHECKED"]
        n = M * N
        buf = self.pool.temp(max(1, L * n * rt.ELEM_BYTES[_store_dt(out_dt)]))
        cspec = LeafSpec(buf.ptr, _store_dt(out_dt), LaneOff(0, n), (N, 1), 0, L * n, keep=(buf,))
        _fill_leaf(d.c, cspec, L, 2, keep)
        if acc is not None and acc.e.kind == "const" and float(acc.e.attr) == 0.0 \
                and tuple(acc.shape) == (M, N):
            d.accumulate = 2          # outs is a zero splat: C = 0.0 + A@B
        elif acc is not None:
            lc, _ = self._mm_leaf(acc) if not (acc.e.kind == "const") else (None, None)
            if lc is None:
                lc = self.materialize(acc).e.attr
            _fill_leaf(d.c0, lc.with_strides(tuple(lc.strides[-2:])), L, 2, keep)
            d.accumulate = 1
        d.round_dt = rt.DTYPE_CODE[_store_dt(res_dt)]
        quads = _mm_quads(la, lb, L, M, N) if (M, N) == (128, 128) and K % 64 == 0 else None
        if quads is not None:
            qb = self.pool.upload(quads)
            keep.append(qb)
            d.quads, d.n_quads = qb.ptr, len(quads) // 4
        keep.append(buf)
        self.launch("mm", d, keep)
        # the SSA value `name` holds this launch's result; a store of it may
        # still become the launch's own epilogue (fusion.mm_epilogue)
        reads = {id(x.alloc) for x in (la, lb) if x.alloc is not None}
        if d.accumulate == 1 and lc.alloc is not None:
            reads.add(id(lc.alloc))
        self.mm_pending = None if self.eager or name is None else dict(
            desc=d, keep=keep, buf=buf, lanes=L, level=len(self.levels), n=len(self.plan.launches), M=M, N=N,
            name=name, reads=reads)
        return Tile(Expr("ld", cspec.dtype, (M, N), attr=cspec))

    def h_linalg_matmul(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        acc = self.get_value(op.operands[2]) if len(op.operands) > 2 else None
        return self._matmul(a, b, acc if isinstance(acc, Tile) else None, name=op.results[0])

    def h_linalg_batch_matmul(self, op):
        a, b = self.get_value(op.operands[0]), self.get_value(op.operands[1])
        acc = self.get_value(op.operands[2]) if len(op.operands) > 2 else None
        if len(a.shape) != 3:
            raise NotImplementedError("batch_matmul on tiles of rank != 3")
        outs = []
        for i in range(a.shape[0]):
            ai = Tile(self._slice_expr(a, [i, 0, 0], [1] + list(a.shape[1:]), [1, 1, 1]))
            bi = Tile(self._slice_expr(b, [i, 0, 0], [1] + list(b.shape[1:]), [1, 1, 1]))
            ai, bi = self.reshape(ai, a.shape[1:]), self.reshape(bi, b.shape[1:])
            ci = None
            if isinstance(acc, Tile):
                ci = self.reshape(Tile(self._slice_expr(acc, [i, 0, 0], [1] + list(acc.shape[1:]), [1, 1, 1])),
                                  acc.shape[1:])
            outs.append(self._matmul(ai, bi, ci))
        shape = (len(outs),) + tuple(outs[0].shape)
        n = _prod(shape)
        buf = self.pool.temp(max(1, self.L * n * rt.ELEM_BYTES[_store_dt(outs[0].dtype)]))
        cs = _cstrides(shape)
        base = LeafSpec(buf.ptr, _store_dt(outs[0].dtype), LaneOff(0, n), cs, 0, self.L * n, keep=(buf,))
        per = _prod(outs[0].shape)
        for i, t in enumerate(outs):
            self.materialize(t, dest=base.with_strides(cs[1:], LaneOff(i * per, n)))
        return Tile(Expr("ld", base.dtype, shape, attr=base))

    def h_linalg_index(self, op):
        dim = op.attributes.get("dim", 0)
        shape = self._linalg_shape[-1]
        return Tile(Expr("idx", "i32", shape, attr=dim))

    def _gather_input(self, v: Tile, imap: AffineMap, target) -> Tile:
        exprs = imap.exprs
        if all(e[0] == "dim" for e in exprs):
            plain = [e[1] for e in exprs]
            srt = sorted(plain)
            t = v
            if plain != srt:
                t = self.transpose(t, [plain.index(d) for d in srt])
            src = tuple(t.shape)
            target = tuple(target)
            keep = srt

            def lf(spec):
                st = [0] * len(target)
                for k, d in enumerate(keep):
                    st[d] = spec.strides[k] if src[k] == target[d] else 0
                return spec.with_strides(tuple(st))

            def idxf(d):
                td = keep[d]
                if src[d] != target[td]:
                    return E_const(0, "i32", target)
                return Expr("idx", "i32", target, attr=td)

            e = t.e if not t.e.has_fold else self.materialize(t).e
            try:
                return Tile(_map_leaf_idx(e, target, lf, idxf))
            except CompileError:
                return Tile(_map_leaf_idx(self.materialize(Tile(e)).e, target, lf, idxf))
        # general affine map: coordinate gather from a materialised copy
        m = self.materialize(v)
        spec = m.e.attr
        pts = np.indices(target).reshape(len(target), -1)
        coords = np.stack([np.asarray(evaluate(e, list(pts)), dtype=np.int64) * np.ones(pts.shape[1], np.int64)
                           for e in exprs], axis=1)
        offs = coords @ np.asarray(spec.strides, dtype=np.int64)
        s2 = LeafSpec(spec.ptr, spec.dtype, spec.lane, _cstrides(target), spec.lo, spec.hi, keep=spec.keep)
        s2.offsets, s2.offsets_ls = self.pool.upload(offs), 0
        return Tile(Expr("ld", spec.dtype, tuple(target), attr=s2))

    def h_linalg_generic(self, op):
        """Reference dialects/linalg_ops.py:467-585."""
        n_ins = op.attributes.get("n_ins", 0)
        maps = op.attributes.get("indexing_maps", [])
        it = op.attributes.get("iterator_types")
        ins = [self.get_value(op.operands[i]) for i in range(n_ins)]
        outs_val = self.get_value(op.operands[n_ins])
        region = op.regions[0]
        names = [n for n, _ in region.args]
        body = region.ops
        if not isinstance(outs_val, Tile):
            raise TypeError("linalg.generic: outs must be a Tile")
        out_shape = tuple(outs_val.shape)
        red = [i for i, t in enumerate(it or []) if t == "reduction"]
        if not red:
            iter_shape = out_shape
        else:
            shapes = [v.shape for v in ins if isinstance(v, Tile)] + [out_shape]
            ext = [None] * maps[0].n_dims
            for m, s in zip(maps[:len(shapes)], shapes):
                for k, e in enumerate(m.exprs):
                    if e[0] == "dim" and ext[e[1]] is None:
                        ext[e[1]] = s[k]
            if any(e is None for e in ext):
                raise ValueError("linalg.generic: cannot infer iteration extents")
            iter_shape = tuple(ext)
        self.push_scope()
        self._linalg_shape.append(iter_shape)
        try:
            for i, (v, m) in enumerate(zip(ins, maps[:n_ins])):
                arg = self._gather_input(v, m, iter_shape) if isinstance(v, Tile) else v
                if i < len(names):
                    self.set_value(names[i], arg)
            if not red:
                if n_ins < len(names):
                    self.set_value(names[n_ins], outs_val)
                res = self._run(body)
                od = _unwrap(res)
            else:
                outs_name = names[n_ins] if n_ins < len(names) else None
                y = next((o for o in body if o.op_type == "linalg.yield"), None)
                comb = None
                if y is not None:
                    yn = y.operands[0] if y.operands else None
                    comb = next((o for o in body if o.result == yn and outs_name in o.operands), None)
                if comb is None:
                    raise ValueError("linalg.generic: cannot identify combiner op for reduction")
                if comb.op_type not in COMBINER_IDENTITY:
                    raise ValueError(f"linalg.generic: unsupported combiner '{comb.op_type}' for reduction")
                if n_ins < len(names):
                    ident = COMBINER_IDENTITY[comb.op_type]
                    self.set_value(names[n_ins], Tile(E_const(_round_val(ident, outs_val.dtype), outs_val.dtype,
                                                             iter_shape)))
                res = self._run(body)
                od = _unwrap(res)
        finally:
            self._linalg_shape.pop()
            self.pop_scope()
        if not red:
            if isinstance(od, Tile):
                od = self.broadcast_to(od, out_shape)
                return self._cast_tile(od, outs_val.dtype) if od.dtype != outs_val.dtype else od
            return Tile(E_scalar(np.asarray(od), outs_val.dtype if is_float(outs_val.dtype) else "i32", out_shape))
        if not isinstance(od, Tile):
            od = Tile(E_scalar(np.asarray(od), outs_val.dtype, iter_shape))
        cregion = Region([("%__fold_lhs__", None), ("%__fold_rhs__", None)], [
            Operation(comb.op_type, ["%__fold_combined__"], ["%__fold_lhs__", "%__fold_rhs__"],
                      dict(comb.attributes), list(comb.result_types)),
            Operation("linalg.yield", [], ["%__fold_combined__"])])
        folded = od
        for d in sorted(red, reverse=True):
            folded = self.fold(folded, d, cregion)
        c = self._combine(cregion, folded, outs_val if tuple(outs_val.shape) == tuple(folded.shape)
                          else self.reshape(outs_val, folded.shape))
        c = c if c.dtype == outs_val.dtype else self._cast_tile(c, outs_val.dtype)
        return self.reshape(c, out_shape) if tuple(c.shape) != out_shape else c

    def h_linalg_yield(self, op):
        return _Yield([self.get_value(n) for n in op.operands])

    h_scf_yield = h_linalg_yield
    h_tensor_yield = h_linalg_yield

    # ======================================================================
    # inter-tile communication (reference dialects/ktdp_ops.py:951-1230,
    # ops/comm_ops.py:229-345)
    # ======================================================================
    def h_ktdp_inter_tile_produce(self, op):
        """Each lane's group g (the one group whose producer set holds its
        core, dialects/ktdp_ops.py:917-944), the producer region run with
        %gid = g, its yielded partial(s) kept on a future."""
        P = op.attributes["producer_tiles_per_group"]
        G = op.attributes["groups"]
        n = self.n_cores
        keys = [g for g in range(n) if G.contains([g])]
        gid = np.empty(self.L, dtype=np.int64)
        for c in np.unique(self.lanes.cores):
            hits = [g for g in keys if P.contains([int(c)], [g])]
            if not hits:
                raise RuntimeError(f"tile {int(c)} is not contained in any producer group")
            if len(hits) > 1:
                raise RuntimeError(f"tile {int(c)} matched multiple groups {hits} — violates the disjointness "
                                   f"invariant")
            gid[self.lanes.cores == c] = hits[0]
        region = op.regions[0] if op.regions else None
        if region is not None and region.args:
            self.set_value(region.args[0][0], gid)
        y = self._run(region.ops) if region is not None else None
        vals = y.values if isinstance(y, _Yield) else ([y] if y is not None else None)
        return _Future(tuple(vals) if vals else None, gid, P, G)

    def h_ktdp_yield_partial(self, op):
        return _Yield([self.get_value(n) for n in op.operands])

    h_ktdp_yield_reduced = h_ktdp_yield_partial

    def h_ktdp_inter_tile_reduce(self, op):
        """The ring reduce of every core at once: lane c starts from its own
        partial and, for k = 1 .. n-1, folds in the partial of core
        (c - k) mod n as combine(acc, partial) when that core produces for
        c's group -- the fold order of the reference's ring, where round k
        delivers that core's seed.  Cores outside the consumer set get the
        value too (the reference leaves it unbound; a valid function does
        not read it there)."""
        fut = self.get_value(op.operands[0])
        if not isinstance(fut, _Future):
            raise TypeError(f"ktdp.inter_tile_reduce: operand 0 must be a TileFuture, got {type(fut)}")
        for name in op.operands[1:]:
            self.get_value(name)
        if self.sequential:
            raise NotImplementedError("ktdp.inter_tile_reduce: the cores of this function cannot run in lockstep "
                                      "(it reads tile data on the host or has a cross-core memory dependence)")
        n, L = self.n_cores, self.L
        cores = self.lanes.cores.astype(np.int64)
        if L != n or not np.array_equal(np.sort(cores), np.arange(n)):
            raise NotImplementedError("ktdp.inter_tile_reduce reached by other than one lane per core")
        why = verify(self.accesses, self.insts)
        if why is not None:
            raise NotImplementedError(f"cross-core dependence through memory before ktdp.inter_tile_reduce: {why}")
        self.accesses.clear()
        self.had_reduce = True
        region = op.regions[0] if op.regions else None
        if region is None or len(region.args) < 2:
            raise ValueError("ktdp.inter_tile_reduce: combiner region needs >=2 block args (lhs, rhs)")
        lhs, rhs = region.args[0][0], region.args[1][0]
        if not fut.partials or not isinstance(fut.partials[0], Tile):
            raise NotImplementedError("ktdp.inter_tile_reduce of a non-tile partial")
        P = fut.producer_set
        prod = {int(g): np.array([P.contains([i], [int(g)]) for i in range(n)]) for g in np.unique(fut.gid)}
        pm = np.stack([prod[int(g)] for g in fut.gid])                     # lane x core
        lane_of = np.empty(n, dtype=np.int64)
        lane_of[cores] = np.arange(L)
        seed = self.materialize(fut.partials[0])
        acc = seed
        for k in range(1, n):
            origin = (cores - k) % n
            fold = pm[np.arange(L), origin]
            if not fold.any():
                continue
            got = Tile(remap_lanes(seed.e, lane_of[origin]))
            self.push_scope()
            self._lat_mask = fold          # the combiner runs on the cores that fold at this round
            try:
                self.set_value(lhs, acc)
                self.set_value(rhs, got)
                r = _unwrap(self._run(region.ops))
            finally:
                self._lat_mask = None
                self.pop_scope()
            if not isinstance(r, Tile):
                raise TypeError(f"ktdp.inter_tile_reduce: combiner did not yield a Tile, got {type(r)}")
            if not fold.all():
                ea = acc.e if tuple(acc.shape) == tuple(r.shape) else self._operand(acc, r.dtype, r.shape, False)
                r = Tile(Expr("sel", r.dtype, r.shape, [E_scalar(fold.astype(np.int64), "i32", r.shape), r.e, ea]))
            acc = self.materialize(r)
        if self.lat is not None:
            # every core sends its seed n - 1 times (ops/comm_ops.py:229-345);
            # the reference's latency tracker needs a result on every core
            # (latency.py:533-558), so a non-consumer is an error there
            C = op.attributes["consumer_tiles_per_group"]
            for c, g in zip(cores, fut.gid):
                if not C.contains([int(c)], [int(g)]):
                    raise RuntimeError("_comm_size: comm op result must be a Tile, got NoneType")
            self._lat_comm = (n - 1) * _prod(seed.shape) * rt.ELEM_BYTES[seed.dtype]
        rs = op.attributes.get("_result_shape")
        if rs is not None and tuple(rs) != tuple(acc.shape):
            acc = self.reshape(acc, tuple(rs))
        return acc

    # ======================================================================
    # scf (reference dialects/scf_ops.py, ops/control_ops.py)
    # ======================================================================
    def h_scf_if(self, op):
        c = self.get_value(op.operands[0])
        if isinstance(c, Tile):
            raise NeedEager("scf.if on a tile value")
        c = np.broadcast_to(np.asarray(c).astype(bool), (self.L,))
        regions = op.regions
        if c.size and np.any(c != c.flat[0]) and not op.results:
            # lanes split: each branch runs on the lanes that take it
            for region, sel in ((regions[0], c), (regions[1] if len(regions) > 1 else None, ~c)):
                if region is None or not region.ops or not sel.any():
                    continue
                active = np.flatnonzero(sel)
                cur = self.lanes
                self.levels.append(_Level(Lanes(cur.cores[active], cur.inst[active]), active))
                self.push_scope()
                try:
                    self._run(region.ops)
                finally:
                    self.pop_scope()
                    self.levels.pop()
            return None
        cu = bool(_uniform(c, "scf.if condition"))
        region = regions[0] if cu else (regions[1] if len(regions) > 1 else None)
        if region is None or not region.ops:
            return None
        self.push_scope()
        res = self._run(region.ops)
        self.pop_scope()
        out = _unwrap(res)
        return self._own(out)

    def _own(self, v):
        if isinstance(v, tuple):
            return tuple(self._own(x) for x in v)
        return v

    def h_return(self, op):
        return self.get_value(op.operands[0]) if op.operands else None

    h_func_return = h_return

    def h_scf_for(self, op):
        lb = np.asarray(self.get_value(op.operands[0]), dtype=np.int64)
        ub = np.asarray(self.get_value(op.operands[1]), dtype=np.int64)
        st = np.maximum(np.asarray(self.get_value(op.operands[2]), dtype=np.int64), 1)
        L = self.L
        lb, ub, st = (np.broadcast_to(x, (L,)).copy() for x in (lb, ub, st))
        trips = np.maximum(0, (ub - lb + st - 1) // st)
        iv = op.attributes["iter_var"]
        names = op.attributes.get("iter_args", [])
        body = op.regions[0].ops
        inits = [self.get_value(n, peek=True) for n in op.operands[3:]]
        from .fusion import try_fuse_loop
        # the latency model charges the loop body op by op: no fused loop launches
        fused = try_fuse_loop(self, op, lb, st, trips, inits) if self.lat is None else None
        if fused is not None:
            res = fused
        elif not names and self.allow_expand and _expandable(body) and L > 0:
            self._expand(op, lb, st, trips)
            return None
        else:
            res = self._iterate(op, lb, st, trips, inits)
        if not names:
            return None
        for n, v in zip(names, res):
            self.set_value(n, v)
        return res[0] if len(res) == 1 else tuple(res)

    def _expand(self, op, lb, st, trips):
        """Run independent iterations as extra lanes (one lane per (lane,
        iteration)).  Lanes go lane-major (a lane's iterations side by side)
        unless the iteration values are then not affine in the lane and
        iteration-major order makes them so: a loop that strides its lanes'
        rows (row = core + j * cores) then addresses memory with one stride per
        lane instead of an offset table."""
        L = self.L
        tot = int(trips.sum())
        if tot == 0:
            return
        parent = np.repeat(np.arange(L, dtype=np.int64), trips)
        first = np.repeat(np.cumsum(trips) - trips, trips)
        j = np.arange(tot, dtype=np.int64) - first
        ivals = lb[parent] + j * st[parent]
        if L > 1 and np.all(trips == trips[0]) and not _affine(ivals):
            T = int(trips[0])
            p2 = np.tile(np.arange(L, dtype=np.int64), T)
            j2 = np.repeat(np.arange(T, dtype=np.int64), L)
            iv2 = lb[p2] + j2 * st[p2]
            if _affine(iv2):
                parent, j, ivals = p2, j2, iv2
        cur = self.lanes
        new = Lanes(cur.cores[parent], self.insts.new(cur.inst[parent]))
        self.levels.append(_Level(new, parent))
        self.push_scope()
        try:
            self.set_value(op.attributes["iter_var"], ivals)
            self._run(op.regions[0].ops)
        finally:
            self.pop_scope()
            self.levels.pop()

    def _iterate(self, op, lb, st, trips, inits):
        names = op.attributes.get("iter_args", [])
        iv = op.attributes["iter_var"]
        body = op.regions[0].ops
        L = self.L
        carries = [self._carry_init(v) for v in inits]
        for n, v in zip(names, inits):
            self.set_value(n, v)
        maxt = int(trips.max()) if L else 0
        for j in range(maxt):
            active = np.flatnonzero(trips > j)
            sub = len(active) != L
            if sub:
                cur = self.lanes
                self.levels.append(_Level(Lanes(cur.cores[active], cur.inst[active]), active))
            self.push_scope()
            try:
                self.set_value(iv, lb[active] + j * st[active])
                if names:
                    for n, c in zip(names, carries):
                        self.set_value(n, self._carry_get(c, active, j))
                res = self._run(body)
                if names:
                    if not isinstance(res, _Yield) or len(res.values) != len(names):
                        raise RuntimeError("scf.for: yield does not match iter_args")
                    for c, v in zip(carries, res.values):
                        self._carry_put(c, v, active, j)
            finally:
                self.pop_scope()
                if sub:
                    self.levels.pop()
        return [self._carry_final(c, trips) for c in carries]

    # loop-carried values: scalars are per-lane vectors; tiles live in a
    # two-slot device buffer per lane (slot j%2 holds iteration j's yield)
    def _carry_init(self, v):
        if isinstance(v, Tile):
            shape, dt = tuple(v.shape), _store_dt(v.dtype)
            n = _prod(shape) if shape else 1
            L = self.L
            buf = self.pool.temp(max(1, 2 * L * n * rt.ELEM_BYTES[dt]))
            cs = _cstrides(shape) if shape else (1,)
            spec = LeafSpec(buf.ptr, dt, LaneOff(0, n), cs, 0, 2 * L * n, keep=(buf,))
            # the initial value goes to slot 1, so iteration 0 writes slot 0
            self.materialize(self._cast_tile(v, dt) if v.dtype != dt else v,
                             dest=spec.with_strides(cs, LaneOff(L * n, n)))
            return {"kind": "tile", "spec": spec, "n": n, "shape": shape, "dt": dt, "L": L}
        return {"kind": "scalar", "val": np.array(v, copy=True)}

    def _carry_get(self, c, active, j):
        if c["kind"] == "scalar":
            return c["val"][active]
        slot = (j + 1) % 2
        spec, n, L = c["spec"], c["n"], c["L"]
        lane = LaneOff.from_array((slot * L + active) * n)
        return Tile(Expr("ld", c["dt"], c["shape"], attr=spec.with_strides(spec.strides, lane)))

    def _carry_put(self, c, v, active, j):
        if c["kind"] == "scalar":
            c["val"][active] = np.asarray(v)
            return
        if not isinstance(v, Tile):
            v = Tile(E_scalar(np.asarray(v), c["dt"], c["shape"]))
        if tuple(v.shape) != c["shape"]:
            v = self.broadcast_to(v, c["shape"])
        slot = j % 2
        spec, n, L = c["spec"], c["n"], c["L"]
        lane = LaneOff.from_array((slot * L + active) * n)
        v = self._cast_tile(v, c["dt"]) if v.dtype != c["dt"] else v
        self.materialize(v, dest=spec.with_strides(spec.strides, lane))

    def _carry_final(self, c, trips):
        if c["kind"] == "scalar":
            return c["val"]
        spec, n, L = c["spec"], c["n"], c["L"]
        slot = (trips + 1) % 2
        lane = LaneOff.from_array((slot * L + np.arange(L)) * n)
        return Tile(Expr("ld", c["dt"], c["shape"], attr=spec.with_strides(spec.strides, lane)))


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

class _Wrap:
    def __init__(self, ptr):
        self.ptr = ptr


def _affine(a: np.ndarray) -> bool:
    """Whether the values step by one constant difference."""
    if a.size < 3:
        return True
    d = np.diff(a)
    return bool(np.all(d == d[0]))


def _prod(s) -> int:
    n = 1
    for x in s:
        n *= int(x)
    return n


def _cstrides(shape) -> Tuple[int, ...]:
    st, acc = [], 1
    for s in reversed(tuple(shape)):
        st.append(acc)
        acc *= int(s)
    return tuple(reversed(st)) if st else (1,)


def _contiguous(strides, shape) -> bool:
    return tuple(strides) == _cstrides(shape)


def _store_dt(dt: str) -> str:
    return "i32" if dt == "index" else dt


def _round_val(v, dt):
    if is_float(dt):
        return round_host(float(v), dt)
    return int(v)


def _bshape(a, b):
    shapes = [x.shape for x in (a, b) if isinstance(x, Tile)]
    return tuple(np.broadcast_shapes(*shapes))


def _res_float_dt(a, b) -> str:
    ta = a.dtype if isinstance(a, Tile) else None
    tb = b.dtype if isinstance(b, Tile) else None
    if ta is None:
        return tb
    if tb is None or ta == tb:
        return ta
    if ta == "bf16":
        return "bf16"
    if "f32" in (ta, tb) or "bf16" in (ta, tb):
        return "f32"
    return ta


def _fold_space(e: Expr) -> Tuple[int, ...]:
    for n in topo(e):
        if n.kind == "fold":
            return tuple(n.args[0].shape)
    return ()


def _reads(e: Expr, alloc: Alloc) -> bool:
    for n in topo(e):
        if n.kind == "ld" and n.attr.alloc is alloc:
            return True
    return False


def _same_access(e: Expr, dest: LeafSpec, alloc: Alloc) -> bool:
    """True if every leaf of `e` reading `alloc` reads exactly the element the
    store writes at the same position (an in-place elementwise update)."""
    for n in topo(e):
        if n.kind == "ld" and n.attr.alloc is alloc:
            s = n.attr
            if s.offsets is not None or dest.offsets is not None:
                return False
            if s.strides != dest.strides or s.lane.base != dest.lane.base or s.lane.stride != dest.lane.stride:
                return False
            if (s.lane.arr is None) != (dest.lane.arr is None):
                return False
            if s.lane.arr is not None and not np.array_equal(s.lane.arr, dest.lane.arr):
                return False
    return True


def _replace(e: Expr, old: Expr, new: Expr, memo=None) -> Expr:
    if memo is None:
        memo = {}
    if e is old:
        return new
    k = id(e)
    if k in memo:
        return memo[k]
    if not e.args:
        return e
    args = [_replace(a, old, new, memo) for a in e.args]
    r = e if all(x is y for x, y in zip(args, e.args)) else Expr(e.kind, e.dtype, e.shape, args, e.attr, e.rowc)
    memo[k] = r
    return r


def _reshape_strides(strides, old, new) -> Optional[Tuple[int, ...]]:
    """Strides of a row-major reshape of a strided view, if expressible
    without a copy (NumPy's rule): the non-unit dims of both shapes split
    into consecutive groups of equal size; a group of old dims must be one
    contiguous run (each stride the next one times its size), and is then
    split into its group of new dims, whatever its stride (a broadcast dim,
    stride 0, splits into stride-0 dims).  Size-1 dims get stride 0."""
    od = [(int(s), int(t)) for s, t in zip(old, strides) if int(s) != 1]
    nd = [int(n) for n in new]
    nn = [n for n in nd if n != 1]
    if [s for s, _ in od] == nn:
        it = iter(t for _, t in od)
        return tuple(0 if n == 1 else next(it) for n in nd)
    if any(s == 0 for s, _ in od) or 0 in nn:
        return None
    out: List[int] = []
    i = j = 0
    while i < len(od) and j < len(nn):
        i2, j2, pi, pj = i + 1, j + 1, od[i][0], nn[j]
        while pi != pj:
            if pi < pj:
                if i2 >= len(od):
                    return None
                pi *= od[i2][0]
                i2 += 1
            else:
                if j2 >= len(nn):
                    return None
                pj *= nn[j2]
                j2 += 1
        for k in range(i, i2 - 1):
            if od[k][1] != od[k + 1][1] * od[k + 1][0]:
                return None
        acc, grp = od[i2 - 1][1], []
        for k in range(j2 - 1, j - 1, -1):
            grp.append(acc)
            acc *= nn[k]
        out.extend(reversed(grp))
        i, j = i2, j2
    if i != len(od) or j != len(nn):
        return None
    it = iter(out)
    return tuple(0 if n == 1 else next(it) for n in nd)


def _use_counts(ops) -> Dict[str, int]:
    counts: Dict[str, int] = {}
    for op in ops:
        for n in op.operands:
            counts[n] = counts.get(n, 0) + 1
        for r in op.regions:
            for n, c in _use_counts(r.ops).items():
                counts[n] = counts.get(n, 0) + c
    return counts


def _has_op(ops, name: str) -> bool:
    return any(op.op_type == name or any(_has_op(r.ops, name) for r in op.regions) for op in ops)


def _expandable(ops) -> bool:
    """Iterations can run as lanes: no indirect stores, no ops whose result
    depends on another iteration.  (A host read of tile data inside, such as
    an index_cast of a tile element, raises NeedEager while the lanes are
    walked, as it would without the expansion.)"""
    for op in ops:
        if op.op_type in ("ktdp.construct_indirect_access_tile", "ktdp.inter_tile_produce",
                          "ktdp.inter_tile_reduce"):
            return False
        for r in op.regions:
            if not _expandable(r.ops):
                return False
    return True
