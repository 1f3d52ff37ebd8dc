"""SPMD lockstep executor: runs a parsed KTIR function on the GPU.

Reference execution model (``interpreter.py:122-194``, ``grid.py:524-623``):
every simulated core runs the whole function body, one core after another in
core-id order, and every tile op is a NumPy call.

Here the host walks the IR once for a *lane set* (``Lanes``): all simulated
cores at once, plus, for ``scf.for`` loops whose iterations are independent,
every (core, iteration) pair side by side.  Scalars (addresses, loop bounds,
offsets) are per-lane NumPy vectors on the host, i.e. launch parameters; every
tile value lives on the GPU as a lazy expression (``program.Expr``) that is
evaluated by one fused kernel at the point it has to exist in memory.

Reordering work across lanes is only valid when lanes do not communicate
through HBM.  The walk therefore *records* launches and HBM accesses first;
``verify`` checks that no two lanes that the reference orders differently
touch the same bytes with a store involved.  If they might, or if the
function needs device data to continue the walk (an integer read from a
tile by ``tensor.extract``, or a scalar read from a tile and then used as
an address, a bound or a condition), the executor falls back to running one
core at a time, in core-id order, still entirely on the GPU, which is the
reference's order by construction.
"""

from __future__ import annotations

import bisect
import weakref
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import runtime as rt
from .program import (CompileError, Expr, LaneOff, LeafSpec, compile_program, is_float, round_host, topo)

STICK_BYTES = 128
HBM_BASE = 0x10000


class NeedEager(Exception):
    """The walk needs device data (or a per-core hazard) -> sequential mode."""


# ---------------------------------------------------------------------------
# arena: the reference's simulated HBM (memory.py:311-398) on the device
# ---------------------------------------------------------------------------

@dataclass
class Alloc:
    name: str
    dtype: str
    addr: int          # reference byte address (stick-aligned, from 0x10000)
    nbytes: int
    shape: Tuple[int, ...]
    off: int = 0       # byte offset inside the device arena (or inside `buf`)
    buf: Any = None    # a device buffer of its own (the LX space), else the arena's

    @property
    def n_elems(self) -> int:
        return self.nbytes // rt.ELEM_BYTES[self.dtype]


# an arena spanning more bytes than this is refused (sparse seeded addresses)
MAX_ARENA_SPAN = 1 << 37


class Arena:
    """Allocations at the byte addresses the reference's HBM simulator gives
    them, in one device buffer that spans them: the byte address of every
    element matches the reference."""

    def __init__(self):
        self.allocs: List[Alloc] = []
        self.buf: Optional[rt.DeviceBuffer] = None
        self._starts: List[int] = []
        self.base = HBM_BASE

    def layout(self, specs: List[Tuple[str, str, int, int, Tuple[int, ...]]]):
        """`specs`: (name, dtype, byte address, nbytes, shape) per allocation;
        allocations must not overlap."""
        order = sorted(specs, key=lambda t: t[2])
        for (n0, _, a0, b0, _), (n1, _, a1, _, _) in zip(order, order[1:]):
            if a0 + b0 > a1:
                raise NotImplementedError(f"HBM allocations {n0!r} and {n1!r} overlap "
                                          f"(0x{a0:x}+{b0} > 0x{a1:x})")
        self.base = min([HBM_BASE] + [t[2] & ~(STICK_BYTES - 1) for t in order])
        end = max([HBM_BASE + STICK_BYTES] + [t[2] + max(t[3], 1) for t in order])
        if end - self.base > MAX_ARENA_SPAN:
            raise NotImplementedError(f"HBM allocations span {end - self.base} bytes")
        self.allocs = [Alloc(name, dt, addr, nbytes, shape, addr - self.base) for name, dt, addr, nbytes, shape in order]
        total = (end - self.base + STICK_BYTES - 1) & ~(STICK_BYTES - 1)
        if self.buf is None or self.buf.nbytes < total:
            if self.buf is not None:
                self.buf.free()
            self.buf = rt.DeviceBuffer(total)
        self._starts = [a.addr for a in self.allocs]

    def find(self, addr: int) -> Alloc:
        i = bisect.bisect_right(self._starts, addr) - 1
        if i >= 0:
            a = self.allocs[i]
            if a.addr <= addr < a.addr + max(a.nbytes, 1):
                return a
        raise ValueError(f"Read from unmapped address 0x{int(addr):x}")

    def ptr_of(self, a: Alloc) -> int:
        return (a.buf if a.buf is not None else self.buf).ptr + a.off


class LXSpace:
    """Every core's LX scratchpad (reference ``memory.py:400-446``) in one
    device buffer: core c's byte b lives at ``c * bytes_per_core + b``.

    Reads and writes address LX as a flat per-core byte array: bytes never
    written read zero, and an access that leaves ``[0, bytes_per_core)``
    is refused by the walker.  One allocation record (byte-sized elements)
    stands for the whole space, so the hazard check sees two lanes that
    touch the same core's bytes, whatever their dtypes."""

    def __init__(self, n_cores: int, bytes_per_core: int):
        self.n_cores = int(n_cores)
        self.bytes_per_core = int(bytes_per_core)
        total = self.n_cores * self.bytes_per_core
        self.buf = rt.DeviceBuffer(total)
        self.alloc = Alloc("__lx__", "i8", -1, total, (total,), 0, self.buf)
        self.seeds: List[Tuple[int, int, np.ndarray]] = []

    def seed(self, seeds: List[Tuple[int, int, np.ndarray]]):
        """(core, byte address, data) written before the run; zero elsewhere."""
        for core, addr, data in seeds:
            raw = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
            if not (0 <= core < self.n_cores) or addr < 0 or addr + raw.size > self.bytes_per_core:
                raise NotImplementedError(f"LX seed of {raw.size} bytes at 0x{addr:x} on core {core} lies outside "
                                          f"the {self.bytes_per_core}-byte scratchpad")
        self.seeds = list(seeds)
        self.reset()

    def reset(self):
        self.buf.memset(0)
        for core, addr, data in self.seeds:
            raw = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
            self.buf.upload(raw, core * self.bytes_per_core + addr)

    def free(self):
        self.buf.free()


# ---------------------------------------------------------------------------
# device memory for temporaries
# ---------------------------------------------------------------------------

class TempBuf:
    """A pooled device buffer that returns to its pool when unreferenced.

    All work runs in order on one stream, so a buffer released by the host may
    be handed to any later launch, recorded or not."""

    __slots__ = ("buf", "pool", "__weakref__")

    def __init__(self, pool: "Pool", nbytes: int):
        self.pool = pool
        self.buf = pool._take(nbytes)

    @property
    def ptr(self):
        return self.buf.ptr

    def __del__(self):
        try:
            self.pool._give(self.buf)
        except Exception:
            pass


class Pool:
    def __init__(self):
        self._free: Dict[int, List[rt.DeviceBuffer]] = {}
        self.owned: List[rt.DeviceBuffer] = []
        self.uploads: Dict[Tuple, rt.DeviceBuffer] = {}

    @staticmethod
    def _bucket(n: int) -> int:
        n = max(int(n), 256)
        if n <= (1 << 20):
            return 1 << (n - 1).bit_length()
        return ((n + (1 << 20) - 1) >> 20) << 20

    def _take(self, nbytes: int) -> rt.DeviceBuffer:
        b = self._bucket(nbytes)
        lst = self._free.get(b)
        if lst:
            return lst.pop()
        d = rt.DeviceBuffer(b)
        self.owned.append(d)
        return d

    def _give(self, d: rt.DeviceBuffer):
        self._free.setdefault(d.nbytes, []).append(d)

    def temp(self, nbytes: int) -> TempBuf:
        return TempBuf(self, nbytes)

    def upload(self, arr: np.ndarray) -> rt.DeviceBuffer:
        """Immutable device copy of host data, kept for the life of the pool
        (recorded launches may read it later); identical contents are shared."""
        a = np.ascontiguousarray(arr)
        key = (a.dtype.str, a.shape, hash(a.tobytes()))
        d = self.uploads.get(key)
        if d is None:
            d = rt.DeviceBuffer(a.nbytes)
            d.upload(a)
            self.uploads[key] = d
        return d

    def free_all(self):
        for d in self.owned:
            d.free()
        for d in self.uploads.values():
            d.free()
        self.owned.clear()
        self.uploads.clear()
        self._free.clear()


# ---------------------------------------------------------------------------
# values
# ---------------------------------------------------------------------------

@dataclass
class View:
    """ktdp.construct_memory_view (reference ir_types.py:52-123)."""
    base: np.ndarray            # per-lane element index of the view origin (pointer value)
    shape: Tuple[int, ...]
    strides: Tuple[int, ...]
    dtype: str
    space: str
    cs: Any = None
    core: Optional[np.ndarray] = None   # LX views: per-lane core whose scratchpad is addressed

    def take(self, idx):
        return View(self.base[idx], self.shape, self.strides, self.dtype, self.space, self.cs,
                    None if self.core is None else self.core[idx])


@dataclass
class DistView:
    """ktdp.construct_distributed_memory_view (reference ir_types.py:126-316):
    partition views, each with a box coordinate set in global coordinates."""
    parts: List[View]
    shape: Tuple[int, ...]
    dtype: str

    def take(self, idx):
        return DistView([p.take(idx) for p in self.parts], self.shape, self.dtype)


@dataclass
class DistATile:
    """An access tile over a distributed view: per-lane global origin `x`
    (one array per dimension) and the access tile set."""
    dist: DistView
    x: Tuple[np.ndarray, ...]
    shape: Tuple[int, ...]
    cs: Any

    def take(self, idx):
        return DistATile(self.dist.take(idx), tuple(v[idx] for v in self.x), self.shape, self.cs)


@dataclass
class ATile:
    """ktdp.construct_access_tile (reference ir_types.py:444-461)."""
    view: View
    origin: np.ndarray          # per-lane element offset of the tile origin from the view origin
    shape: Tuple[int, ...]
    cs: Any
    co: Any

    def take(self, idx):
        return ATile(self.view.take(idx), self.origin[idx], self.shape, self.cs, self.co)


@dataclass
class IATile:
    """ktdp.construct_indirect_access_tile (reference ir_types.py:464-477)."""
    parent: View
    shape: Tuple[int, ...]
    subs: List[Dict]
    views: List[View]
    vss: Any
    vso: Any
    ssa: Dict[str, np.ndarray]  # per-lane values of outer SSA names in the subscripts

    def take(self, idx):
        ssa = {k: ({i: a[idx] for i, a in v.items()} if isinstance(v, dict) else v[idx])
               for k, v in self.ssa.items()}
        return IATile(self.parent.take(idx), self.shape, self.subs, [v.take(idx) for v in self.views],
                      self.vss, self.vso, ssa)


class Tile:
    """A per-lane tile value: a lazy expression over the tile shape."""

    __slots__ = ("e", "__weakref__")

    def __init__(self, e: Expr):
        self.e = e

    @property
    def dtype(self):
        return self.e.dtype

    @property
    def shape(self):
        return self.e.shape

    def nbytes(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n * rt.ELEM_BYTES.get(self.dtype, 4)


class DevScalar:
    """A per-lane float scalar that stays on the device: the one element of
    `t`, a tile of shape () or (1,), read from tile data by tensor.extract
    or a reduction over every axis (reference dialects/tensor_ops.py:88-102,
    dialects/linalg_ops.py:197-240).  tensor.extract gives the reference a
    NumPy scalar of the tile's type: `t.dtype` is that type ("f16" or "f32";
    a bf16 element is held as f32), which decides how later scalar ops
    round.  A reduction over every axis gives it a Python float (`weak`):
    `t` holds its value exactly, and ops that would compute on it in
    float64 read it on the host.  Host code that needs the value reads it
    (Executor.get_value)."""

    __slots__ = ("t", "weak")

    def __init__(self, t: Tile, weak: bool = False):
        self.t = t
        self.weak = weak

    @property
    def dtype(self):
        return self.t.dtype


@dataclass
class Lanes:
    cores: np.ndarray           # simulated core id of every lane
    inst: np.ndarray            # instance id (core or (core, iteration ...)) of every lane

    @property
    def n(self) -> int:
        return len(self.cores)


# ---------------------------------------------------------------------------
# HBM access log + cross-lane hazard check
# ---------------------------------------------------------------------------

@dataclass
class Access:
    alloc: Alloc
    store: bool
    inst: np.ndarray
    base: np.ndarray            # per-lane element offset (relative to the allocation) of the tile origin
    shape: Tuple[int, ...]
    strides: Tuple[int, ...]
    whole: bool = False         # data-dependent addresses: the whole allocation
    group: Optional[int] = None # accesses of one fused launch that orders its lanes itself


class Instances:
    """Parent links of lane instances: core instances are roots, an expanded
    loop iteration's instance is a child of the lane it was expanded from."""

    def __init__(self, n_cores: int):
        self.parent: List[int] = [-1] * n_cores

    def new(self, parents: np.ndarray) -> np.ndarray:
        start = len(self.parent)
        self.parent.extend(int(p) for p in parents)
        return np.arange(start, start + len(parents), dtype=np.int64)

    def chain(self, i: int) -> List[int]:
        out = []
        while i >= 0:
            out.append(i)
            i = self.parent[i]
        return out

    def comparable(self, a: int, b: int) -> bool:
        return a in self.chain(b) or b in self.chain(a)


def _decompose(base: np.ndarray, shape, strides) -> Optional[np.ndarray]:
    """Coordinates of `base` in a row-major nest of `strides`, or None."""
    st = list(strides)
    order = sorted(range(len(st)), key=lambda d: -st[d])
    if any(s <= 0 for s in st):
        return None
    for i in range(len(order) - 1):
        a, b = order[i], order[i + 1]
        if st[a] % st[b] != 0 or st[a] < st[b] * shape[b]:
            return None
    coords = np.zeros((len(base), len(st)), dtype=np.int64)
    rem = base.copy()
    for d in order:
        coords[:, d] = rem // st[d]
        rem = rem - coords[:, d] * st[d]
    if np.any(rem != 0):
        return None
    return coords


def verify(accesses: List[Access], insts: Instances) -> Optional[str]:
    """Return None when reordering lanes cannot change any HBM result, else a reason."""
    by_alloc: Dict[int, List[Access]] = {}
    for a in accesses:
        by_alloc.setdefault(id(a.alloc), []).append(a)
    for lst in by_alloc.values():
        if not any(a.store for a in lst):
            continue
        name = lst[0].alloc.name
        groups = {a.group for a in lst}
        if len(groups) == 1 and None not in groups:
            continue
        all_insts = np.concatenate([a.inst for a in lst])
        if len(np.unique(all_insts)) == 1:
            continue
        if any(a.whole for a in lst):
            roots = set(int(i) for i in np.unique(all_insts))
            if not _all_comparable(roots, insts):
                return f"data-dependent access to {name!r} from several lanes"
            continue
        key0 = (lst[0].shape, lst[0].strides)
        same = all((a.shape, a.strides) == key0 for a in lst)
        if same:
            shape, strides = key0
            cells, inst_all, store_all = [], [], []
            ok = True
            for a in lst:
                c = _decompose(a.base, shape, strides)
                if c is None:
                    ok = False
                    break
                cells.append(c)
                inst_all.append(a.inst)
                store_all.append(np.full(len(a.inst), a.store))
            aligned = ok and not any(np.any(c % np.maximum(np.asarray(shape, dtype=np.int64), 1) != 0)
                                     for c in cells)
            if ok and not aligned and _no_carry(np.concatenate(cells), shape, strides):
                why = _box_hazard(np.concatenate(cells), shape, np.concatenate(inst_all),
                                  np.concatenate(store_all), insts, name)
                if why is not None:
                    return why
                continue
            if aligned:
                cells = np.concatenate(cells)
                inst_all = np.concatenate(inst_all)
                store_all = np.concatenate(store_all)
                _, key = np.unique(cells, axis=0, return_inverse=True)
                key = key.reshape(-1)
                order = np.lexsort((inst_all, key))
                k, ins, st = key[order], inst_all[order], store_all[order]
                # cells touched by more than one instance
                brk = np.flatnonzero(np.diff(k) != 0) + 1
                starts = np.concatenate([[0], brk])
                ends = np.concatenate([brk, [len(k)]])
                multi = [(s, e) for s, e in zip(starts, ends) if ins[s] != ins[e - 1]]
                if len(multi) > 4096:
                    return f"{name!r}: many tiles shared between lanes"
                for s, e in multi:
                    if not st[s:e].any():
                        continue
                    if not _all_comparable(set(int(x) for x in ins[s:e]), insts):
                        return f"{name!r}: lanes of different cores/iterations share a tile"
                continue
        # general case: byte intervals
        lo, hi, ins, sto = [], [], [], []
        for a in lst:
            ext = sum((s - 1) * abs(st) for s, st in zip(a.shape, a.strides) if s > 0)
            neg = sum((s - 1) * st for s, st in zip(a.shape, a.strides) if st < 0 and s > 0)
            lo.append(a.base + neg)
            hi.append(a.base + neg + ext + 1)
            ins.append(a.inst)
            sto.append(np.full(len(a.inst), a.store))
        lo, hi, ins, sto = map(np.concatenate, (lo, hi, ins, sto))
        order = np.argsort(lo, kind="stable")
        lo, hi, ins, sto = lo[order], hi[order], ins[order], sto[order]
        run_hi = np.maximum.accumulate(hi)
        overl = np.flatnonzero(lo[1:] < run_hi[:-1]) + 1
        if len(overl) > 20000:
            return f"{name!r}: overlapping accesses between lanes"
        for j in overl:
            i = j - 1
            while i >= 0 and run_hi[i] > lo[j]:
                if hi[i] > lo[j] and (sto[i] or sto[j]) and ins[i] != ins[j] \
                        and not insts.comparable(int(ins[i]), int(ins[j])):
                    return f"{name!r}: overlapping accesses between lanes"
                i -= 1
                if j - i > 64:
                    return f"{name!r}: overlapping accesses between lanes"
    return None


def _no_carry(c: np.ndarray, shape, strides) -> bool:
    """Whether boxes of `shape` at digit coordinates `c` (rows, from
    `_decompose`) stay inside each digit's range: then two boxes share an
    element exactly when their coordinates differ by less than the shape in
    every dimension."""
    st = list(strides)
    order = sorted(range(len(st)), key=lambda d: -st[d])
    for p in range(1, len(order)):
        d, up = order[p], order[p - 1]
        if np.any(c[:, d] + shape[d] > st[up] // st[d]):
            return False
    return True


def _box_hazard(c: np.ndarray, shape, inst: np.ndarray, store: np.ndarray, insts: Instances,
                name) -> Optional[str]:
    """Exact conflict test for equal boxes that need not sit on multiples of
    their shape (a tile that starts at row 9 of 2-row tiles): each box
    touches at most two shape-sized grid cells per dimension, boxes that
    share no grid cell share no element, and the candidates that do share
    one are compared coordinate by coordinate."""
    shp = np.maximum(np.asarray(shape, dtype=np.int64), 1)
    g = c // shp
    un = np.flatnonzero(np.any(c % shp != 0, axis=0))
    if len(un) > 6:
        return f"{name!r}: overlapping accesses between lanes"
    n = len(c)
    keys = []
    for bits in range(1 << len(un)):
        gg = g.copy()
        for k, d in enumerate(un):
            if bits >> k & 1:
                gg[:, d] += 1
        keys.append(gg)
    owner = np.tile(np.arange(n, dtype=np.int64), 1 << len(un))
    _, kid = np.unique(np.concatenate(keys), axis=0, return_inverse=True)
    kid = kid.reshape(-1)
    order = np.argsort(kid, kind="stable")
    kid, owner = kid[order], owner[order]
    big = int(np.unique(kid, return_counts=True)[1].max())
    if big > 64:
        return f"{name!r}: many tiles shared between lanes"
    for k in range(1, big):
        same = kid[k:] == kid[:-k]
        i, j = owner[:-k][same], owner[k:][same]
        hit = (np.all(np.abs(c[i] - c[j]) < shp, axis=1) & (store[i] | store[j]) & (inst[i] != inst[j]))
        pairs = np.flatnonzero(hit)
        if len(pairs) > 4096:
            return f"{name!r}: many tiles shared between lanes"
        for q in pairs:
            if not insts.comparable(int(inst[i[q]]), int(inst[j[q]])):
                return f"{name!r}: overlapping accesses between lanes"
    return None


def _all_comparable(ids: set, insts: Instances) -> bool:
    ids = list(ids)
    if len(ids) > 64:
        return False
    for i in range(len(ids)):
        for j in range(i + 1, len(ids)):
            if not insts.comparable(ids[i], ids[j]):
                return False
    return True


# ---------------------------------------------------------------------------
# launch plan
# ---------------------------------------------------------------------------

class V16Copy:
    """The f16 copy of a bf16 V range that an attention launch makes: valid
    on a replay when no launch of the plan stores into V (`ok`, set when the
    walk ends) and the buffer holding V has had no host write since the
    launch that made it (`gen`)."""

    def __init__(self, alloc, buf):
        self.alloc, self.buf = alloc, buf
        self.ok = False
        self.gen = None


class Plan:
    """The recorded launch sequence of one execute_function call."""

    def __init__(self, pool: Pool):
        self.pool = pool
        self.launches: List[Tuple] = []
        self.replayable = True
        self.ran_during_walk = False     # launches already ran as they were walked
        self.mode = "lockstep"
        self.fallback_reason = None
        self.v16: Dict[int, V16Copy] = {}   # id(attention descriptor) -> its V copy

    def add(self, kind, desc, keep=()):
        # a list stays shared with the caller, who may still append buffers
        # that a later rewrite of `desc` points at
        self.launches.append((kind, desc, keep if isinstance(keep, list) else tuple(keep)))

    def run(self, after=None, reuse_v16=True):
        """Replay every launch; `after(i)`, if given, runs after launch i is
        queued (the bench records a HIP event there).  With reuse_v16 false
        every attention launch converts its V again, as a call with a new V
        does."""
        L = rt.lib()
        for i, (kind, desc, _) in enumerate(self.launches):
            c = self.v16.get(id(desc)) if kind == "attn" else None
            if c is not None:
                desc.v16_ready = int(reuse_v16 and c.ok and c.gen is not None and c.gen == c.buf.host_writes)
                _launch(L, kind, desc)
                c.gen = c.buf.host_writes
            else:
                _launch(L, kind, desc)
            if after is not None:
                after(i)

    def counts(self) -> Dict[str, int]:
        out: Dict[str, int] = {}
        for kind, _, _ in self.launches:
            out[kind] = out.get(kind, 0) + 1
        return out

    def rmw_variants(self) -> List[str]:
        """The apply kernel of each ordered row RMW launch ("rows" or "generic")."""
        import ctypes as C
        names = {rt.K["KTIR_RMW_ROWS"]: "rows", rt.K["KTIR_RMW_GENERIC"]: "generic"}
        out = []
        for kind, desc, _ in self.launches:
            if kind == "rmw":
                v = rt.lib().ktir_rmw_variant(C.byref(desc))
                if v < 0:
                    rt.check(v, "ktir_rmw_variant")
                out.append(names[v])
        return out


def _launch(L, kind, desc):
    import ctypes as C
    if kind == "prog":
        rt.check(L.ktir_launch_program(C.byref(desc)), "ktir_launch_program")
    elif kind == "mm":
        rt.check(L.ktir_launch_matmul(C.byref(desc)), "ktir_launch_matmul")
    elif kind == "iat":
        rt.check(L.ktir_iat_offsets(C.byref(desc)), "ktir_iat_offsets")
    elif kind == "winners":
        leaf, lanes, n, ptr = desc
        rt.check(L.ktir_scatter_winners(C.byref(leaf), lanes, n, ptr), "ktir_scatter_winners")
    elif kind == "rmw":
        rt.check(L.ktir_launch_row_rmw(C.byref(desc)), "ktir_launch_row_rmw")
    elif kind == "attn":
        rt.check(L.ktir_launch_attention(C.byref(desc)), "ktir_launch_attention")
    elif kind == "pattn":
        rt.check(L.ktir_launch_paged_attention(C.byref(desc)), "ktir_launch_paged_attention")
    elif kind == "memset":
        ptr, val, nbytes = desc
        rt.check(L.ktir_memset(ptr, val, nbytes), "ktir_memset")
    else:
        raise ValueError(kind)
