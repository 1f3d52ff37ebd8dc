"""`KTIRInterpreter`: the drop-in API of the reference, executed on an MI355X.

Same surface as the reference's ``ktir_cpu/interpreter.py:40-395``:
``load``, ``arg_names``, ``tensor_input_output_sizes``, ``execute_function``
(returns every ndarray argument read back after the run, inputs included)
and ``get_latency_report``.  The arguments are laid out in a device arena at
the byte addresses the reference's HBM simulator gives them
(``interpreter.py:161-172``: one stick-aligned allocation per array, pointer
argument = element index), the function runs through the lockstep executor
(``walker.Executor``) and the results are copied back into fresh arrays.
There is no CPU execution path: a missing library or GPU raises.
"""

from __future__ import annotations

import time
from typing import Any, Dict, List, Optional

import numpy as np

from . import runtime as rt
from .executor import Arena, LXSpace, NeedEager, Plan, Pool, STICK_BYTES
from .ir import IRModule
from .latency import LatencyReport, LatencyTracker
from .memory import DeviceMemory
from .parser import KTIRParser
from .walker import Executor, _has_op

_NP_TO_KTIR = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.int32): "i32",
               np.dtype(np.int64): "i64", np.dtype(np.uint16): "bf16", np.dtype(np.bool_): "i1",
               np.dtype(np.int8): "i8", np.dtype(np.int16): "i16"}


def ktir_dtype_of(arr: np.ndarray) -> str:
    """KTIR dtype of a host array; bf16 tensors travel as uint16 bit patterns."""
    try:
        return _NP_TO_KTIR[arr.dtype]
    except KeyError:
        raise ValueError(f"Unsupported array dtype {arr.dtype} (reference dtypes.py:24-39 plus bf16 as uint16)")


def _uses_lx(ops) -> bool:
    """Whether any memory view of the function lies in LX (ct_local)."""
    for op in ops:
        if op.attributes.get("memory_space") == "LX":
            return True
        if any(_uses_lx(r.ops) for r in op.regions):
            return True
    return False


# the LX space of one run (cores x LX bytes) is refused above this size
MAX_LX_SPACE = 32 << 30


def _storage_dtype(arr: np.ndarray) -> str:
    """KTIR dtype of a staged HBM seed (any host dtype: one of the same size)."""
    try:
        return ktir_dtype_of(arr)
    except ValueError:
        return {1: "i8", 2: "i16", 4: "i32", 8: "i64"}[arr.dtype.itemsize]


class Prepared:
    """Arguments resident on the device plus the launch plan of one function:
    `run()` replays the device work only (no host walk, no copies)."""

    def __init__(self, interp: "KTIRInterpreter", fn_name: str, names: List[str], plan: Plan, arena: Arena,
                 arrays: Dict[str, np.ndarray], initial: Optional[Dict[str, np.ndarray]] = None, lx=None):
        self.interp = interp
        self.lx = lx
        self.fn_name = fn_name
        self.names = names
        self.plan = plan
        self.arena = arena
        self.arrays = arrays
        self.initial = initial if initial is not None else arrays

    def run(self):
        self.plan.run()

    def reset_inputs(self):
        for a in self.arena.allocs:
            arr = self.initial[a.name]
            self.arena.buf.upload(np.ascontiguousarray(arr).reshape(-1).view(np.uint8), a.off)
        if self.lx is not None:
            self.lx.reset()

    def outputs(self) -> Dict[str, np.ndarray]:
        """Every array argument read back (staged HBM seeds are not arguments)."""
        rt.sync()
        out = {}
        for a in self.arena.allocs:
            if a.name not in self.arrays:
                continue
            src = self.arrays[a.name]
            dst = np.empty(src.shape, dtype=src.dtype)
            self.arena.buf.download_into(dst, a.off)
            out[a.name] = dst
        return out


class KTIRInterpreter:
    """Drop-in for the reference ``KTIRInterpreter`` running on one MI355X."""

    def __init__(self, latency_config=None, trace_latency: bool = False, parser=None, lx_size_mb: Optional[int] = None):
        self.module: Optional[IRModule] = None
        self._parser = parser or KTIRParser()
        self.latency_config = latency_config
        self.trace_latency = trace_latency
        if lx_size_mb is None:
            lx_size_mb = int(getattr(latency_config, "lx_size_mb", 2) or 2) if latency_config is not None else 2
        self.lx_size_mb = lx_size_mb
        self.last_plan: Optional[Plan] = None
        self._arena = Arena()
        self._pool = None
        self._lx: Optional[LXSpace] = None
        self.memory: Optional[DeviceMemory] = None
        # latency model (reference interpreter.py:76-78): charged op by op during the run
        self._latency_tracker = LatencyTracker(latency_config, trace=trace_latency) if latency_config is not None \
            else None

    # -- reference API ------------------------------------------------------
    def load(self, src: str):
        """Path to a .mlir file, or inline KTIR text (reference interpreter.py:81-93)."""
        if "\n" in src or src.lstrip().startswith("module"):
            self.module = self._parser.parse_module(src)
        else:
            self.module = self._parser.parse_file(src)

    def arg_names(self, fn: str) -> List[str]:
        if not self.module:
            raise RuntimeError("No module loaded. Call load() first.")
        return self.module.get_function(fn).arg_names

    def tensor_input_output_sizes(self, fn: str):
        if not self.module:
            raise RuntimeError("No module loaded. Call load() first.")
        return self.module.get_function(fn).tensor_sizes

    def get_latency_report(self) -> Optional[LatencyReport]:
        """Latency report of the last run, or None when no latency_config was given."""
        if self._latency_tracker is None:
            return None
        return self._latency_tracker.report()

    def execute_function(self, fn_name: str, **kwargs) -> Dict[str, np.ndarray]:
        """Run `fn_name` on the GPU; returns every ndarray argument (reference interpreter.py:122-194)."""
        prep = self.prepare(fn_name, **kwargs)
        return prep.outputs()

    def _prepare_execution(self, grid_shape):
        """A fresh memory for one run (reference interpreter.py:95-120).
        Callers may wrap this to seed ``self.memory.hbm`` at literal sticks."""
        nx, ny, nz = grid_shape
        self.memory = DeviceMemory(nx * ny * nz, self.lx_size_mb)

    # -- GPU-specific ---------------------------------------------------------
    def prepare(self, fn_name: str, **kwargs) -> Prepared:
        """Place the arguments on the device, walk the function once, launch
        it, and return a handle that can replay the device work."""
        if not self.module:
            raise RuntimeError("No module loaded. Call load() first.")
        fn = self.module.get_function(fn_name)
        self._prepare_execution(fn.grid)
        hbm = self.memory.hbm
        declared = fn.arg_names
        if kwargs and declared and not any(k in declared for k in kwargs):
            if len(kwargs) == len(declared):
                kwargs = dict(zip(declared, kwargs.values()))
        rt.lib()
        arrays = {k: v for k, v in kwargs.items() if isinstance(v, np.ndarray)}
        initial: Dict[str, np.ndarray] = dict(arrays)
        specs = []
        for k, v in arrays.items():
            specs.append((k, ktir_dtype_of(v), hbm.allocate(v.nbytes) * STICK_BYTES, int(v.nbytes), tuple(v.shape)))
        for addr, v in hbm.staged():
            name = f"__hbm_0x{addr:x}"
            initial[name] = v
            specs.append((name, _storage_dtype(v), addr, int(v.nbytes), tuple(v.shape)))
        if self._pool is not None:
            self._pool.free_all()
        self._pool = Pool()
        if self._lx is not None:
            self._lx.free()
            self._lx = None
        seeds = self.memory.lx_seeds()
        if seeds or _uses_lx(fn.operations):
            nx, ny, nz = fn.grid
            per = self.memory.lx_size_mb * 1024 * 1024
            if nx * ny * nz * per > MAX_LX_SPACE:
                raise NotImplementedError(f"LX space of {nx * ny * nz} cores x {per} bytes exceeds "
                                          f"{MAX_LX_SPACE} bytes")
            self._lx = LXSpace(nx * ny * nz, per)
            self._lx.seed(seeds)
        self.memory.attach_lx(self._lx)
        arena = Arena()
        arena.layout(specs)
        self._arena = arena
        args: Dict[str, Any] = {}
        for a in arena.allocs:
            v = initial[a.name]
            arena.buf.upload(np.ascontiguousarray(v).reshape(-1).view(np.uint8), a.off)
            if a.name in arrays:
                args[a.name] = np.int64(a.addr // rt.ELEM_BYTES[a.dtype])
        hbm.attach(arena, {k: v.dtype for k, v in initial.items()})
        for k, v in kwargs.items():
            if not isinstance(v, np.ndarray):
                args[k] = np.asarray(v)
        plan = None
        lat = self._latency_tracker
        if lat is not None:
            # the latency model needs every op of every core, with the data
            # its memory costs depend on: run core by core, op by op, on the GPU
            nx, ny, nz = fn.grid
            lat.reset()
            lat.set_cores_active(nx * ny * nz)
            # cores that meet at a ring reduce run together (op by op, as walked)
            collective = _has_op(fn.operations, "ktdp.inter_tile_reduce")
            ex = Executor(fn, arena, args, self._pool, sequential=not collective, lx_size_mb=self.lx_size_mb,
                          latency=lat, lx=self._lx)
            try:
                plan = ex.run()
            except NeedEager as why:
                raise NotImplementedError(f"latency model for cores that meet at a ring reduce: {why}") from None
            plan.fallback_reason = "latency model"
        else:
            try:
                ex = Executor(fn, arena, args, self._pool, sequential=False, lx_size_mb=self.lx_size_mb,
                              lx=self._lx)
                plan = ex.run()
                if not plan.ran_during_walk:
                    plan.run()
            except NeedEager as why:
                ex = Executor(fn, arena, args, self._pool, sequential=True, lx_size_mb=self.lx_size_mb,
                              lx=self._lx)
                plan = ex.run()
                plan.fallback_reason = str(why)
        rt.sync()
        self.last_plan = plan
        return Prepared(self, fn_name, list(arrays), plan, arena, arrays, initial, self._lx)
