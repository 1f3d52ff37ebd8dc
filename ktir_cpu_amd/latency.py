"""Host-side latency model of a KTIR kernel on Spyre, fed by the GPU run.

The reference estimates a cycle count per (core, op) while it interprets
(``latency.py:289-506``, called from ``interpreter.py:207-279``) and
reports the critical core, the bottleneck and a roofline
(``latency.py:563-846``).  This module keeps that model and its public names
(``HardwareConfig``, ``ExecutionModel``, ``LatencyCategory``,
``CoreLatencyCounters``, ``LatencyTracker``, ``LatencyReport``) so callers
can switch, but it is fed differently: the executor charges each op once it
has run it on the GPU, with the quantities the model needs computed for that
core.  Those quantities are the result element count, the matmul M/N/K, and
the HBM bytes of a load or store at stick granularity (unique 128-byte
sticks of the data and, for an indirect access, of the index tensor).  The
indirect offsets are the ones the GPU kernel produced.

Cost rules (``latency.py:329-432``):
  memory     bytes / (chip HBM bandwidth / clock / active cores)
  matmul     2 M N K / (2 x SIMD width x systolic rows) per cycle
  float      elements / SIMD width
  transc.    elements / SIMD width x transcendental penalty
  int        elements / SIMD width (0 for scalar index arithmetic)
  comm       bytes / ring bytes per cycle
  zero       free
A core's cycles combine as the execution model's pipeline says; the kernel
takes as long as its slowest core.
"""

from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Dict, List, Optional, Tuple

STICK_BYTES = 128


class LatencyCategory(str, Enum):
    """Cost class of an op (its value is the category string)."""
    ZERO = "zero"
    MEMORY = "memory"
    COMPUTE_FLOAT = "compute_float"
    COMPUTE_TRANSCENDENTAL = "compute_transcendental"
    COMPUTE_INT = "compute_int"
    COMPUTE_MATMUL = "compute_matmul"
    COMM = "comm"

    def __str__(self) -> str:
        return self.value


LC = LatencyCategory

# op type -> category, as the reference's op registry declares them
# (dialects/arith_ops.py, math_ops.py, linalg_ops.py, ktdp_ops.py); every
# other op (casts, views, constants, control flow, linalg.reduce) is free.
_CATEGORY: Dict[str, LatencyCategory] = {}
for _n in ("addf", "subf", "mulf", "divf", "remf", "negf", "absf", "maxf", "maximumf", "maxnumf", "minf",
           "minimumf", "minnumf", "cmpf", "select"):
    _CATEGORY["arith." + _n] = LC.COMPUTE_FLOAT
for _n in ("addi", "subi", "muli", "divui", "divsi", "floordivsi", "remui", "remsi", "andi", "ori", "xori", "shli",
           "shrsi", "shrui", "minsi", "maxsi", "minui", "maxui", "ceildivsi", "ceildivui", "cmpi"):
    _CATEGORY["arith." + _n] = LC.COMPUTE_INT
for _n in ("exp", "sqrt", "rsqrt", "log", "log2", "log1p", "tanh", "sin", "cos", "erf", "powf"):
    _CATEGORY["math." + _n] = LC.COMPUTE_TRANSCENDENTAL
for _n in ("absf", "absi", "ceil", "floor", "fma"):
    _CATEGORY["math." + _n] = LC.COMPUTE_FLOAT
for _n in ("linalg.add", "linalg.max", "linalg.generic"):
    _CATEGORY[_n] = LC.COMPUTE_FLOAT
_CATEGORY["linalg.matmul"] = LC.COMPUTE_MATMUL
_CATEGORY["linalg.batch_matmul"] = LC.COMPUTE_MATMUL
_CATEGORY["ktdp.load"] = LC.MEMORY
_CATEGORY["ktdp.store"] = LC.MEMORY
_CATEGORY["ktdp.inter_tile_reduce"] = LC.COMM


def category_of(op_type: str) -> LatencyCategory:
    """Latency category of an op type (``zero`` when it has none)."""
    return _CATEGORY.get(op_type, LC.ZERO)


@dataclass
class ExecutionModel:
    """How the hardware is programmed (reference ``latency.py:55-96``).

    unit_categories: categories each compute unit claims.
    pipeline: "serial" (compute + memory + comm), "overlapped"
        (max(compute, memory + comm)) or "overlapped_3way"
        (max(compute, memory, comm)).
    bw_sharing: "contended" (chip HBM bandwidth split over the active cores);
        "static" is reserved and rejected.
    fallback_unit: dominant unit when no compute ran.
    """
    unit_categories: Dict[str, set] = field(default_factory=lambda: {
        "systolic": {"compute_matmul"},
        "simd": {"compute_float", "compute_transcendental", "compute_int"},
    })
    pipeline: str = "serial"
    bw_sharing: str = "contended"
    fallback_unit: str = "simd"

    def __post_init__(self):
        if self.bw_sharing == "static":
            raise NotImplementedError("bw_sharing='static' is reserved; only 'contended' is available")
        if self.bw_sharing != "contended":
            raise ValueError(f"bw_sharing must be 'contended' (got {self.bw_sharing!r})")


@dataclass
class HardwareConfig:
    """Spyre parameters of the model (reference ``latency.py:103-187``);
    the defaults are the reference's example values."""
    num_cores: int = 32
    clock_ghz: float = 1.0
    hbm_bandwidth_tb_s: float = 0.128
    ring_bandwidth_tb_s: float = 0.064
    simd_elements_per_cycle: int = 64
    systolic_rows: int = 8
    transcendental_penalty: int = 4
    lx_size_mb: int = 2

    @property
    def clock_hz(self) -> float:
        return self.clock_ghz * 1e9

    @property
    def hbm_bw_chip(self) -> float:
        """Aggregate HBM bandwidth in B/s."""
        return self.hbm_bandwidth_tb_s * 1e12

    @property
    def systolic_flops_per_cycle(self) -> int:
        """Each systolic row does one FMA (2 FLOP) on a SIMD-width vector per cycle."""
        return 2 * self.simd_elements_per_cycle * self.systolic_rows

    @property
    def systolic_peak(self) -> float:
        return self.systolic_flops_per_cycle * self.clock_hz

    @property
    def simd_peak(self) -> float:
        return self.simd_elements_per_cycle * self.clock_hz

    def lx_bytes_per_cycle(self) -> float:
        return self.ring_bandwidth_tb_s * 1e12 / (self.clock_ghz * 1e9)

    def lx_bytes_per_cycle_per_core(self) -> float:
        return self.lx_bytes_per_cycle()

    @property
    def ring_bytes_per_cycle(self) -> float:
        return self.ring_bandwidth_tb_s * 1e12 / self.clock_hz


@dataclass
class _TraceEntry:
    op_type: str
    cycles: float
    category: str


@dataclass
class CoreLatencyCounters:
    """Cycles, FLOPs and bytes charged to one core (reference ``latency.py:202-281``)."""
    memory_cycles: float = 0.0
    comm_cycles: float = 0.0
    flops_by_category: Dict[str, float] = field(default_factory=dict)
    cycles_by_category: Dict[str, float] = field(default_factory=dict)
    bytes_by_category: Dict[str, int] = field(default_factory=dict)
    trace: Optional[List[_TraceEntry]] = None

    @property
    def compute_cycles(self) -> float:
        return sum(self.cycles_by_category.values())

    @property
    def total_cycles(self) -> float:
        return self.compute_cycles + self.memory_cycles + self.comm_cycles

    @property
    def total_flops(self) -> float:
        return sum(self.flops_by_category.values())

    @property
    def total_bytes(self) -> int:
        return sum(self.bytes_by_category.values())

    @property
    def comm_bytes(self) -> int:
        return self.bytes_by_category.get("comm", 0)

    @property
    def dram_bytes(self) -> int:
        """HBM bytes only (the roofline's arithmetic-intensity denominator)."""
        return self.bytes_by_category.get("memory", 0)

    def record(self, category: str, cycles: float, op_type: str = "", flops: float = 0.0, nbytes: int = 0):
        category = str(category)
        if category.startswith("compute_"):
            self.cycles_by_category[category] = self.cycles_by_category.get(category, 0.0) + cycles
            self.flops_by_category[category] = self.flops_by_category.get(category, 0.0) + flops
        elif category == "memory":
            self.memory_cycles += cycles
        elif category == "comm":
            self.comm_cycles += cycles
        if nbytes:
            self.bytes_by_category[category] = self.bytes_by_category.get(category, 0) + nbytes
        if self.trace is not None:
            self.trace.append(_TraceEntry(op_type=op_type, cycles=cycles, category=category))


class LatencyTracker:
    """Per-core counters, filled by the executor as it runs ops."""

    def __init__(self, config: HardwareConfig, trace: bool = False):
        self.config = config
        self._trace = trace
        self.counters: Dict[int, CoreLatencyCounters] = {}
        self._cores_active = config.num_cores

    def set_cores_active(self, cores_active: int):
        """Cores sharing the HBM bandwidth (the grid size)."""
        self._cores_active = cores_active

    def reset(self):
        self.counters.clear()

    def cost(self, op_type: str, n_elems: int = 1, mnk: Optional[Tuple[int, int, int]] = None,
             nbytes: int = 0) -> Tuple[str, float, float, int]:
        """(category, cycles, flops, bytes) of one op on one core."""
        cfg = self.config
        cat = category_of(op_type)
        if cat == LC.ZERO:
            return ("zero", 0.0, 0.0, 0)
        if cat == LC.MEMORY:
            bw = cfg.hbm_bw_chip / cfg.clock_hz / self._cores_active
            return ("memory", nbytes / bw if bw > 0 else 0.0, 0.0, int(nbytes))
        if cat == LC.COMPUTE_MATMUL:
            m, n, k = mnk or (1, 1, 1)
            flops = 2.0 * m * n * k
            return (str(cat), flops / cfg.systolic_flops_per_cycle, flops, 0)
        if cat == LC.COMPUTE_TRANSCENDENTAL:
            return (str(cat), n_elems / cfg.simd_elements_per_cycle * cfg.transcendental_penalty, float(n_elems), 0)
        if cat == LC.COMPUTE_FLOAT:
            return (str(cat), n_elems / cfg.simd_elements_per_cycle, float(n_elems), 0)
        if cat == LC.COMPUTE_INT:
            if n_elems <= 1:
                return (str(cat), 0.0, 0.0, 0)
            return (str(cat), n_elems / cfg.simd_elements_per_cycle, float(n_elems), 0)
        bw = cfg.ring_bytes_per_cycle
        return ("comm", nbytes / bw if bw > 0 else 0.0, 0.0, int(nbytes))

    def record_op(self, core_id: int, op_type: str, n_elems: int = 1, mnk: Optional[Tuple[int, int, int]] = None,
                  nbytes: int = 0):
        """Charge one op run on `core_id`."""
        c = self.counters.get(core_id)
        if c is None:
            c = self.counters[core_id] = CoreLatencyCounters(trace=[] if self._trace else None)
        cat, cycles, flops, b = self.cost(op_type, n_elems, mnk, nbytes)
        c.record(cat, cycles, op_type, flops=flops, nbytes=b)

    def report(self) -> "LatencyReport":
        return LatencyReport(config=self.config, counters=dict(self.counters))


@dataclass
class LatencyReport:
    """Kernel latency, bottleneck and roofline (reference ``latency.py:563-846``)."""
    config: HardwareConfig
    counters: Dict[int, CoreLatencyCounters]
    model: ExecutionModel = field(default_factory=ExecutionModel)

    def _effective_cycles(self, c: CoreLatencyCounters) -> float:
        p = self.model.pipeline
        if p == "overlapped":
            return max(c.compute_cycles, c.memory_cycles + c.comm_cycles)
        if p == "overlapped_3way":
            return max(c.compute_cycles, c.memory_cycles, c.comm_cycles)
        return c.compute_cycles + c.memory_cycles + c.comm_cycles

    @property
    def critical_core(self) -> CoreLatencyCounters:
        return max(self.counters.values(), key=self._effective_cycles)

    @property
    def kernel_cycles(self) -> float:
        return self._effective_cycles(self.critical_core) if self.counters else 0.0

    @property
    def kernel_time_us(self) -> float:
        return self.kernel_cycles / (self.config.clock_hz / 1e6)

    @property
    def bottleneck(self) -> str:
        if not self.counters:
            return "none"
        c = self.critical_core
        parts = {"compute": c.compute_cycles, "memory": c.memory_cycles, "comm": c.comm_cycles}
        return max(parts, key=parts.get)

    def per_core_summary(self) -> List[Dict[str, Any]]:
        return [{"core_id": k, "compute_cycles": c.compute_cycles, "memory_cycles": c.memory_cycles,
                 "comm_cycles": c.comm_cycles, "total_cycles": self._effective_cycles(c)}
                for k, c in sorted(self.counters.items())]

    # -- roofline -------------------------------------------------------------
    @staticmethod
    def _roofline_at(flops: float, nbytes: float, peak_compute: float, peak_bw: float,
                     elapsed_s: float) -> Dict[str, Any]:
        inf = float("inf")
        ai = flops / nbytes if nbytes > 0 else inf
        achieved = flops / elapsed_s if elapsed_s > 0 else 0.0
        ceiling = min(peak_compute, peak_bw * ai) if ai != inf else peak_compute
        return {
            "AI": ai,
            "compute_throughput": achieved / peak_compute if peak_compute > 0 else 0.0,
            "dram_throughput": nbytes / (peak_bw * elapsed_s) if elapsed_s > 0 and peak_bw > 0 else 0.0,
            "achieved_gflops": achieved / 1e9,
            "ceiling_gflops": ceiling / 1e9,
            "attainment": achieved / ceiling if ceiling > 0 else 0.0,
            "ridge": peak_compute / peak_bw if peak_bw > 0 else inf,
            "peak_gflops": peak_compute / 1e9,
        }

    def _dominant_unit(self) -> str:
        """The unit with the most cycles over the whole chip."""
        per_cat: Dict[str, float] = {}
        for c in self.counters.values():
            for cat, cyc in c.cycles_by_category.items():
                per_cat[cat] = per_cat.get(cat, 0.0) + cyc
        totals = {u: sum(per_cat.get(cat, 0.0) for cat in cats) for u, cats in self.model.unit_categories.items()}
        return max(totals, key=totals.get) if any(totals.values()) else self.model.fallback_unit

    def _unit_peaks(self) -> Dict[str, float]:
        return {"systolic": self.config.systolic_peak, "simd": self.config.simd_peak}

    def _cores_active(self) -> int:
        return sum(1 for c in self.counters.values() if self._effective_cycles(c) > 0)

    def chip_roofline(self) -> Dict[str, Any]:
        """The whole chip as one unit."""
        if not self.counters:
            return {}
        dom = self._dominant_unit()
        cats = self.model.unit_categories[dom]
        n_cores = self.config.num_cores
        elapsed_cycles = self.kernel_cycles
        elapsed_s = elapsed_cycles / self.config.clock_hz
        flops = sum(c.flops_by_category.get(cat, 0.0) for c in self.counters.values() for cat in cats)
        dram = sum(c.dram_bytes for c in self.counters.values())
        busy = sum(self._effective_cycles(c) for c in self.counters.values())
        active = self._cores_active()
        rf = self._roofline_at(flops, dram, self._unit_peaks()[dom] * n_cores, self.config.hbm_bw_chip, elapsed_s)
        rf.update({
            "mean_core_active_frac": busy / (n_cores * elapsed_cycles) if n_cores > 0 and elapsed_cycles > 0 else 0.0,
            "grid_coverage": active / n_cores if n_cores > 0 else 0.0,
            "dominant_unit": dom,
            "num_cores": n_cores,
            "cores_active": active,
        })
        return rf

    def core_roofline(self) -> Dict[str, Any]:
        """The critical core, unit by unit, at its share of the HBM bandwidth."""
        if not self.counters:
            return {}
        dom = self._dominant_unit()
        crit = self.critical_core
        elapsed_s = self.kernel_cycles / self.config.clock_hz
        peak_bw = self.config.hbm_bw_chip / self._cores_active()
        units = {}
        for unit, peak in self._unit_peaks().items():
            flops = sum(crit.flops_by_category.get(cat, 0.0) for cat in self.model.unit_categories[unit])
            units[unit] = self._roofline_at(flops, crit.dram_bytes, peak, peak_bw, elapsed_s)
        return {
            "core_AI": units[dom]["AI"],
            "core_attainment": units[dom]["attainment"],
            "core_dominant_unit": dom,
            "peak_bw_gb_s": peak_bw / 1e9,
            "ridge": units[dom]["ridge"],
            "units": units,
        }

    def roofline(self) -> Dict[str, Any]:
        if not self.counters:
            return {}
        return {**self.core_roofline(), **self.chip_roofline()}

    def summary_dict(self) -> Dict[str, Any]:
        return {
            "kernel_cycles": self.kernel_cycles,
            "kernel_time_us": self.kernel_time_us,
            "bottleneck": self.bottleneck,
            "grid_cores": len(self.counters),
            "num_cores": self.config.num_cores,
            "per_core": self.per_core_summary(),
        }

    def __str__(self) -> str:
        bar = "=" * 60
        out = [bar, "KTIR Latency Estimation Report", bar,
               f"  Kernel cycles : {self.kernel_cycles:,.1f}",
               f"  Kernel time   : {self.kernel_time_us:.3f} us",
               f"  Bottleneck    : {self.bottleneck}",
               f"  Cores         : {len(self.counters)}",
               "-" * 60,
               f"  {'Core':>4}  {'Compute':>12}  {'Memory':>12}  {'Comm':>12}  {'Total':>12}",
               "-" * 60]
        for k, c in sorted(self.counters.items()):
            out.append(f"  {k:>4}  {c.compute_cycles:>12.1f}  {c.memory_cycles:>12.1f}  {c.comm_cycles:>12.1f}  "
                       f"{self._effective_cycles(c):>12.1f}")
        out.append(bar)
        if not self.counters:
            return "\n".join(out)
        crit = self.critical_core
        if crit.total_flops > 0 or crit.total_bytes > 0:
            chip, core = self.chip_roofline(), self.core_roofline()

            def ai_text(ai: float) -> str:
                if ai != float("inf"):
                    return f"{ai:.2f} FLOP/B"
                return "inf (no HBM traffic)" if crit.total_bytes > 0 else "inf (no memory traffic)"

            out += ["", "Roofline: CHIP-LEVEL  (whole chip as one unit)", "-" * 60,
                    f"  AI                    : {ai_text(chip['AI'])}",
                    f"  compute_throughput    : {chip['compute_throughput']:.1%}",
                    f"  dram_throughput       : {chip['dram_throughput']:.1%}",
                    f"  attainment            : {chip['attainment']:.1%}",
                    f"  mean_core_active_frac : {chip['mean_core_active_frac']:.1%}",
                    f"  grid_coverage         : {chip['cores_active']}/{chip['num_cores']}  "
                    f"({chip['grid_coverage']:.1%})",
                    f"  dominant_unit         : {chip['dominant_unit']}"]
            dom = core["core_dominant_unit"]
            out += ["", "Roofline: PER-CORE  (critical-path core)", "-" * 60,
                    f"  core_AI               : {ai_text(core['core_AI'])}",
                    f"  core_attainment       : {core['core_attainment']:.1%}",
                    f"  core_dominant_unit    : {dom}",
                    f"  peak_bw (per-core)    : {core['peak_bw_gb_s']:.2f} GB/s", "",
                    f"  {'Unit':>10}  {'Achieved':>12}  {'Ceiling':>12}  {'Ridge':>10}  {'Attain':>7}",
                    f"  {'-' * 10}  {'-' * 12}  {'-' * 12}  {'-' * 10}  {'-' * 7}"]
            for unit, u in core["units"].items():
                mark = " *" if unit == dom else "  "
                out.append(f"{mark} {unit:>10}  {u['achieved_gflops']:>10.2f} G  {u['ceiling_gflops']:>10.2f} G  "
                           f"{u['ridge']:>8.1f} F/B  {u['attainment']:>6.1%}")
            out.append(bar)
        return "\n".join(out)


# -- stick counting (the data-dependent input of the memory cost) ----------------

def unique_sticks_rows(starts_b, run_bytes: int) -> int:
    """Unique 128-byte sticks touched by byte runs [s, s + run_bytes) for s in `starts_b`."""
    import numpy as np
    s = np.asarray(starts_b, dtype=np.int64).reshape(-1)
    if s.size == 0 or run_bytes <= 0:
        return 0
    s0 = np.sort(s) // STICK_BYTES
    s1 = (np.sort(s) + run_bytes - 1) // STICK_BYTES
    # after sorting by start, a run adds the sticks above every earlier run's last stick
    prev = np.maximum.accumulate(np.concatenate([[-1], s1[:-1]]))
    return int(np.sum(np.maximum(0, s1 - np.maximum(s0, prev + 1) + 1)))


def unique_sticks_elems(byte_offsets) -> int:
    """Unique 128-byte sticks of single elements at the given byte offsets."""
    import numpy as np
    b = np.asarray(byte_offsets, dtype=np.int64).reshape(-1)
    return int(np.unique(b // STICK_BYTES).size) if b.size else 0
