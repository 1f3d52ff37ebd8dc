"""The latency model's arithmetic on the host (no GPU): cost rules, stick
counting, the report and its roofline, each pinned by a closed form or a
brute-force count (reference latency.py:289-846)."""
import itertools

import numpy as np
import pytest

from ktir_cpu_amd.latency import (STICK_BYTES, CoreLatencyCounters, ExecutionModel, HardwareConfig, LatencyReport,
                                  LatencyTracker, category_of, unique_sticks_elems, unique_sticks_rows)


def test_category_table():
    # the reference registry's categories (dialects/*_ops.py @register(latency_category=...))
    assert category_of("arith.addf") == "compute_float"
    assert category_of("arith.maximumf") == "compute_float"
    assert category_of("arith.select") == "compute_float"
    assert category_of("arith.cmpf") == "compute_float"
    assert category_of("arith.cmpi") == "compute_int"
    assert category_of("arith.addi") == "compute_int"
    assert category_of("math.exp") == "compute_transcendental"
    assert category_of("math.rsqrt") == "compute_transcendental"
    assert category_of("math.powf") == "compute_transcendental"
    assert category_of("math.absf") == "compute_float"
    assert category_of("math.fma") == "compute_float"
    assert category_of("linalg.generic") == "compute_float"
    assert category_of("linalg.matmul") == "compute_matmul"
    assert category_of("ktdp.load") == "memory" and category_of("ktdp.store") == "memory"
    assert category_of("ktdp.inter_tile_reduce") == "comm"
    for free in ("arith.extf", "arith.truncf", "arith.constant", "linalg.reduce", "scf.for", "tensor.splat",
                 "ktdp.construct_access_tile"):
        assert category_of(free) == "zero"


def test_cost_formulas():
    cfg = HardwareConfig(hbm_bandwidth_tb_s=0.256, clock_ghz=2.0, simd_elements_per_cycle=32, systolic_rows=4,
                         transcendental_penalty=5, ring_bandwidth_tb_s=0.05)
    t = LatencyTracker(cfg)
    t.set_cores_active(16)
    bw = 0.256e12 / 2e9 / 16                      # bytes per cycle per core
    assert t.cost("ktdp.load", nbytes=4096) == ("memory", pytest.approx(4096 / bw), 0.0, 4096)
    cat, cyc, fl, b = t.cost("linalg.matmul", mnk=(32, 64, 16))
    assert (cat, fl, b) == ("compute_matmul", 2.0 * 32 * 64 * 16, 0)
    assert cyc == pytest.approx(2.0 * 32 * 64 * 16 / (2 * 32 * 4))
    assert t.cost("arith.mulf", n_elems=1000) == ("compute_float", pytest.approx(1000 / 32), 1000.0, 0)
    assert t.cost("math.exp", n_elems=1000) == ("compute_transcendental", pytest.approx(1000 / 32 * 5), 1000.0, 0)
    assert t.cost("arith.addi", n_elems=1) == ("compute_int", 0.0, 0.0, 0)     # scalar index math is free
    assert t.cost("arith.addi", n_elems=64) == ("compute_int", 2.0, 64.0, 0)
    assert t.cost("ktdp.inter_tile_reduce", nbytes=1000)[1] == pytest.approx(1000 / (0.05e12 / 2e9))
    assert t.cost("arith.extf", n_elems=10 ** 6) == ("zero", 0.0, 0.0, 0)


def _brute_rows(starts, run):
    return len({b // STICK_BYTES for s in starts for b in range(s, s + run)})


def test_unique_sticks_against_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = int(rng.integers(1, 12))
        run = int(rng.integers(1, 700))
        starts = rng.integers(0, 3000, n)
        assert unique_sticks_rows(starts, run) == _brute_rows(starts.tolist(), run)
    b = rng.integers(0, 10000, 300)
    assert unique_sticks_elems(b) == len(set((b // STICK_BYTES).tolist()))
    assert unique_sticks_rows(np.array([], np.int64), 64) == 0
    # 128 f16 elements aligned = 2 sticks; 3 such runs back to back = 6
    assert unique_sticks_rows(np.array([0, 256, 512]), 256) == 6


def _counters(compute_f=0.0, transc=0.0, matmul=0.0, mem=0.0, comm=0.0, flops=0.0, dram=0):
    c = CoreLatencyCounters()
    if compute_f:
        c.record("compute_float", compute_f, "arith.addf", flops=flops)
    if transc:
        c.record("compute_transcendental", transc, "math.exp")
    if matmul:
        c.record("compute_matmul", matmul, "linalg.matmul", flops=flops)
    if mem or dram:
        c.record("memory", mem, "ktdp.load", nbytes=dram)
    if comm:
        c.record("comm", comm, "ktdp.inter_tile_reduce", nbytes=8)
    return c


def test_pipeline_models_and_bottleneck():
    cfg = HardwareConfig(num_cores=4)
    counters = {0: _counters(compute_f=100, mem=70, comm=50), 1: _counters(compute_f=10, mem=300)}
    serial = LatencyReport(cfg, counters)
    assert serial.kernel_cycles == 310 and serial.bottleneck == "memory"
    over = LatencyReport(cfg, counters, ExecutionModel(pipeline="overlapped"))
    assert over.kernel_cycles == 300                     # core 1: max(10, 300 + 0)
    three = LatencyReport(cfg, counters, ExecutionModel(pipeline="overlapped_3way"))
    assert three.kernel_cycles == 300
    assert serial.kernel_time_us == pytest.approx(310 / 1e3)
    s = serial.summary_dict()
    assert s["grid_cores"] == 2 and [p["total_cycles"] for p in s["per_core"]] == [220, 310]


def test_roofline_closed_forms():
    cfg = HardwareConfig(num_cores=4, clock_ghz=1.0, hbm_bandwidth_tb_s=0.128, simd_elements_per_cycle=64)
    # two equal cores: 640 float FLOPs in 10 compute cycles, 1280 HBM bytes in 40 memory cycles
    counters = {k: _counters(compute_f=10, mem=40, flops=640, dram=1280) for k in range(2)}
    r = LatencyReport(cfg, counters)
    chip = r.chip_roofline()
    elapsed = 50 / 1e9
    assert chip["AI"] == pytest.approx(1280 / 2560)
    assert chip["dominant_unit"] == "simd"
    assert chip["compute_throughput"] == pytest.approx((1280 / elapsed) / (64e9 * 4))
    assert chip["dram_throughput"] == pytest.approx(2560 / (0.128e12 * elapsed))
    assert chip["mean_core_active_frac"] == pytest.approx(100 / (4 * 50))
    assert chip["grid_coverage"] == pytest.approx(0.5) and chip["cores_active"] == 2
    core = r.core_roofline()
    assert core["peak_bw_gb_s"] == pytest.approx(0.128e12 / 2 / 1e9)
    assert core["units"]["simd"]["AI"] == pytest.approx(0.5)
    assert core["units"]["simd"]["ceiling_gflops"] == pytest.approx(min(64.0, 64.0 * 0.5))
    # the dominant unit is decided by chip-wide cycles, not FLOPs
    mixed = {0: _counters(compute_f=5, matmul=1000, flops=10), 1: _counters(compute_f=5000, flops=10)}
    assert LatencyReport(cfg, mixed).chip_roofline()["dominant_unit"] == "simd"
    assert "Roofline: CHIP-LEVEL" in str(r) and "KTIR Latency Estimation Report" in str(r)


def test_empty_report():
    r = LatencyReport(HardwareConfig(), {})
    assert r.kernel_cycles == 0.0 and r.bottleneck == "none" and r.roofline() == {}
    assert "KTIR Latency Estimation Report" in str(r)


def test_execution_model_validation():
    with pytest.raises(NotImplementedError):
        ExecutionModel(bw_sharing="static")
    with pytest.raises(ValueError):
        ExecutionModel(bw_sharing="other")


def test_tracker_trace_and_reset():
    t = LatencyTracker(HardwareConfig(), trace=True)
    t.record_op(3, "math.exp", n_elems=128)
    t.record_op(3, "scf.yield")
    assert [e.op_type for e in t.counters[3].trace] == ["math.exp", "scf.yield"]
    assert t.counters[3].cycles_by_category["compute_transcendental"] == pytest.approx(128 / 64 * 4)
    t.reset()
    assert t.counters == {}


@pytest.mark.parametrize("n", [1, 2, 3, 5, 4096, 4097])
def test_fold_level_sizes_sum(n):
    """The combiner runs on n//2, then on the carried halves, ...: the element
    counts charged sum to n - 1 per row (one combine per removed element)."""
    total, m = 0, n
    while m > 1:
        total += m // 2
        m = m // 2 + m % 2
    assert total == n - 1
