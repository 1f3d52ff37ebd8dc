"""The latency model on real runs (GPU): the quantities the executor feeds
it, checked against what the kernels' shapes and data fix.  The expectations
restate the reference's tests (tests/test_latency.py:306-316 vector_add
bytes, :708-746 softmax, :899-929 matmul) on this repository's own
generated kernels."""
import math

import numpy as np
import pytest

from ktir_cpu_amd import HardwareConfig, KTIRInterpreter
from ktir_cpu_amd.latency import STICK_BYTES
from tests import _cases

pytestmark = pytest.mark.gpu


def _run(case, cfg, trace=False):
    src, fn, kw = case
    g = KTIRInterpreter(latency_config=cfg, trace_latency=trace)
    g.load(src)
    out = g.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})
    return g.get_latency_report(), out


def test_no_config_no_report_and_identical_results():
    case = _cases.vector_add(4096, 128, 32)
    g = KTIRInterpreter()
    g.load(case[0])
    plain = g.execute_function(case[1], **case[2])
    assert g.get_latency_report() is None
    rep, out = _run(case, HardwareConfig())
    for k in plain:
        np.testing.assert_array_equal(out[k], plain[k])
    assert rep is not None


def test_vector_add_bytes_and_flops():
    rep, _ = _run(_cases.vector_add(4096, 128, 32), HardwareConfig())
    assert len(rep.counters) == 32
    c0 = rep.counters[0]
    # 2 loads + 1 store of 128 f16 elements = 3 x 256 bytes
    assert c0.total_bytes == 768
    assert c0.total_flops >= 128
    assert rep.bottleneck == "memory"


@pytest.mark.parametrize("bw", [0.5, 2.0])
def test_memory_cycles_scale_with_bandwidth(bw):
    case = _cases.vector_add(4096, 128, 32)
    base, _ = _run(case, HardwareConfig(hbm_bandwidth_tb_s=1.0))
    scaled, _ = _run(case, HardwareConfig(hbm_bandwidth_tb_s=bw))
    assert scaled.counters[0].memory_cycles == pytest.approx(base.counters[0].memory_cycles / bw)


def test_matmul_entries_and_cycles():
    M = N = 256
    K, bm, bn, bk = 512, 128, 128, 64
    cfg = HardwareConfig()
    rep, _ = _run(_cases.gemm(M, N, K, bm, bn, bk, 2, 2), cfg, trace=True)
    assert len(rep.counters) == 4
    per = 2.0 * bm * bn * bk / cfg.systolic_flops_per_cycle
    for c in rep.counters.values():
        mm = [e for e in c.trace if e.op_type == "linalg.matmul"]
        assert len(mm) == K // bk                     # one matmul per K step of the core's one tile
        assert all(e.cycles == pytest.approx(per) for e in mm)
        # A and B tiles per step, C once: 128-byte rows are one stick each
        assert c.dram_bytes == (K // bk) * (bm * bk * 2 + bk * bn * 2) + bm * bn * 2
    rows4, _ = _run(_cases.gemm(M, N, K, bm, bn, bk, 2, 2), HardwareConfig(systolic_rows=4))
    assert rows4.counters[0].cycles_by_category["compute_matmul"] == pytest.approx(
        2 * rep.counters[0].cycles_by_category["compute_matmul"])


def test_softmax_exp_dominates():
    rows, cols, cores, rblk = 64, 256, 8, 4
    cfg = HardwareConfig()
    rep, _ = _run(_cases.softmax(rows, cols, cores, rblk), cfg, trace=True)
    assert len(rep.counters) == cores
    for c in rep.counters.values():
        assert c.compute_cycles > 0 and c.memory_cycles > 0
    c0 = rep.counters[0]
    by_op = {}
    for e in c0.trace:
        if e.category.startswith("compute_"):
            by_op[e.op_type] = by_op.get(e.op_type, 0.0) + e.cycles
    assert max(by_op, key=by_op.get) == "math.exp"
    one_pass = (rows // cores) * cols / cfg.simd_elements_per_cycle * cfg.transcendental_penalty
    assert one_pass * 0.99 <= by_op["math.exp"] <= one_pass * 2.5
    # the row max / row sum reductions charge their combiner per halving level:
    # (cols - 1) combines per row and reduction
    red = sum(e.cycles for e in c0.trace if e.op_type in ("arith.maximumf", "arith.addf"))
    assert red >= 2 * (rows // cores) * (cols - 1) / cfg.simd_elements_per_cycle * 0.99


def test_gather_bytes_from_device_offsets():
    """The indirect loads and stores charge the unique sticks of the rows the
    GPU gathered plus those of the index reads: recomputed here from the
    index values."""
    rows, dim, n_idx, cores, chunk = 1024, 32, 512, 4, 32
    case = _cases.gather_scatter_add(rows, dim, n_idx, cores, chunk)
    idx = case[2]["idx_ptr"]
    rep, _ = _run(case, HardwareConfig())
    per_core = n_idx // cores
    for c in range(cores):
        want = 0
        for ch in range(per_core // chunk):
            p0 = c * per_core + ch * chunk
            r = idx[p0:p0 + chunk].astype(np.int64)
            idx_sticks = len({(p * 4) // STICK_BYTES for p in range(p0, p0 + chunk)})
            tab = len({(int(x) * dim * 2 + b) // STICK_BYTES for x in r for b in (0, dim * 2 - 1)})
            out = len({(int(x) * dim * 4 + b) // STICK_BYTES for x in r for b in (0, dim * 4 - 1)})
            want += (tab + idx_sticks) + 2 * (out + idx_sticks)
        assert rep.counters[c].dram_bytes == want * STICK_BYTES, c


def test_report_text_and_summary():
    rep, _ = _run(_cases.vector_add(4096, 128, 32), HardwareConfig())
    s = str(rep)
    assert "Kernel cycles" in s and "Roofline: PER-CORE" in s
    d = rep.summary_dict()
    assert d["grid_cores"] == 32 and math.isclose(d["kernel_cycles"], rep.kernel_cycles)


@pytest.mark.parametrize("group_size,folds", [(None, 3), (2, 1)])
def test_ring_reduce_comm_charge(group_size, folds):
    """The reference's ring-reduce latency breakdown
    (tests/test_latency.py:2235-2420) on this repository's 4-core ring
    kernel: every core's reduce is charged (n - 1) x 256 ring bytes in the
    comm bucket (the ring spans the whole workgroup, whatever the groups),
    the combiner's linalg.add runs once per round that folds a producer of
    the core's group (3 in one group of 4, 1 in pairs), produce is free,
    and the results match the run without the model."""
    from tests.test_inter_tile import ring_inputs
    cfg = HardwareConfig()
    kw = {} if group_size is None else {"group_size": group_size}
    x = ring_inputs(kw, seed=4)
    case = (_cases.ring_reduce(**kw), "ring_reduce", {"in_ptr": x, "out_ptr": np.zeros_like(x)})
    rep, out = _run(case, cfg, trace=True)
    g = KTIRInterpreter()
    g.load(case[0])
    plain = g.execute_function("ring_reduce", in_ptr=x, out_ptr=np.zeros_like(x))
    np.testing.assert_array_equal(out["out_ptr"], plain["out_ptr"])
    ring = 3 * 128 * 2
    assert set(rep.counters) == {0, 1, 2, 3}
    for core, cc in rep.counters.items():
        ops = [t.op_type for t in cc.trace]
        assert ops.count("ktdp.inter_tile_produce") == 1 and ops.count("ktdp.inter_tile_reduce") == 1
        assert ops.count("linalg.add") == folds
        prod = next(t for t in cc.trace if t.op_type == "ktdp.inter_tile_produce")
        assert prod.cycles == 0 and prod.category == "zero"
        red = next(t for t in cc.trace if t.op_type == "ktdp.inter_tile_reduce")
        assert red.category == "comm" and red.cycles == pytest.approx(ring / cfg.ring_bytes_per_cycle)
        assert cc.comm_bytes == ring
        assert cc.comm_cycles == pytest.approx(ring / cfg.ring_bytes_per_cycle)
        # one 1 x 128 f16 load and one store: two sticks each
        assert cc.dram_bytes == 2 * 2 * STICK_BYTES
        assert cc.total_bytes == cc.dram_bytes + cc.comm_bytes
