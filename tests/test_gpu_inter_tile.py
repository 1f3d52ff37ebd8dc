"""ktdp.inter_tile_produce / inter_tile_reduce on the GPU, bit-exact against
the oracle (reference ops/comm_ops.py:229-345, dialects/ktdp_ops.py:951-1230):
group sums and maxima over contiguous, paired and strided groups, the ring's
fold order where f16 rounding shows it, a reduce inside an scf.for, and a
2 x 2 RMSNorm whose rows cross a distributed view (one half in core 1's LX)
and whose mean square is folded across the column partners."""
import numpy as np
import pytest

from tests import _cases
from tests.test_inter_tile import (FOLD_WANT, FOLD_X, VARIANTS, oracle_ring, oracle_rmsnorm_2x2, ring_expected,
                                   ring_inputs, rms_args, rms_inputs, rms_model, RMS_H, RMS_ROWS)

pytestmark = pytest.mark.gpu


def gpu_ring(kw, x):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    interp = KTIRInterpreter()
    interp.load(_cases.ring_reduce(**kw))
    out = interp.execute_function("ring_reduce", in_ptr=x, out_ptr=np.zeros_like(x))["out_ptr"]
    return out, interp.last_plan


@pytest.mark.parametrize("name,kw", VARIANTS, ids=[v[0] for v in VARIANTS])
def test_ring_reduce_groups(name, kw):
    print(f"[ring] {name}", flush=True)
    x = ring_inputs(kw, seed=1)
    got, plan = gpu_ring(kw, x)
    np.testing.assert_array_equal(got, oracle_ring(kw, x))
    np.testing.assert_array_equal(got, ring_expected(kw, x))
    assert plan.mode == "lockstep"


@pytest.mark.parametrize("name,kw", VARIANTS[:3], ids=[v[0] for v in VARIANTS[:3]])
def test_ring_reduce_random_f16_bit_exact(name, kw):
    """Values where every fold rounds: the GPU must fold in the ring's order."""
    print(f"[ring] random {name}", flush=True)
    n = kw.get("n_cores", 4)
    x = (np.random.default_rng(5).standard_normal((n, 128)) * 100).astype(np.float16)
    got, _ = gpu_ring(kw, x)
    np.testing.assert_array_equal(got, oracle_ring(kw, x))


def test_ring_fold_order():
    print("[ring] fold order", flush=True)
    got, _ = gpu_ring({}, FOLD_X)
    np.testing.assert_array_equal(got, FOLD_WANT[:, None].repeat(128, 1))


def test_ring_reduce_by_one_core_is_refused():
    """Only core 0 reaches the reduce (the reference deadlocks): refused
    before the reduce runs, with no GPU work left waiting."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    interp = KTIRInterpreter()
    interp.load(_cases.ring_reduce(only_core0=True))
    x = ring_inputs({})
    with pytest.raises(NotImplementedError):
        interp.execute_function("ring_reduce", in_ptr=x, out_ptr=np.zeros_like(x))


def gpu_rmsnorm_2x2(X, W):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    interp = KTIRInterpreter()
    interp.load(_cases.rmsnorm_2x2(RMS_ROWS, RMS_H))
    orig = interp._prepare_execution

    def prepare_and_seed(grid):
        orig(grid)
        interp.memory.get_lx(1).write(0, np.ascontiguousarray(X[:, RMS_H // 2:]).reshape(-1))

    interp._prepare_execution = prepare_and_seed
    out = interp.execute_function("rmsnorm_2x2", **rms_args(X, W))
    return np.concatenate([out["Y0"], out["Y1"]], 1), interp


def test_rmsnorm_2x2_distributed_ring():
    print("[ring] rmsnorm 2x2", flush=True)
    X, W = rms_inputs()
    Y, interp = gpu_rmsnorm_2x2(X, W)
    np.testing.assert_array_equal(Y, oracle_rmsnorm_2x2(X, W))
    np.testing.assert_allclose(Y.astype(np.float64), rms_model(X, W), rtol=1e-2, atol=1e-2)
    # core 1's LX still holds the right half of X
    got_lx = interp.memory.get_lx(1).read(0, RMS_ROWS * RMS_H // 2, "f16")
    np.testing.assert_array_equal(got_lx, np.ascontiguousarray(X[:, RMS_H // 2:]).reshape(-1))


def test_splitk_pv_strided_groups():
    """Split-K decode P @ V over a [2, 4] grid with strided reduce groups:
    integer data (every product, partial and fold exact) must match the
    integer product; random data the oracle (rtol 1e-2 / atol 1e-3: the f32
    summation order inside each partial's matmul differs) and P @ V at the
    reference's split-K tolerance."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    from tests.test_inter_tile import oracle_splitk, splitk_inputs
    print("[ring] split-K P@V", flush=True)

    def run(P, V):
        g = KTIRInterpreter()
        g.load(_cases.splitk_pv(P.shape[1], V.shape[1]))
        return g.execute_function("splitk_pv", p_ptr=P, v_ptr=V, c_ptr=np.zeros((1, V.shape[1]), np.float16))["c_ptr"]

    Pi = np.random.default_rng(1).integers(-2, 3, (1, 1024)).astype(np.float16)
    Vi = np.random.default_rng(2).integers(-2, 3, (1024, 128)).astype(np.float16)
    np.testing.assert_array_equal(run(Pi, Vi), (Pi.astype(np.int64) @ Vi.astype(np.int64)).astype(np.float16))
    P, V = splitk_inputs()
    C = run(P, V)
    np.testing.assert_allclose(C.astype(np.float32), oracle_splitk(P, V).astype(np.float32), rtol=1e-2, atol=1e-3)
    np.testing.assert_allclose(C.astype(np.float32), P.astype(np.float32) @ V.astype(np.float32), rtol=2e-2, atol=2e-1)


def test_ffn_swiglu_4core():
    """SwiGLU FFN with the hidden dimension split over 4 cores and the
    partials summed by the ring reduce: against the oracle (f16 matmuls:
    rtol 1e-2 / atol 1e-3 over the f32 summation order) and a float64 model."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    from tests.test_inter_tile import ffn_inputs, ffn_model, oracle_ffn
    print("[ring] ffn swiglu", flush=True)
    x, wg, wu, wd = ffn_inputs()
    g = KTIRInterpreter()
    g.load(_cases.ffn_swiglu_4core())
    out = g.execute_function("ffn_swiglu", x_ptr=x, wg_ptr=wg, wu_ptr=wu, wd_ptr=wd, out_ptr=np.zeros_like(x))
    y = out["out_ptr"].astype(np.float64)
    np.testing.assert_allclose(y, oracle_ffn(x, wg, wu, wd).astype(np.float64), rtol=1e-2, atol=1e-3)
    np.testing.assert_allclose(y, ffn_model(x, wg, wu, wd), rtol=2e-2, atol=2e-2)
