"""GPU parity for linalg.reduce over other axes, several axes and all axes
(a scalar), linalg.generic with reduction iterators (one and two reduction
axes, permuted and computed indexing maps) and linalg.batch_matmul, on the
kernels whose oracle results tests/test_oracle_linalg_pins.py pins.

Folds and generic reductions are bit-exact (the GPU keeps the reference's
pairwise-halving order); batch_matmul is bit-exact on small-integer data and
within the north star's matmul tolerance (rtol 1e-2 / atol 1e-3) on random
data, where the f32 summation order of the products differs from NumPy's."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases as C

pytestmark = pytest.mark.gpu

_NP = {"f16": np.float16, "f32": np.float32}


def _both(src, fn, out, **kw):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: v.copy() for k, v in kw.items()})[out]
    g = KTIRInterpreter()
    g.load(src)
    print(fn, {k: v.shape for k, v in kw.items()}, flush=True)
    got = g.execute_function(fn, **kw)[out]
    print("  ", g.last_plan.mode, g.last_plan.counts(), flush=True)
    return got, ref


def _bits(got, ref):
    u = {2: np.uint16, 4: np.uint32}[got.dtype.itemsize]
    nan = np.isnan(got) & np.isnan(ref)
    np.testing.assert_array_equal(np.where(nan, 0, got.view(u)), np.where(nan, 0, ref.view(u)))


@pytest.mark.parametrize("shape,dims", [((3, 4, 2), (0, 2)), ((2, 3), (0, 1)), ((5, 6), (0,)), ((4, 3, 5), (1,)),
                                        ((3, 4, 6), (0, 1, 2)), ((4, 8), None), ((7, 5, 3), (2, 0)),
                                        ((16, 64), (0,)), ((8, 16, 32), (0, 2))])
@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_reduce_axes_bit_exact(shape, dims, dt):
    rng = np.random.default_rng(len(shape) * 7 + (len(dims) if dims else 0))
    src, fn, full, rfull = C.reduce_kernel(shape=shape, dims=dims, dt=dt, init=0.5, cores=4)
    x = (rng.standard_normal(full) * 10.0 ** rng.integers(-3, 4, full)).astype(_NP[dt])
    _bits(*_both(src, fn, "y_ptr", x_ptr=x, y_ptr=np.zeros(rfull, _NP[dt])))


def test_reduce_reference_golden_on_gpu():
    src, fn, full, rfull = C.reduce_kernel(shape=(3, 4, 2), dims=(0, 2), dt="f16", cores=2)
    x = np.ones(full, np.float16)
    x[0, :, 0], x[2, :, 0] = 10000, -10000
    x[3:] = np.arange(24).reshape(3, 4, 2)
    got, ref = _both(src, fn, "y_ptr", x_ptr=x, y_ptr=np.zeros(rfull, np.float16))
    np.testing.assert_array_equal(got, [0, 0, 0, 0, 51, 63, 75, 87])
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("combiner", ["arith.maximumf", "arith.mulf", "arith.minnumf"])
def test_reduce_other_combiners_region_form_bit_exact(combiner):
    rng = np.random.default_rng(3)
    src, fn, full, rfull = C.reduce_kernel(shape=(3, 5, 4), dims=(0, 2), dt="f32", init=1.0, cores=4,
                                           combiner=combiner, region=True)
    x = rng.uniform(0.5, 1.5, full).astype(np.float32)
    x[1, 2, 3] = np.nan
    _bits(*_both(src, fn, "y_ptr", x_ptr=x, y_ptr=np.zeros(rfull, np.float32)))


def test_generic_reduction_reference_contraction():
    src, fn, a, b, c = C.generic_contraction()
    A = np.arange(np.prod(a)).reshape(a).astype(np.float32)
    B = np.arange(np.prod(b)).reshape(b).astype(np.float32)
    got, ref = _both(src, fn, "c_ptr", a_ptr=A, b_ptr=B, c_ptr=np.ones(c, np.float32))
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got[:3], A[:3].astype(np.int64) @ B[:5].astype(np.int64) + 1)


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_generic_reduction_fold_order_bit_exact(dt):
    rng = np.random.default_rng(4)
    src, fn, a, b, c = C.generic_contraction(M=8, N=16, K=32, dt=dt, cores=4)
    A = (rng.standard_normal(a) * 10.0 ** rng.integers(-2, 3, a)).astype(_NP[dt])
    B = (rng.standard_normal(b) * 10.0 ** rng.integers(-2, 3, b)).astype(_NP[dt])
    C0 = rng.standard_normal(c).astype(_NP[dt])
    _bits(*_both(src, fn, "c_ptr", a_ptr=A, b_ptr=B, c_ptr=C0))


def test_generic_max_reduction_bit_exact():
    rng = np.random.default_rng(6)
    src, fn, a, b, c = C.generic_contraction(M=4, N=8, K=16, dt="f32", cores=2, combiner="arith.maximumf")
    A, B, C0 = (rng.standard_normal(s).astype(np.float32) for s in (a, b, c))
    _bits(*_both(src, fn, "c_ptr", a_ptr=A, b_ptr=B, c_ptr=C0))


def test_generic_two_reduction_axes_permuted_and_computed_maps():
    src, fn, full = C.generic_stick_contraction(cores=4)
    rng = np.random.default_rng(7)
    A = np.arange(np.prod(full["a"])).reshape(full["a"]).astype(np.float32)
    W = np.arange(np.prod(full["w"])).reshape(full["w"]).astype(np.float32)
    got, ref = _both(src, fn, "c_ptr", a_ptr=A, w_ptr=W, c_ptr=np.zeros(full["c"], np.float32))
    np.testing.assert_array_equal(got, ref)
    A = rng.standard_normal(full["a"]).astype(np.float32)
    W = rng.standard_normal(full["w"]).astype(np.float32)
    _bits(*_both(src, fn, "c_ptr", a_ptr=A, w_ptr=W, c_ptr=rng.standard_normal(full["c"]).astype(np.float32)))


@pytest.mark.parametrize("out_dt", ["f32", "f16"])
def test_batch_matmul_small_integers_bit_exact(out_dt):
    rng = np.random.default_rng(5)
    src, fn, a, b, c = C.batch_matmul(Bt=2, M=16, N=32, K=64, cores=4, out_dt=out_dt)
    A = rng.integers(-4, 5, a).astype(np.float16)
    B = rng.integers(-4, 5, b).astype(np.float16)
    C0 = rng.integers(-50, 50, c).astype(_NP[out_dt])
    got, ref = _both(src, fn, "c_ptr", a_ptr=A, b_ptr=B, c_ptr=C0)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_batch_matmul_random_within_tolerance(dt):
    from oracle.interp import bf16_bits
    rng = np.random.default_rng(8)
    src, fn, a, b, c = C.batch_matmul(Bt=3, M=32, N=64, K=128, dt=dt, cores=2, out_dt="f32")
    A = rng.standard_normal(a).astype(np.float32) / 8
    B = rng.standard_normal(b).astype(np.float32) / 8
    A, B = (x.astype(np.float16) if dt == "f16" else bf16_bits(x) for x in (A, B))
    C0 = rng.standard_normal(c).astype(np.float32)
    got, ref = _both(src, fn, "c_ptr", a_ptr=A, b_ptr=B, c_ptr=C0)
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-3)


def test_tensor_slices_generate_from_elements_reshape_bit_exact():
    from tests.test_oracle_linalg_pins import tensor_ops_brute
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw = C.tensor_ops()
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: v.copy() for k, v in kw.items()})
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function(fn, **kw)
    print(fn, g.last_plan.mode, g.last_plan.counts(), flush=True)
    for k, v in tensor_ops_brute(kw).items():
        np.testing.assert_array_equal(got[k], ref[k], err_msg=k)
        np.testing.assert_array_equal(got[k], v, err_msg=k)


@pytest.mark.parametrize("rows,cols,rblk", [(16, 256, 4), (64, 16, 16), (64, 512, 8)])
def test_softmax_rows_that_expose_the_broadcast_axis(rows, cols, rblk):
    """The oracle's closed-form softmax case on the GPU: exact where the
    closed form is exact (1 / k at the top entries, 0 elsewhere)."""
    from tests.test_oracle_linalg_pins import broadcast_softmax_rows
    src, fn, kw = C.softmax(rows=rows, cols=cols, cores=4, rblk=rblk)
    kw["x_ptr"] = broadcast_softmax_rows(rows, cols).astype(np.float16)
    got, ref = _both(src, fn, "y_ptr", **kw)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols,rblk", [(16, 512, 4), (64, 16, 16)])
def test_rmsnorm_constant_rows_column_weights_bit_exact(dt, rows, cols, rblk):
    from oracle.interp import bf16_bits
    c = np.array([(-1) ** r * 0.25 * (r % 16 + 1) * (1 + r // 16) for r in range(rows)])
    x = np.repeat(c[:, None], cols, axis=1)
    w = np.linspace(0.5, 1.5, cols)
    src, fn, kw = C.rmsnorm(rows=rows, cols=cols, cores=4, rblk=rblk, dt=dt)
    if dt == "f16":
        kw["x_ptr"], kw["w_ptr"] = x.astype(np.float16), w.astype(np.float16)
    else:
        kw["x_ptr"], kw["w_ptr"] = bf16_bits(x.astype(np.float32)), bf16_bits(w.astype(np.float32))
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})["y_ptr"]
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function(fn, **kw)["y_ptr"]
    np.testing.assert_array_equal(got, ref)
