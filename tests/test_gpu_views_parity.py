"""GPU parity for the general indirect path (direct_expr subscripts, a
permuted variables_space_order for gathers and colliding scatters, and the
two error paths) and for memory views with SSA sizes / strides and symbolic
coordinate sets, against the oracle, bit for bit.  The oracle is pinned on
the same kernels by brute force and the reference's own cases in
tests/test_oracle_views_pins.py."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases as C
from tests.test_oracle_views_pins import brute_perm_gather, brute_perm_scatter, perm_inputs

pytestmark = pytest.mark.gpu


def _both(src, fn, out, **kw):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})[out]
    g = KTIRInterpreter()
    g.load(src)
    print(fn, {k: getattr(v, "shape", v) for k, v in kw.items()}, flush=True)
    got = g.execute_function(fn, **kw)[out]
    print("  ", g.last_plan.mode, g.last_plan.counts(), flush=True)
    return got, ref


def test_direct_expr_gather_bit_exact():
    src, fn = C.iat_direct_expr(cores=4)
    X = np.arange(64 * 128, dtype=np.float16).reshape(64, 128)
    idx = np.array([3, 7, 50, 63, 0, 1, 62, 5, 9, 9, 9, 9, 63, 0, 31, 32], np.int32)
    got, ref = _both(src, fn, "y_ptr", x_ptr=X, i_ptr=idx, y_ptr=np.zeros((16, 60), np.float16))
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, np.array([[X[idx[e], 2 * m + 1] for m in range(60)] for e in range(16)]))


@pytest.mark.parametrize("vso", ["(d1, d0)", "(d0, d1)"])
@pytest.mark.parametrize("M,K", [(4, 8), (16, 32)])
def test_permuted_order_gather_bit_exact(vso, M, K):
    X, I1, I2, _ = perm_inputs(M, K, rows=64, cols=64, cores=4, seed=2)
    src, fn = C.iat_permuted(M=M, K=K, rows=64, cols=64, cores=4, vso=vso)
    got, ref = _both(src, fn, "y_ptr", x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=np.zeros((4 * M, K), np.float16))
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, brute_perm_gather(X, I1, I2, M, K, 4, vso))


@pytest.mark.parametrize("vso", ["(d1, d0)", "(d0, d1)"])
@pytest.mark.parametrize("M,K", [(4, 8), (16, 32)])
def test_permuted_order_scatter_last_writer_bit_exact(vso, M, K):
    X, I1, I2, Y = perm_inputs(M, K, rows=16, cols=16, cores=4, seed=3, hot=True)
    src, fn = C.iat_permuted(M=M, K=K, rows=16, cols=16, cores=4, vso=vso, scatter=True)
    got, ref = _both(src, fn, "x_ptr", x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=Y)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, brute_perm_scatter(X, I1, I2, Y, M, K, 4, vso))


def test_iat_error_paths_raise_before_any_launch():
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    X, I1, I2, Y = perm_inputs()
    for kw, match in ((dict(vso="(d0, d0)"), "permut"), (dict(scatter=True, store_shape=(32,)), "does not match")):
        src, fn = C.iat_permuted(**kw)
        g = KTIRInterpreter()
        g.load(src)
        with pytest.raises(ValueError, match=match):
            g.execute_function(fn, x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=Y)


@pytest.mark.parametrize("n,cores", [(256, 1), (512, 1), (1000, 1), (1024, 1), (2048, 2), (3000, 3)])
def test_dynamic_view_vector_add_bit_exact(n, cores):
    """Every core's tile starts inside the n-element allocations (a start
    past them would be another argument's memory or unmapped, as in the
    reference); positions past n read zero and their writes are dropped."""
    src, fn = C.dyn_vector_add(cores=cores)
    rng = np.random.default_rng(42)
    x, y = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    got, ref = _both(src, fn, "out_ptr", x_ptr=x, y_ptr=y, out_ptr=np.zeros(n, np.float32), n_elements=np.int32(n))
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, x + y)


@pytest.mark.parametrize("s0", [16, 32, 96])
@pytest.mark.parametrize("merge_rows", [False, True])
def test_dynamic_distributed_copy_bit_exact(s0, merge_rows):
    src, fn = C.dyn_distributed_copy(merge_rows=merge_rows)
    rng = np.random.default_rng(42)
    if merge_rows:
        a = rng.standard_normal((128, s0)).astype(np.float16)
        a0, a1 = a[:64], a[64:]
    else:
        a = rng.standard_normal((64, 2 * s0)).astype(np.float16)
        a0, a1 = a[:, :s0], a[:, s0:]
    got, ref = _both(src, fn, "b_ptr", a0_ptr=np.ascontiguousarray(a0), a1_ptr=np.ascontiguousarray(a1),
                     b_ptr=np.zeros_like(a), s0_in=np.int32(s0))
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, a)
