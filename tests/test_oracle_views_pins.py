"""Oracle pins for the general indirect path and for memory views with SSA
sizes / strides and symbolic coordinate sets (CPU only):

* direct_expr subscripts: the reference's case Y[e, m] = X[IDX[e], 2 m + 1]
  (tests/test_blocked_indirect_fast_path.py:360-391);
* a permuted variables_space_order: the points are visited in the order of
  the map's image (ops/memory_ops.py:491-508), which sets both the layout of
  the loaded values and the last-writer-wins order of a scatter; brute
  force over the points in that order;
* the two error paths: a non-permutation order (:886-891) and a scatter
  whose tile shape differs from the access tile's (:937-941);
* dynamic views: the reference's own vector_add_dynamic parameters
  n = 256, 512, 1024 (tests/conftest.py:168-176) plus a ragged n, and the
  dynamic distributed copies with s0 = 16, 32 (tests/test_examples.py:248-308),
  against the closed forms (x + y; B = A)."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases as C


def _run(src, fn, **kw):
    o = OracleInterpreter()
    o.load(src)
    return o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})


def perm_inputs(M=4, K=8, rows=16, cols=16, cores=2, seed=0, hot=False):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((rows, cols)).astype(np.float16)
    hi = 3 if hot else rows
    I1 = rng.integers(0, hi, (M * cores, K)).astype(np.int32)
    I2 = rng.integers(0, 3 if hot else cols, (M * cores, K)).astype(np.int32)
    Y = rng.standard_normal((M * cores, K)).astype(np.float16)
    return X, I1, I2, Y


def perm_points(M, K, vso):
    pts = [(m, k) for m in range(M) for k in range(K)]
    key = {"(d1, d0)": lambda p: (p[1], p[0]), "(d0, d1)": lambda p: p}[vso]
    return sorted(pts, key=key)


def brute_perm_gather(X, I1, I2, M, K, cores, vso):
    out = np.zeros((M * cores, K), np.float16)
    for c in range(cores):
        vals = [X[I1[c * M + m, k], I2[c * M + m, k]] for m, k in perm_points(M, K, vso)]
        out[c * M:(c + 1) * M] = np.array(vals, np.float16).reshape(M, K)
    return out


def brute_perm_scatter(X, I1, I2, Y, M, K, cores, vso):
    X = X.copy()
    for c in range(cores):
        v = (Y[c * M:(c + 1) * M].astype(np.float32) * 2).astype(np.float16).reshape(-1)
        for t, (m, k) in enumerate(perm_points(M, K, vso)):
            X[I1[c * M + m, k], I2[c * M + m, k]] = v[t]
    return X


def test_oracle_direct_expr_reference_case():
    src, fn = C.iat_direct_expr()
    X = np.arange(64 * 128, dtype=np.float16).reshape(64, 128)
    idx = np.array([3, 7, 50, 63, 0, 1, 62, 5], np.int32)
    got = _run(src, fn, x_ptr=X, i_ptr=idx, y_ptr=np.zeros((8, 60), np.float16))["y_ptr"]
    want = np.array([[X[idx[e], 2 * m + 1] for m in range(60)] for e in range(8)], np.float16)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("vso", ["(d1, d0)", "(d0, d1)"])
def test_oracle_permuted_order_gather_layout(vso):
    M, K = 4, 8
    X, I1, I2, _ = perm_inputs(M, K)
    src, fn = C.iat_permuted(M=M, K=K, vso=vso)
    got = _run(src, fn, x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=np.zeros((2 * M, K), np.float16))["y_ptr"]
    np.testing.assert_array_equal(got, brute_perm_gather(X, I1, I2, M, K, 2, vso))


@pytest.mark.parametrize("vso", ["(d1, d0)", "(d0, d1)"])
def test_oracle_permuted_order_scatter_last_writer(vso):
    """Colliding targets (three rows x three columns for 64 points): the last
    point in the map's order writes, and element t of the tile goes to the
    t-th point in that order."""
    M, K = 4, 8
    X, I1, I2, Y = perm_inputs(M, K, hot=True, seed=1)
    src, fn = C.iat_permuted(M=M, K=K, vso=vso, scatter=True)
    got = _run(src, fn, x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=Y)["x_ptr"]
    np.testing.assert_array_equal(got, brute_perm_scatter(X, I1, I2, Y, M, K, 2, vso))
    if vso == "(d1, d0)":
        assert not np.array_equal(got, brute_perm_scatter(X, I1, I2, Y, M, K, 2, "(d0, d1)"))


def test_oracle_iat_error_paths():
    X, I1, I2, Y = perm_inputs()
    src, fn = C.iat_permuted(vso="(d0, d0)")
    with pytest.raises(ValueError, match="permut"):
        _run(src, fn, x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=Y)
    src, fn = C.iat_permuted(scatter=True, store_shape=(32,))
    with pytest.raises(ValueError, match="does not match"):
        _run(src, fn, x_ptr=X, i1_ptr=I1, i2_ptr=I2, y_ptr=Y)


@pytest.mark.parametrize("n", [256, 512, 1000, 1024])
def test_oracle_dynamic_view_vector_add(n):
    src, fn = C.dyn_vector_add()
    rng = np.random.default_rng(42)
    x, y = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    got = _run(src, fn, x_ptr=x, y_ptr=y, out_ptr=np.zeros(n, np.float32), n_elements=np.int32(n))["out_ptr"]
    np.testing.assert_array_equal(got, x + y)


@pytest.mark.parametrize("s0", [16, 32])
@pytest.mark.parametrize("merge_rows", [False, True])
def test_oracle_dynamic_distributed_copy(s0, merge_rows):
    src, fn = C.dyn_distributed_copy(merge_rows=merge_rows)
    rng = np.random.default_rng(42)
    if merge_rows:
        a = rng.standard_normal((128, s0)).astype(np.float16)
        a0, a1 = a[:64], a[64:]
    else:
        a = rng.standard_normal((64, 2 * s0)).astype(np.float16)
        a0, a1 = a[:, :s0], a[:, s0:]
    got = _run(src, fn, a0_ptr=np.ascontiguousarray(a0), a1_ptr=np.ascontiguousarray(a1), b_ptr=np.zeros_like(a),
               s0_in=np.int32(s0))["b_ptr"]
    np.testing.assert_array_equal(got, a)
