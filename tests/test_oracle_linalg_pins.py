"""Oracle pins for linalg.reduce over other and several axes and to a
scalar, linalg.generic with reduction iterators, linalg.batch_matmul and
linalg.broadcast, each on small KTIR kernels run by the oracle:

* the reference's own expected values (tests/test_dialects_exec.py:856-1047,
  :1222-1330), including its strict-xfail tree-fold case whose result is
  0 where a sequential sum gives 1;
* a scalar brute force of the pairwise-halving fold on Python lists, with
  each combine rounded to the tile dtype, applied axis by axis (rightmost
  first), then the outs combine (dialects/linalg_ops.py:86-246);
* exact integer products for contractions and batch_matmul (every product
  and partial sum is an integer below 2^24, so any summation order gives
  the int64 result).
CPU only."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases as C

_NP = {"f16": np.float16, "f32": np.float32}


def _run(src, fn, **kw):
    o = OracleInterpreter()
    o.load(src)
    return o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})


def _fold_list(vals, op, dt):
    """Pairwise halving of a Python list: element i combines with i + n/2,
    an odd tail is carried; every combine rounds to dt."""
    while len(vals) > 1:
        h = len(vals) // 2
        vals = [_NP[dt](op(float(vals[i]), float(vals[h + i]))) for i in range(h)] + vals[2 * h:]
    return vals[0]


def _brute_reduce(x, dims, op, dt, init):
    """Fold axis by axis, rightmost first, then combine with init."""
    if dims is None:
        r = _fold_list(list(x.reshape(-1)), op, dt)
        return _NP[dt](op(float(r), float(init)))
    cur = x
    for d in sorted(dims, reverse=True):
        moved = np.moveaxis(cur, d, -1)
        out = np.empty(moved.shape[:-1], moved.dtype)
        for idx in np.ndindex(*moved.shape[:-1]):
            out[idx] = _fold_list(list(moved[idx]), op, dt)
        cur = out
    return np.vectorize(lambda v: _NP[dt](op(float(v), float(init))))(cur).astype(_NP[dt])


_OPS = {"arith.addf": lambda a, b: a + b, "arith.maximumf": max, "arith.mulf": lambda a, b: a * b}


@pytest.mark.parametrize("shape,dims", [((3, 4, 2), (0, 2)), ((2, 3), (0, 1)), ((5, 6), (0,)), ((4, 3, 5), (1,)),
                                        ((3, 4, 6), (0, 1, 2)), ((4, 8), None), ((7, 5, 3), (2, 0))])
@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_oracle_reduce_axes_against_brute_force(shape, dims, dt):
    rng = np.random.default_rng(len(shape) * 7 + (len(dims) if dims else 0))
    cores = 2
    src, fn, full, rfull = C.reduce_kernel(shape=shape, dims=dims, dt=dt, init=0.5, cores=cores)
    x = (rng.standard_normal(full) * 10.0 ** rng.integers(-3, 4, full)).astype(_NP[dt])
    got = _run(src, fn, x_ptr=x, y_ptr=np.zeros(rfull, _NP[dt]))["y_ptr"]
    for c in range(cores):
        blk = x[c * shape[0]:(c + 1) * shape[0]]
        want = _brute_reduce(blk, dims, _OPS["arith.addf"], dt, 0.5)
        n = 1 if np.ndim(want) == 0 else np.shape(want)[0]
        np.testing.assert_array_equal(got[c * n:(c + 1) * n].reshape(np.shape(want)), want)


def test_oracle_reduce_reference_golden_values():
    # (3, 4, 2) over dims [0, 2] with cancelling 10000 / -10000: the tree fold
    # gives 0 (the reference's strict xfail, tests/test_dialects_exec.py:980-995)
    src, fn, full, rfull = C.reduce_kernel(shape=(3, 4, 2), dims=(0, 2), dt="f16", cores=2)
    x = np.ones(full, np.float16)
    x[0, :, 0], x[2, :, 0] = 10000, -10000
    x[3:] = np.arange(24).reshape(3, 4, 2)
    got = _run(src, fn, x_ptr=x, y_ptr=np.zeros(rfull, np.float16))["y_ptr"]
    np.testing.assert_array_equal(got, [0, 0, 0, 0, 51, 63, 75, 87])
    # (2, 3) over [0, 1]: 15 (:920-930), a Python scalar stored through splat
    src, fn, full, rfull = C.reduce_kernel(shape=(2, 3), dims=(0, 1), dt="f16", cores=2)
    x = np.concatenate([np.arange(6).reshape(2, 3), np.ones((2, 3))]).astype(np.float16)
    np.testing.assert_array_equal(_run(src, fn, x_ptr=x, y_ptr=np.zeros(rfull, np.float16))["y_ptr"], [15, 6])
    # outs init 100 folds in: sum(1..4) -> 110 (:997-1010), explicit region form
    src, fn, full, rfull = C.reduce_kernel(shape=(1, 4), dims=(1,), dt="f16", init=100.0, cores=2, region=True)
    x = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float16)
    np.testing.assert_array_equal(_run(src, fn, x_ptr=x, y_ptr=np.zeros(rfull, np.float16))["y_ptr"], [110, 126])


@pytest.mark.parametrize("combiner", ["arith.maximumf", "arith.mulf"])
def test_oracle_reduce_other_combiners_against_brute_force(combiner):
    rng = np.random.default_rng(3)
    src, fn, full, rfull = C.reduce_kernel(shape=(3, 5, 4), dims=(0, 2), dt="f32", init=1.0, cores=2,
                                           combiner=combiner, region=True)
    x = rng.uniform(0.5, 1.5, full).astype(np.float32)
    got = _run(src, fn, x_ptr=x, y_ptr=np.zeros(rfull, np.float32))["y_ptr"]
    want = np.concatenate([_brute_reduce(x[c * 3:(c + 1) * 3], (0, 2), _OPS[combiner], "f32", 1.0) for c in (0, 1)])
    np.testing.assert_array_equal(got, want)


def test_oracle_generic_reduction_reference_contraction():
    """A @ B + C with arange data (tests/test_dialects_exec.py:1222-1277), exact."""
    src, fn, a, b, c = C.generic_contraction()
    A = np.arange(np.prod(a)).reshape(a).astype(np.float32)
    B = np.arange(np.prod(b)).reshape(b).astype(np.float32)
    got = _run(src, fn, a_ptr=A, b_ptr=B, c_ptr=np.ones(c, np.float32))["c_ptr"]
    for k in range(2):
        want = A[3 * k:3 * k + 3].astype(np.int64) @ B[5 * k:5 * k + 5].astype(np.int64) + 1
        np.testing.assert_array_equal(got[3 * k:3 * k + 3], want)


def test_oracle_generic_reduction_fold_order_against_brute_force():
    """The body runs once on the iteration space with outs bound to the
    combiner's identity, the products are then tree-folded over the
    reduction axis and combined with outs (dialects/linalg_ops.py:531-585):
    on f16 data of spread magnitudes the fold order shows."""
    rng = np.random.default_rng(4)
    M, N, K = 4, 6, 16
    src, fn, a, b, c = C.generic_contraction(M=M, N=N, K=K, dt="f16")
    A = (rng.standard_normal(a) * 10.0 ** rng.integers(-2, 3, a)).astype(np.float16)
    B = (rng.standard_normal(b) * 10.0 ** rng.integers(-2, 3, b)).astype(np.float16)
    C0 = rng.standard_normal(c).astype(np.float16)
    got = _run(src, fn, a_ptr=A, b_ptr=B, c_ptr=C0)["c_ptr"]
    for k in range(2):
        Ab, Bb = A[M * k:M * (k + 1)], B[K * k:K * (k + 1)]
        for i in range(M):
            for j in range(N):
                prods = [np.float16(np.float16(float(Ab[i, t]) * float(Bb[t, j])) + np.float16(0.0))
                         for t in range(K)]
                s = _fold_list(prods, _OPS["arith.addf"], "f16")
                want = np.float16(float(s) + float(C0[M * k + i, j]))
                assert got[M * k + i, j].view(np.uint16) == want.view(np.uint16), (k, i, j)


def test_oracle_generic_two_reduction_axes_permuted_and_computed_maps():
    """The reference's issue-174 stick contraction (tests/test_dialects_exec.py:1279-1330): exact."""
    src, fn, full = C.generic_stick_contraction()
    A = np.arange(np.prod(full["a"])).reshape(full["a"]).astype(np.float32)
    W = np.arange(np.prod(full["w"])).reshape(full["w"]).astype(np.float32)
    got = _run(src, fn, a_ptr=A, w_ptr=W, c_ptr=np.zeros(full["c"], np.float32))["c_ptr"]
    for k in range(2):
        a = A[2 * k:2 * k + 2].astype(np.int64)
        w = W[k:k + 1].reshape(1, 2, 4, 4).astype(np.int64)
        want = np.einsum("kmj,nkjo->nmo", a, w)
        np.testing.assert_array_equal(got[k:k + 1], want)


@pytest.mark.parametrize("out_dt", ["f32", "f16"])
def test_oracle_batch_matmul_exact(out_dt):
    """The reference's batch case (tests/test_dialects_exec.py:1037-1047) and
    small-integer batches of a non-square shape, against int64 products plus
    the outs accumulator."""
    src, fn, a, b, c = C.batch_matmul(Bt=3, M=2, N=2, K=2, cores=1, out_dt=out_dt)
    A = np.array([[[1, 2], [3, 4]], [[2, 0], [1, 3]], [[1, 1], [0, 2]]], np.float16)
    B = np.array([[[5, 6], [7, 8]], [[1, 2], [3, 4]], [[2, 3], [1, 0]]], np.float16)
    got = _run(src, fn, a_ptr=A, b_ptr=B, c_ptr=np.zeros(c, _NP[out_dt]))["c_ptr"]
    np.testing.assert_array_equal(got, np.einsum("bij,bjk->bik", A.astype(np.int64), B.astype(np.int64)))
    rng = np.random.default_rng(5)
    src, fn, a, b, c = C.batch_matmul(Bt=2, M=8, N=16, K=32, cores=2, out_dt=out_dt)
    A = rng.integers(-4, 5, a).astype(np.float16)
    B = rng.integers(-4, 5, b).astype(np.float16)
    C0 = rng.integers(-50, 50, c).astype(_NP[out_dt])
    got = _run(src, fn, a_ptr=A, b_ptr=B, c_ptr=C0)["c_ptr"]
    want = np.einsum("bij,bjk->bik", A.astype(np.int64), B.astype(np.int64)) + C0.astype(np.int64)
    np.testing.assert_array_equal(got, want)


def broadcast_softmax_rows(rows=16, cols=256):
    """Rows that make a wrong broadcast visible: row r holds r + 1 entries
    equal to its base and the rest 30 below it; the bases are -150, -50, 50,
    150 in turn, so the maximum of another row subtracted from this one
    overflows exp (inf / inf = NaN), and another row's sum gives the wrong
    fraction.  The exact result is 1 / (r + 1) at the r + 1 top entries and
    e^-30 / (r + 1) (0 in f16) elsewhere."""
    x = np.full((rows, cols), -30.0)
    for r in range(rows):
        x[r, np.arange(min(r + 1, cols)) * 7 % cols] = 0.0
        x[r] += -150.0 + 100.0 * (r % 4)
    return x


@pytest.mark.parametrize("rows,cols,rblk", [(16, 256, 4), (64, 16, 16)])
def test_oracle_softmax_config_closed_form_pins_broadcast(rows, cols, rblk):
    """The softmax config kernel (two row reductions broadcast back along
    dimension 1 by linalg.broadcast) against the closed form; the square
    16 x 16 blocks are where a broadcast along the wrong axis would not fail
    on shape and would transpose silently."""
    x = broadcast_softmax_rows(rows, cols).astype(np.float16)
    src, fn, kw = C.softmax(rows=rows, cols=cols, cores=4, rblk=rblk)
    kw["x_ptr"] = x
    got = _run(src, fn, **kw)["y_ptr"].astype(np.float64)
    for r in range(rows):
        top = np.zeros(cols, bool)
        top[np.arange(min(r + 1, cols)) * 7 % cols] = True
        np.testing.assert_array_equal(got[r, top], np.float16(1.0 / top.sum()))
        np.testing.assert_array_equal(got[r, ~top], 0.0)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols,rblk", [(16, 512, 4), (64, 16, 16)])
def test_oracle_rmsnorm_config_closed_form_pins_broadcast(dt, rows, cols, rblk):
    """The RMSNorm config kernel on rows that are each one constant c_r
    (a different one per row) with a weight that varies by column: every
    output is c_r w_j / sqrt(c_r^2 + eps), within one ulp of the output type.
    The mean of squares is exact here (equal terms, pairwise halving), so a
    broadcast of the row scale or of w along the wrong axis fails."""
    from oracle.interp import bf16_bits, bf16_from_bits
    c = np.array([(-1) ** r * 0.25 * (r % 16 + 1) * (1 + r // 16) for r in range(rows)])
    w = np.linspace(0.5, 1.5, cols)
    x = np.repeat(c[:, None], cols, axis=1)
    src, fn, kw = C.rmsnorm(rows=rows, cols=cols, cores=4, rblk=rblk, dt=dt)
    if dt == "f16":
        kw["x_ptr"], kw["w_ptr"] = x.astype(np.float16), w.astype(np.float16)
        cq, wq = kw["x_ptr"][:, 0].astype(np.float64), kw["w_ptr"].astype(np.float64)
    else:
        kw["x_ptr"], kw["w_ptr"] = bf16_bits(x.astype(np.float32)), bf16_bits(w.astype(np.float32))
        cq, wq = bf16_from_bits(kw["x_ptr"][:, 0]).astype(np.float64), bf16_from_bits(kw["w_ptr"]).astype(np.float64)
    got = _run(src, fn, **kw)["y_ptr"]
    want = cq[:, None] * wq[None, :] / np.sqrt(cq[:, None] ** 2 + 1e-6)
    if dt == "f16":
        g16, w16 = got, want.astype(np.float16)
        d = np.abs(g16.view(np.int16).astype(np.int32) - w16.view(np.int16).astype(np.int32))
    else:
        w16 = bf16_bits(want.astype(np.float32))
        d = np.abs(got.view(np.int16).astype(np.int32) - w16.view(np.int16).astype(np.int32))
    assert d.max() <= 1, d.max()


def tensor_ops_brute(kw, cores=4):
    """The tensor_ops kernel's outputs by NumPy slicing, per core (the
    reference's semantics, dialects/tensor_ops.py:133-359)."""
    X = kw["x_ptr"]
    want = {k: np.zeros_like(v) for k, v in kw.items() if k != "x_ptr"}
    i, j = np.meshgrid(np.arange(4), np.arange(16), indexing="ij")
    for c in range(cores):
        Xc = X[4 * c:4 * c + 4]
        k, k2 = c % 4, 2 * (c % 4)
        want["a_ptr"][2 * c:2 * c + 2] = Xc[1:3, 2:10]
        want["b_ptr"][5 * c:5 * c + 5] = Xc[k, 1:14:3]
        want["c_ptr"][4 * c + 2:4 * c + 4, k2:k2 + 8] = Xc[1:3, 2:10]
        want["g_ptr"][4 * c:4 * c + 4] = (i >= j).astype(np.float16)
        want["r_ptr"][2 * c:2 * c + 2] = Xc.reshape(2, 32)
    return want


def test_oracle_tensor_slices_generate_from_elements_reshape():
    """extract_slice (static; dynamic offset with stride 3, rank-reduced),
    insert_slice at a dynamic offset, generate (the reference's 2-d cmpi
    case, tests/test_dialects_exec.py:1700-1716), from_elements feeding
    reshape, each against NumPy slicing."""
    src, fn, kw = C.tensor_ops()
    got = _run(src, fn, **kw)
    for k, v in tensor_ops_brute(kw).items():
        np.testing.assert_array_equal(got[k], v, err_msg=k)
