"""ktdp.inter_tile_produce / inter_tile_reduce in the oracle (no GPU).

The reference's ring (ops/comm_ops.py:229-345) folds, at core c, its own
partial and then the partials of cores c-1, c-2, ... (mod n) that produce
for c's group, as combine(acc, received), with cores scheduled as in
grid.py:524-623.  Pinned by: the exact group sums and maxima of small
integers (any fold order gives them); f16 values where the order shows, with
the expected results worked out by hand below; the reference's deadlock
error when one core alone reaches the reduce; and an RMSNorm whose mean
square crosses cores, against a float64 model.
"""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases

VARIANTS = [
    ("one_group", dict()),
    ("pairs", dict(group_size=2)),
    ("strided_8x4", dict(n_cores=8, group_size=4, strided=True)),
    ("max", dict(combiner="max")),
    ("inner_loop_3", dict(iters=3)),
]


def ring_inputs(kw, seed=0):
    n = kw.get("n_cores", 4)
    rng = np.random.default_rng(seed)
    return rng.integers(-8, 9, size=(n, 128)).astype(np.float16)


def ring_expected(kw, x):
    """Each core's group result from the group membership alone."""
    n = x.shape[0]
    gs = kw.get("group_size") or n
    ng = n // gs
    out = np.empty_like(x)
    for c in range(n):
        members = [i for i in range(n) if (i % ng == c % ng)] if kw.get("strided") else \
            [i for i in range(n) if i // gs == c // gs]
        v = x[members].astype(np.float64)
        out[c] = v.max(0) if kw.get("combiner") == "max" else v.sum(0) * max(1, kw.get("iters", 0))
    return out


def oracle_ring(kw, x):
    o = OracleInterpreter()
    o.load(_cases.ring_reduce(**kw))
    return o.execute_function("ring_reduce", in_ptr=x, out_ptr=np.zeros_like(x))["out_ptr"]


@pytest.mark.parametrize("name,kw", VARIANTS, ids=[v[0] for v in VARIANTS])
def test_oracle_ring_reduce_group_results(name, kw):
    x = ring_inputs(kw)
    np.testing.assert_array_equal(oracle_ring(kw, x), ring_expected(kw, x))


# partials 2048, 1, 1, 1 (f16 spacing at 2048 is 2, ties round to even):
#   core 0: 2048 +1 -> 2048, +1 -> 2048, +1 -> 2048            = 2048
#   core 1: 1 + 2048 -> 2048 (2049 ties to even), +1, +1        = 2048
#   core 2: 1 + 1 = 2, + 2048 = 2050, + 1 -> 2052 (2051 ties up) = 2052
#   core 3: 1 + 1 + 1 = 3, + 2048 -> 2052 (2051 ties up)        = 2052
FOLD_X = np.array([2048, 1, 1, 1], np.float16)[:, None].repeat(128, 1)
FOLD_WANT = np.array([2048, 2048, 2052, 2052], np.float16)


def test_oracle_ring_fold_order():
    out = oracle_ring({}, FOLD_X)
    np.testing.assert_array_equal(out, FOLD_WANT[:, None].repeat(128, 1))


def test_oracle_ring_deadlock_when_one_core_reduces():
    o = OracleInterpreter()
    o.load(_cases.ring_reduce(only_core0=True))
    x = ring_inputs({})
    with pytest.raises(RuntimeError, match="Deadlock detected: core 0 waiting on recv from core 3"):
        o.execute_function("ring_reduce", in_ptr=x, out_ptr=np.zeros_like(x))


RMS_ROWS, RMS_H = 16, 256


def rms_inputs(seed=3):
    rng = np.random.default_rng(seed)
    X = (rng.standard_normal((RMS_ROWS, RMS_H)) * 2).astype(np.float16)
    W = rng.uniform(0.5, 1.5, (1, RMS_H)).astype(np.float16)
    return X, W


def rms_args(X, W):
    h = RMS_H // 2
    z = np.zeros((RMS_ROWS, h), np.float16)
    return dict(X0=np.ascontiguousarray(X[:, :h]), W=W, Y0=z, Y1=z.copy(), eps=np.float16(1e-5))


def oracle_rmsnorm_2x2(X, W):
    o = OracleInterpreter()
    o.load(_cases.rmsnorm_2x2(RMS_ROWS, RMS_H))

    def seed(o):
        o.lxs[1].memory.write(0, np.ascontiguousarray(X[:, RMS_H // 2:]).reshape(-1))
        o.lxs[1].next_ptr = 1 << 20
    o.prepare_hook = seed
    out = o.execute_function("rmsnorm_2x2", **rms_args(X, W))
    return np.concatenate([out["Y0"], out["Y1"]], 1)


def rms_model(X, W):
    x = X.astype(np.float64)
    return x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-5) * W.astype(np.float64)


def test_oracle_rmsnorm_2x2_distributed():
    X, W = rms_inputs()
    Y = oracle_rmsnorm_2x2(X, W)
    np.testing.assert_allclose(Y.astype(np.float64), rms_model(X, W), rtol=1e-2, atol=1e-2)
    # a row whose right half is zero: only core (0, r) contributes to the fold
    X2 = X.copy()
    X2[3, RMS_H // 2:] = 0
    Y2 = oracle_rmsnorm_2x2(X2, W)
    np.testing.assert_allclose(Y2.astype(np.float64), rms_model(X2, W), rtol=1e-2, atol=1e-2)


def splitk_inputs(K=1024, N=128, seed=9):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((1, K)).astype(np.float16), rng.standard_normal((K, N)).astype(np.float16)


def oracle_splitk(P, V):
    o = OracleInterpreter()
    o.load(_cases.splitk_pv(P.shape[1], V.shape[1]))
    return o.execute_function("splitk_pv", p_ptr=P, v_ptr=V, c_ptr=np.zeros((1, V.shape[1]), np.float16))["c_ptr"]


def test_oracle_splitk_pv_strided_groups():
    """Split-K decode P @ V with strided reduce groups: C = P @ V within the
    f16 rounding of the partials and of every fold (the reference's own
    tolerance for its split-K kernel, tests/test_examples.py:683-723)."""
    P, V = splitk_inputs()
    C = oracle_splitk(P, V)
    want = P.astype(np.float32) @ V.astype(np.float32)
    np.testing.assert_allclose(C.astype(np.float32), want, rtol=2e-2, atol=2e-1)
    # the same with integer data, where every product, partial and fold is exact
    Pi = np.random.default_rng(1).integers(-2, 3, (1, 1024)).astype(np.float16)
    Vi = np.random.default_rng(2).integers(-2, 3, (1024, 128)).astype(np.float16)
    np.testing.assert_array_equal(oracle_splitk(Pi, Vi), (Pi.astype(np.int64) @ Vi.astype(np.int64)).astype(np.float16))


def ffn_inputs(seq=4, d=256, f=1024, seed=11):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((seq, d)).astype(np.float16)
    wg = (rng.standard_normal((d, f)) / 16).astype(np.float16)
    wu = (rng.standard_normal((d, f)) / 16).astype(np.float16)
    wd = (rng.standard_normal((f, d)) / 32).astype(np.float16)
    return x, wg, wu, wd


def ffn_model(x, wg, wu, wd):
    x64 = x.astype(np.float64)
    g, u = x64 @ wg.astype(np.float64), x64 @ wu.astype(np.float64)
    h = g / (1 + np.exp(-g)) * u
    return h @ wd.astype(np.float64) + x64


def oracle_ffn(x, wg, wu, wd):
    o = OracleInterpreter()
    o.load(_cases.ffn_swiglu_4core(x.shape[0], x.shape[1], wg.shape[1]))
    return o.execute_function("ffn_swiglu", x_ptr=x, wg_ptr=wg, wu_ptr=wu, wd_ptr=wd,
                              out_ptr=np.zeros_like(x))["out_ptr"]


def test_oracle_ffn_swiglu_4core():
    """The 4-core SwiGLU FFN against a float64 model, at the tolerance of
    the reference's own check of its 4-core FFN example
    (tests/test_examples.py:932-1030: f16 matmuls and f16 folds)."""
    x, wg, wu, wd = ffn_inputs()
    np.testing.assert_allclose(oracle_ffn(x, wg, wu, wd).astype(np.float64), ffn_model(x, wg, wu, wd),
                               rtol=2e-2, atol=2e-2)
