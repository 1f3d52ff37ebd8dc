"""Checks that pin the oracle's matmul, exp and attention against what the
mathematics fixes (no GPU): exact small-integer products, float64 exp, and
the closed form of attention with uniform scores.  Each would fail for a
transposed operand, a wrong mask direction or a missing normalisation."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter, bf16_bits, bf16_from_bits
from tests import _cases


def _exec(case):
    src, fn, kw = case
    o = OracleInterpreter()
    o.load(src)
    return o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})


@pytest.mark.parametrize("shape", [(128, 128, 128, 64, 64, 32, 2, 2), (256, 128, 64, 64, 64, 32, 2, 2)])
def test_oracle_matmul_integer_exact(shape):
    """Entries in {-2..2}: every product and partial sum is an integer below
    2^11, so f16 operands, f32 accumulation and the f16 store are all exact
    and the tiled K loop must equal the integer product (A is not square in
    the second case, so swapped operands cannot match)."""
    M, N, K = shape[:3]
    rng = np.random.default_rng(11)
    a = rng.integers(-2, 3, (M, K)).astype(np.float16)
    b = rng.integers(-2, 3, (K, N)).astype(np.float16)
    src, fn, kw = _cases.gemm(*shape)
    kw.update(a_ptr=a, b_ptr=b)
    out = _exec((src, fn, kw))
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float16)
    np.testing.assert_array_equal(out["c_ptr"], want)


def test_oracle_exp_against_float64():
    """math.exp on f32 tiles: within 4 f32 ulps of exp computed in float64
    (NumPy's float32 exp, which the reference calls too, is off by up to about
    2.3 ulps; a wrong base or sign is off by orders of magnitude)."""
    from ktir_cpu_amd import configs
    n = 4096
    x = np.linspace(-80.0, 80.0, n).astype(np.float32)
    body = "\n".join([
        configs._view("X", "x_ptr", [n], [1], "f32"),
        configs._view("Y", "y_ptr", [n], [1], "f32"),
        "    %c0 = arith.constant 0 : index",
        configs._tile("xt", "X", ["%c0"], [n], [n], "f32"),
        configs._tile("yt", "Y", ["%c0"], [n], [n], "f32"),
        f"    %v = ktdp.load %xt : !ktdp.access_tile<{n}xindex> -> tensor<{n}xf32>",
        f"    %e = math.exp %v : tensor<{n}xf32>",
        f"    ktdp.store %e, %yt : tensor<{n}xf32>, !ktdp.access_tile<{n}xindex>",
    ])
    src = ("module {\n  func.func @ex(%x_ptr: index, %y_ptr: index) attributes {grid = [1, 1]} {\n"
           + body + "\n    return\n  }\n}\n")
    out = _exec((src, "ex", dict(x_ptr=x, y_ptr=np.zeros(n, np.float32))))
    exact = np.exp(x.astype(np.float64))
    ulp = np.spacing(exact.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(out["y_ptr"].astype(np.float64) - exact) <= 4 * ulp)


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_attention_uniform_scores(causal):
    """Q = 0 makes every score 0, so softmax is uniform over the keys a query
    may see: O[i] = mean of V[0..i] (causal) or of all V (full), in f32
    before the bf16 store."""
    B, H, S, D = 1, 2, 256, 128
    src, fn, kw = _cases.flash_attention(B=B, H=H, S=S, D=D, blk=128, causal=causal)
    kw["q_ptr"] = np.zeros_like(kw["q_ptr"])
    out = _exec((src, fn, kw))
    v = bf16_from_bits(kw["v_ptr"]).astype(np.float64)
    if causal:
        want = np.cumsum(v, axis=2) / np.arange(1, S + 1)[None, None, :, None]
    else:
        want = np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape)
    got = bf16_from_bits(out["o_ptr"]).astype(np.float64)
    np.testing.assert_allclose(got, bf16_from_bits(bf16_bits(want.astype(np.float32))), rtol=1e-2, atol=1e-3)
