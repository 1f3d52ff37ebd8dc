"""Pins for the oracle's scalars read from tile data: tensor.extract gives a
NumPy scalar of the tile's type, a reduction over every axis a Python float
(reference dialects/tensor_ops.py:88-102, dialects/linalg_ops.py:197-240),
and scalar ops follow the reference's rules for those types:

* a float op of two scalars rounds both to f16 and gives an f16
  (dialects/_helpers.py:47-50), so a value f16 cannot hold is lost even
  when both scalars came from f32 tiles;
* a math op keeps a NumPy scalar's type and computes on a Python float in
  float64 (ops/_helpers.py:50-60);
* tensor.splat / linalg.fill convert the scalar once to the tile's type.

Each case is checked against a value fixed by hand (closed forms chosen
so that the other rule gives a different answer), not against a NumPy
restatement of the same rule.  Scalar min / max has no reference
behaviour to match for a Python-float operand (the reference's handler
reads `.data` from both operands, which a Python float lacks); the oracle
gives NumPy's result there, and the two-NumPy-scalar case below is the
reference's own (NumPy promotion of the two buffers' types)."""
import math

import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases as C

_NP = {"f16": np.float16, "f32": np.float32}


def run_chain(body, x, dt="f32", out_dt="f32", idx="%c0", fill=False):
    cores, cols = x.shape
    src, fn = C.scalar_chain(body, dt=dt, out_dt=out_dt, cores=cores, C=cols, idx=idx, fill=fill)
    o = OracleInterpreter()
    o.load(src)
    y0 = np.zeros((cores, cols), np.int32 if out_dt == "i32" else _NP[out_dt])
    return o.execute_function(fn, x_ptr=x.astype(_NP[dt]), y_ptr=y0)["y_ptr"]


def rows(*pairs, cols=16, fill=0.25):
    """One row per (s, t): x[c, 0] = s, x[c, cols - 1] = t, `fill` elsewhere."""
    x = np.full((len(pairs), cols), fill, np.float64)
    for c, (s, t) in enumerate(pairs):
        x[c, 0], x[c, -1] = s, t
    return x


def test_two_f32_scalars_are_added_in_f16():
    # 1e-8 is 0 in f16 (an f32 sum would be 2e-8); 1/3 + 1/3 rounds to f16
    y = run_chain("    %r = arith.addf %s, %t : {dt}", rows((1e-8, 1e-8), (1 / 3, 1 / 3), (2049.0, 0.0)))
    assert y[0, 0] == 0.0
    assert y[1, 0] == np.float32(0.66650390625)          # 2 * f16(1/3)
    assert y[2, 0] == 2048.0                              # 2049 is not an f16: ties to even


def test_two_f32_scalars_multiply_and_divide_in_f16():
    y = run_chain("    %r = arith.mulf %s, %t : {dt}", rows((300.0, 300.0), (-300.0, 300.0)))
    assert y[0, 0] == np.inf and y[1, 0] == -np.inf       # 90000 overflows f16
    y = run_chain("    %r = arith.divf %s, %t : {dt}", rows((1.0, 3.0), (1.0, 0.0)))
    assert y[0, 0] == np.float32(0.333251953125) and y[1, 0] == np.inf


def test_scalar_remf_takes_the_divisor_sign():
    y = run_chain("    %r = arith.remf %s, %t : {dt}", rows((5.5, -2.0), (-5.5, 2.0)))
    assert y[0, 0] == -0.5 and y[1, 0] == 0.5


def test_a_constant_operand_is_rounded_to_f16_too():
    body = "    %k = arith.constant 0.1 : {dt}\n    %r = arith.addf %s, %k : {dt}"
    y = run_chain(body, rows((0.0, 0.0)))
    assert y[0, 0] == np.float32(0.0999755859375)         # f16(0.1), not f32(0.1)


def test_math_keeps_the_scalar_type():
    # f32 scalar: f32 sqrt; f16 scalar (after truncf): f16 sqrt
    y = run_chain("    %r = math.sqrt %s : {dt}", rows((2.0, 0.0)))
    assert y[0, 0] == np.float32(1.4142135)
    body = "    %h = arith.truncf %s : f32 to f16\n    %q = math.sqrt %h : f16\n    %r = arith.extf %q : f16 to f32"
    y = run_chain(body, rows((2.0, 0.0)))
    assert y[0, 0] == np.float32(1.4140625)


def test_a_full_reduction_is_a_python_float():
    # row of 16 x 0.5 = 8.0: float64 sqrt(8), rounded once into the f32 tile
    x = np.full((2, 16), 0.5)
    y = run_chain("    %r = math.sqrt %u : {dt}", x)
    assert y[0, 0] == np.float32(math.sqrt(8.0))
    # the same sum in an f16 tile: the f16 rule would give f16(sqrt 8) = 2.828125
    y = run_chain("    %r = math.sqrt %u : {dt}", x, dt="f16", out_dt="f32")
    assert y[0, 0] == np.float32(math.sqrt(8.0)) != np.float32(2.828125)


def test_rmsnorm_scalar_chain_closed_form():
    # sum 8, / 16 = 0.5, + 0, rsqrt in f16: 1 / f16(sqrt 0.5) = 1 / 0.70703125 -> f16 1.4140625
    body = ("    %n = arith.constant 16.0 : {dt}\n    %eps = arith.constant 0.0 : {dt}\n"
            "    %ms = arith.divf %u, %n : {dt}\n    %a = arith.addf %ms, %eps : {dt}\n"
            "    %r = math.rsqrt %a : {dt}")
    y = run_chain(body, np.full((2, 16), 0.5))
    assert np.all(y == np.float32(1.4140625))


def test_negf_absf_keep_the_value():
    body = "    %a = math.absf %s : {dt}\n    %r = arith.negf %a : {dt}"
    y = run_chain(body, rows((1e-8, 0.0), (-3.5, 0.0)))
    assert y[0, 0] == np.float32(-1e-8) and y[1, 0] == -3.5


def test_two_numpy_scalars_min_max_promote():
    # f32 s against f16 h = f16(t): the f32 result keeps s exactly
    body = ("    %h = arith.truncf %t : f32 to f16\n    %r = arith.maximumf %s, %h : {dt}")
    y = run_chain(body, rows((0.1, 0.05), (0.05, 0.1)))
    assert y[0, 0] == np.float32(0.1)
    assert y[1, 0] == np.float32(0.0999755859375)
    y = run_chain("    %r = arith.maxnumf %s, %t : {dt}", rows((np.nan, 1.0), (2.0, np.nan)))
    assert y[0, 0] == 1.0 and y[1, 0] == 2.0
    y = run_chain("    %r = arith.maximumf %s, %t : {dt}", rows((np.nan, 1.0)))
    assert np.isnan(y[0, 0])


def test_splat_and_fill_convert_once():
    # f16 result 2.25 / -2.75 into an i32 tile: truncation; inf: INT_MIN (x86)
    y = run_chain("    %r = arith.addf %s, %t : {dt}", rows((2.75, -0.5), (-2.75, 0.0), (70000.0, 0.0)),
                  out_dt="i32")
    assert list(y[:, 0]) == [2, -2, np.iinfo(np.int32).min]
    # an f32 scalar into an f16 tile by linalg.fill: one rounding
    y = run_chain("    %r = math.absf %s : {dt}", rows((1 / 3, 0.0)), out_dt="f16", fill=True)
    assert y[0, 0] == np.float16(1 / 3)


def test_per_core_extract_index():
    # x[c, c]: a different element on every core
    x = np.arange(64, dtype=np.float64).reshape(4, 16) / 8
    y = run_chain("    %r = arith.addf %s, %s : {dt}", x, idx="%i_core")
    np.testing.assert_array_equal(y[:, 0], [2 * x[c, c] for c in range(4)])


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_extract_then_splat_is_the_element(dt):
    x = np.random.default_rng(1).standard_normal((4, 16))
    y = run_chain("    %r = math.absf %t : {dt}", x, dt=dt, out_dt=dt)
    np.testing.assert_array_equal(y, np.repeat(np.abs(x[:, -1:].astype(_NP[dt])), 16, axis=1))


def test_a_reduction_into_a_one_element_tile_stays_a_tile():
    # %v: the same row sum reduced into a tensor<1x..> outs is a tile, so
    # math on it is the tile's f16 math, and tensor.splat takes its element
    x = np.full((2, 16), 0.5)
    y = run_chain("    %r = math.sqrt %v : tensor<1x{dt}>", x, dt="f16", out_dt="f32")
    assert y[0, 0] == np.float32(2.828125)


def test_planted_f32_scalar_rule_fails_a_pin(monkeypatch):
    """A float op of two scalars computed in f32 (no f16 rounding) changes
    the first pin's answer."""
    import oracle.interp as oi
    orig = oi._float_binop

    def planted(a, b, fn):
        if oi._is_scalar(a) and oi._is_scalar(b):
            return np.float32(fn(np.float32(a), np.float32(b)))
        return orig(a, b, fn)

    monkeypatch.setattr(oi, "_float_binop", planted)
    y = run_chain("    %r = arith.addf %s, %t : {dt}", rows((1e-8, 1e-8)))
    assert y[0, 0] != 0.0


def extract_softmax_closed_form(got, rows, cols):
    """Rows of tests.test_oracle_linalg_pins.broadcast_softmax_rows: 1 / k
    (rounded to f16) at the k top entries, 0 elsewhere (e^-30 is 0 in f16)."""
    for r in range(rows):
        top = np.zeros(cols, bool)
        top[np.arange(min(r + 1, cols)) * 7 % cols] = True
        np.testing.assert_array_equal(got[r, top], np.float16(1.0 / top.sum()), err_msg=f"row {r}")
        np.testing.assert_array_equal(got[r, ~top], 0.0, err_msg=f"row {r}")


def extract_rmsnorm_rows(rows, cols):
    """Rows that are each one power of two, +-2^k (k from -2 to 2, a new
    sign and k per row), and a weight that varies by column: with eps 0
    every f16 step is exact (c^2, the pairwise sum, / cols, sqrt, 1 / |c|,
    c / |c|), so y = sign(c) w exactly."""
    c = np.array([(-1) ** r * 2.0 ** (r % 5 - 2) for r in range(rows)])
    w = np.linspace(0.5, 1.5, cols).astype(np.float16)
    return np.repeat(c[:, None], cols, axis=1).astype(np.float16), w, np.sign(c)


@pytest.mark.parametrize("rows,cols,cores", [(64, 256, 8), (32, 16, 4)])
def test_oracle_softmax_extract_closed_form(rows, cols, cores):
    from ktir_cpu_amd import configs
    from tests.test_oracle_linalg_pins import broadcast_softmax_rows
    o = OracleInterpreter()
    o.load(configs.softmax_extract(rows, cols, cores))
    x = broadcast_softmax_rows(rows, cols).astype(np.float16)
    got = o.execute_function("softmax_fwd", x_ptr=x, y_ptr=np.zeros_like(x), n_rows=rows)["y_ptr"]
    extract_softmax_closed_form(got, rows, cols)


@pytest.mark.parametrize("rows,cols,cores", [(40, 256, 8), (20, 16, 4)])
def test_oracle_rmsnorm_extract_closed_form(rows, cols, cores):
    from ktir_cpu_amd import configs
    o = OracleInterpreter()
    o.load(configs.rmsnorm_extract(rows, cols, cores))
    x, w, sg = extract_rmsnorm_rows(rows, cols)
    got = o.execute_function("rmsnorm_fwd", x_ptr=x, w_ptr=w.reshape(1, cols), y_ptr=np.zeros_like(x),
                             n_rows=rows, eps=0.0)["y_ptr"]
    np.testing.assert_array_equal(got, (sg[:, None] * w[None, :]).astype(np.float16))
