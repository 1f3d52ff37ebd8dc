"""Oracle pins for the arith rules the config kernels do not reach: integer
tile arithmetic on negative and extreme operands, every cmpi predicate,
int <-> float casts and bitcasts, the f16 coercion of a scalar operand of a
float binop, remf, powf and fma.  Each is checked against a brute force
written from the definitions (tests/_op_tables.py), on the oracle running a
small KTIR kernel, so a wrong rounding, sign, truncation direction or
operand order fails here.  CPU only."""
import math
import struct

import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases
from tests import _op_tables as T

_NP = {"f16": np.float16, "f32": np.float32, "i1": np.bool_, "i32": np.int32, "i64": np.int64}


def _run(body, ins, out_dt, arrays, cores=4):
    n = len(arrays[0])
    src, fn, names = _cases.elementwise(body, ins, out_dt, n=n, cores=cores)
    kw = dict(zip(names, [a.copy() for a in arrays] + [np.zeros(n, _NP[out_dt])]))
    o = OracleInterpreter()
    o.load(src)
    return o.execute_function(fn, **kw)["r_ptr"]


@pytest.mark.parametrize("op", T.INT_OPS)
def test_oracle_int_tile_ops_against_brute_force(op):
    a, b = T.int_operands(op, n=2048)
    with np.errstate(all="ignore"):
        got = _run([f"%r = {op} %a, %b : {{T_i32}}"], ["i32", "i32"], "i32", [a, b], cores=T.int_cores(op))
    want = np.array([T.brute_int(op, x, y) for x, y in zip(a.tolist(), b.tolist())], np.int64)
    bad = got.astype(np.int64) != want
    assert not bad.any(), (op, a[bad][:6], b[bad][:6], got[bad][:6], want[bad][:6])


@pytest.mark.parametrize("op,scalar", [("arith.divsi", -3), ("arith.divsi", 0), ("arith.remsi", -7),
                                       ("arith.ceildivsi", 4), ("arith.floordivsi", -5), ("arith.remui", -5),
                                       ("arith.shrsi", 33), ("arith.shli", 31), ("arith.shrui", 4),
                                       ("arith.maxsi", -2)])
def test_oracle_int_tile_scalar_ops_against_brute_force(op, scalar):
    """A tile with a scalar operand: the scalar joins the tile's int32 arithmetic."""
    a, _ = T.int_operands("arith.addi", n=1024, seed=3)
    body = [f"%s = arith.constant {scalar} : i32", f"%r = {op} %a, %s : {{T_i32}}"]
    with np.errstate(all="ignore"):
        got = _run(body, ["i32"], "i32", [a], cores=T.int_cores(op, scalar=True))
    want = np.array([T.brute_int(op, x, scalar) for x in a.tolist()], np.int64)
    np.testing.assert_array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("pred", sorted(T.CMPI))
def test_oracle_cmpi_against_brute_force(pred):
    a, b = T.int_operands("arith.subi", n=2048, seed=5)
    got = _run([f"%c = arith.cmpi {pred}, %a, %b : {{T_i32}}",
                "%r = arith.select %c, %a, %b : {T_i1}, {T_i32}"], ["i32", "i32"], "i32", [a, b])
    want = np.array([x if T.CMPI[pred](x, y) else y for x, y in zip(a.tolist(), b.tolist())], np.int64)
    np.testing.assert_array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("frm", ["f32", "f16"])
def test_oracle_fptosi_against_brute_force(frm):
    x = T.float_cast_operands(n=2048)
    if frm == "f16":
        with np.errstate(all="ignore"):
            x = x.astype(np.float16)
    with np.errstate(all="ignore"):
        got = _run([f"%r = arith.fptosi %a : {{T_{frm}}} to {{T_i32}}"], [frm], "i32", [x])
    want = np.array([T.fptosi_brute(v) for v in x.tolist()], np.int64)
    bad = got.astype(np.int64) != want
    assert not bad.any(), (x[bad][:6], got[bad][:6], want[bad][:6])


@pytest.mark.parametrize("to", ["f32", "f16"])
def test_oracle_sitofp_against_brute_force(to):
    """int32 -> float: the value rounded once to the target (RNE), overflow to inf."""
    a, _ = T.int_operands("arith.addi", n=2048, seed=7)
    got = _run([f"%r = arith.sitofp %a : {{T_i32}} to {{T_{to}}}"], ["i32"], to, [a])
    if to == "f32":
        want = np.array([float(np.float32(float(v))) for v in a.tolist()])
        # np.float32(float(v)) rounds v once: |v| < 2^53, so float(v) is exact
    else:
        want = np.array([T.f16_coerce_brute(float(v)) for v in a.tolist()])
    np.testing.assert_array_equal(got.astype(np.float64), want)


def test_oracle_uitofp_extsi_trunci_index_cast():
    """uitofp keeps the int32 value (the reference's astype(float32)); extsi
    to i64 and trunci back are the identity on int32 values; an index_cast
    scalar feeds a tile op unchanged."""
    a, _ = T.int_operands("arith.addi", n=1024, seed=9)
    got = _run(["%r = arith.uitofp %a : {T_i32} to {T_f32}"], ["i32"], "f32", [a])
    np.testing.assert_array_equal(got, a.astype(np.float64).astype(np.float32))
    body = ["%w = arith.extsi %a : {T_i32} to {T_i64}", "%r = arith.trunci %w : {T_i64} to {T_i32}"]
    np.testing.assert_array_equal(_run(body, ["i32"], "i32", [a]), a)
    body = ["%k = arith.constant 5 : i32", "%i = arith.index_cast %k : i32 to index",
            "%r = arith.muli %a, %i : {T_i32}"]
    want = np.array([T.wrap32(v * 5) for v in a.tolist()], np.int64)
    np.testing.assert_array_equal(_run(body, ["i32"], "i32", [a]).astype(np.int64), want)


def test_oracle_bitcast_both_ways():
    x = T.float_cast_operands(n=1024, seed=11)
    got = _run(["%r = arith.bitcast %a : {T_f32} to {T_i32}"], ["f32"], "i32", [x])
    want = [struct.unpack("<i", struct.pack("<f", v))[0] for v in x.tolist()]
    np.testing.assert_array_equal(got.astype(np.int64), np.array(want, np.int64))
    i, _ = T.int_operands("arith.addi", n=1024, seed=12)
    got = _run(["%r = arith.bitcast %a : {T_i32} to {T_f32}"], ["i32"], "f32", [i])
    want = [struct.pack("<i", v) for v in i.tolist()]
    np.testing.assert_array_equal(np.frombuffer(got.tobytes(), np.uint8),
                                  np.frombuffer(b"".join(want), np.uint8))


_COERCE = [1.0e-5, 0.1, 3.0e-8, 1.0e-8, 70000.0, 65519.0, -2.0e-7, 1.0 / 3.0]


@pytest.mark.parametrize("c", _COERCE)
def test_oracle_scalar_operand_coerced_to_f16(c):
    """f32 tile * scalar: the scalar is rounded to f16 first (so 1e-8 is 0,
    70000 is inf, 0.1 is 0.0999755859375), then the product is f32."""
    x = np.random.default_rng(13).standard_normal(1024).astype(np.float32) * 1000
    body = [f"%s = arith.constant {c!r} : f32", "%r = arith.mulf %a, %s : {T_f32}"]
    with np.errstate(all="ignore"):
        got = _run(body, ["f32"], "f32", [x])
        want = (x.astype(np.float64) * T.f16_coerce_brute(c)).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def _py_remainder(a: float, b: float) -> float:
    """Python's float % (sign of the divisor), the rule NumPy's remainder follows."""
    if math.isnan(a) or math.isnan(b) or math.isinf(a) or b == 0:
        return math.nan
    return math.fmod(a, b) if math.fmod(a, b) == 0 or (math.fmod(a, b) < 0) == (b < 0) else \
        math.fmod(a, b) + b


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_oracle_remf_against_python_mod(dt):
    rng = np.random.default_rng(14)
    a = (rng.standard_normal(2048) * 10.0 ** rng.uniform(-2, 3, 2048)).astype(_NP[dt])
    b = (rng.standard_normal(2048) * 10.0 ** rng.uniform(-2, 2, 2048)).astype(_NP[dt])
    a[:6] = [5.0, -5.0, 5.0, -5.0, 0.0, 7.0]
    b[:6] = [3.0, 3.0, -3.0, -3.0, 2.0, 0.0]
    with np.errstate(all="ignore"):
        got = _run([f"%r = arith.remf %a, %b : {{T_{dt}}}"], [dt, dt], dt, [a, b])
    want = np.array([_py_remainder(float(x), float(y)) for x, y in zip(a.tolist(), b.tolist())])
    # fmod is exact; adding b rounds once in f32 (and once more to f16)
    want = want.astype(np.float32).astype(_NP[dt])
    both_nan = np.isnan(got) & np.isnan(want)
    np.testing.assert_array_equal(np.where(both_nan, 0, got), np.where(both_nan, 0, want))
    assert got[0] == 2.0 and got[1] == 1.0 and got[2] == -1.0 and got[3] == -2.0


def test_oracle_powf_and_fma():
    """powf: f32 power rounded once to the tile dtype (within an f16 ulp of
    the float64 power); fma: a * b rounded to f32, + c rounded to f32, then to
    the tile dtype (not fused)."""
    rng = np.random.default_rng(15)
    x = rng.uniform(0.1, 4.0, 1024).astype(np.float16)
    e = rng.uniform(-3, 3, 1024).astype(np.float16)
    got = _run(["%r = math.powf %a, %b : {T_f16}"], ["f16", "f16"], "f16", [x, e])
    want = (x.astype(np.float64) ** e.astype(np.float64)).astype(np.float16)
    d = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert d.max() <= 1
    a = np.full(512, 1.0 + 2.0 ** -12, np.float32)
    c = np.full(512, -(1.0 + 2.0 ** -11), np.float32)
    got = _run(["%r = math.fma %a, %b, %c : {T_f32}"], ["f32", "f32", "f32"], "f32", [a, a, c])
    # exactly a * a + c = 2^-24, but a * a = 1 + 2^-11 + 2^-24 is a tie that
    # rounds to 1 + 2^-11 in f32 first, so unfused it is 0
    np.testing.assert_array_equal(got, np.zeros(512, np.float32))


@pytest.mark.parametrize("op,fn", [("math.ceil", math.ceil), ("math.floor", math.floor)])
def test_oracle_ceil_floor_against_math(op, fn):
    x = T.float_cast_operands(n=1024, seed=17)
    x = x[np.isfinite(x)]
    got = _run([f"%r = {op} %a : {{T_f32}}"], ["f32"], "f32", [x[:1024 // 4 * 4]], cores=1)
    want = np.array([float(fn(v)) for v in x[:len(got)].tolist()], np.float64)
    np.testing.assert_array_equal(got.astype(np.float64), np.where(want == 0, 0.0, want))


def test_oracle_absi_against_python_abs():
    """|x| wrapped to int32 (|INT_MIN| stays INT_MIN)."""
    a, _ = T.int_operands("arith.addi", n=1024, seed=19)
    got = _run(["%r = math.absi %a : {T_i32}"], ["i32"], "i32", [a])
    np.testing.assert_array_equal(got.astype(np.int64), np.array([T.wrap32(abs(v)) for v in a.tolist()]))
