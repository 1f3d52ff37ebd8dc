"""GPU parity for the arith rules outside the config kernels: integer tile
arithmetic on negative and extreme operands, every cmpi predicate, int <->
float casts and bitcasts, the f16 coercion of a scalar operand of a float
binop, remf, powf, fma, ceil / floor / absi.  The GPU runs the same small
KTIR kernels as the oracle, and the results are compared bit for bit (powf
within a few f32 ulps: ROCm's powf against the host's).  The oracle is pinned
against brute force on the same tables in tests/test_oracle_op_pins.py."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases
from tests import _op_tables as T

pytestmark = pytest.mark.gpu

_NP = {"f16": np.float16, "f32": np.float32, "i1": np.bool_, "i32": np.int32, "i64": np.int64}


def _both(body, ins, out_dt, arrays, cores=4):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    n = len(arrays[0])
    src, fn, names = _cases.elementwise(body, ins, out_dt, n=n, cores=cores)
    kw = dict(zip(names, list(arrays) + [np.zeros(n, _NP[out_dt])]))
    o = OracleInterpreter()
    o.load(src)
    with np.errstate(all="ignore"):
        ref = o.execute_function(fn, **{k: v.copy() for k, v in kw.items()})["r_ptr"]
    g = KTIRInterpreter()
    g.load(src)
    print(fn, body[-1], flush=True)
    got = g.execute_function(fn, **kw)["r_ptr"]
    print("  ", g.last_plan.mode, g.last_plan.counts(), flush=True)
    return got, ref


def _bits_equal(got, ref):
    g, r = np.asarray(got), np.asarray(ref)
    if g.dtype.kind == "f":
        nan = np.isnan(g) & np.isnan(r)
        u = {2: np.uint16, 4: np.uint32}[g.dtype.itemsize]
        bad = np.where(nan, 0, g.view(u)) != np.where(nan, 0, r.view(u))
    else:
        bad = g != r
    assert not bad.any(), (np.nonzero(bad)[0][:6], g[bad][:6], r[bad][:6])


@pytest.mark.parametrize("op", T.INT_OPS)
def test_int_tile_ops_bit_exact(op):
    a, b = T.int_operands(op, n=4096)
    got, ref = _both([f"%r = {op} %a, %b : {{T_i32}}"], ["i32", "i32"], "i32", [a, b], cores=T.int_cores(op))
    _bits_equal(got, ref)


def test_shrui_tile_by_tile_on_many_cores():
    """On several cores the reference misplaces the int64 result of a
    tile-by-tile shrui (the oracle's one-core pin shows the values); the GPU
    keeps each core's tile in place, with the brute-force values."""
    a, b = T.int_operands("arith.shrui", n=4096, seed=2)
    got, _ = _both(["%r = arith.shrui %a, %b : {T_i32}"], ["i32", "i32"], "i32", [a, b], cores=8)
    want = np.array([T.brute_int("arith.shrui", x, y) for x, y in zip(a.tolist(), b.tolist())], np.int64)
    np.testing.assert_array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("op,scalar", [("arith.divsi", -3), ("arith.divsi", 0), ("arith.remsi", -7),
                                       ("arith.ceildivsi", 4), ("arith.floordivsi", -5), ("arith.remui", -5),
                                       ("arith.shrsi", 33), ("arith.shli", 31), ("arith.shrui", 4),
                                       ("arith.maxsi", -2), ("arith.muli", -65537)])
def test_int_tile_scalar_ops_bit_exact(op, scalar):
    a, _ = T.int_operands("arith.addi", n=2048, seed=3)
    body = [f"%s = arith.constant {scalar} : i32", f"%r = {op} %a, %s : {{T_i32}}"]
    got, ref = _both(body, ["i32"], "i32", [a], cores=T.int_cores(op, scalar=True))
    _bits_equal(got, ref)


@pytest.mark.parametrize("pred", sorted(T.CMPI))
def test_cmpi_bit_exact(pred):
    a, b = T.int_operands("arith.subi", n=4096, seed=5)
    got, ref = _both([f"%c = arith.cmpi {pred}, %a, %b : {{T_i32}}",
                      "%r = arith.select %c, %a, %b : {T_i1}, {T_i32}"], ["i32", "i32"], "i32", [a, b])
    _bits_equal(got, ref)


@pytest.mark.parametrize("pred", ["slt", "uge", "ne"])
def test_cmpi_stored_as_i1(pred):
    """i1 tiles stored to a bool array: the reference has no KTIR dtype for a
    bool argument (dtypes.py:49-54 raise ValueError), which the oracle keeps;
    this backend accepts one, and the stored predicate is the brute force's."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    a, b = T.int_operands("arith.subi", n=2048, seed=6)
    src, fn, names = _cases.elementwise([f"%r = arith.cmpi {pred}, %a, %b : {{T_i32}}"], ["i32", "i32"], "i1",
                                        n=2048, cores=4)
    kw = dict(zip(names, [a, b, np.zeros(2048, np.bool_)]))
    o = OracleInterpreter()
    o.load(src)
    with pytest.raises(ValueError, match="No KTIR dtype"):
        o.execute_function(fn, **{k: v.copy() for k, v in kw.items()})
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function(fn, **kw)["r_ptr"]
    want = np.array([T.CMPI[pred](x, y) for x, y in zip(a.tolist(), b.tolist())])
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("frm", ["f32", "f16"])
def test_fptosi_bit_exact(frm):
    x = T.float_cast_operands(n=4096)
    if frm == "f16":
        with np.errstate(all="ignore"):
            x = x.astype(np.float16)
    got, ref = _both([f"%r = arith.fptosi %a : {{T_{frm}}} to {{T_i32}}"], [frm], "i32", [x])
    _bits_equal(got, ref)


@pytest.mark.parametrize("to", ["f32", "f16"])
def test_sitofp_bit_exact(to):
    a, _ = T.int_operands("arith.addi", n=4096, seed=7)
    got, ref = _both([f"%r = arith.sitofp %a : {{T_i32}} to {{T_{to}}}"], ["i32"], to, [a])
    _bits_equal(got, ref)


def test_uitofp_extsi_trunci_index_cast_bit_exact():
    a, _ = T.int_operands("arith.addi", n=2048, seed=9)
    _bits_equal(*_both(["%r = arith.uitofp %a : {T_i32} to {T_f32}"], ["i32"], "f32", [a]))
    _bits_equal(*_both(["%w = arith.extsi %a : {T_i32} to {T_i64}",
                        "%r = arith.trunci %w : {T_i64} to {T_i32}"], ["i32"], "i32", [a]))
    _bits_equal(*_both(["%r = arith.extsi %a : {T_i32} to {T_i64}"], ["i32"], "i64", [a]))
    _bits_equal(*_both(["%k = arith.constant 5 : i32", "%i = arith.index_cast %k : i32 to index",
                        "%r = arith.muli %a, %i : {T_i32}"], ["i32"], "i32", [a]))


def test_bitcast_both_ways_bit_exact():
    x = T.float_cast_operands(n=2048, seed=11)
    _bits_equal(*_both(["%r = arith.bitcast %a : {T_f32} to {T_i32}"], ["f32"], "i32", [x]))
    i, _ = T.int_operands("arith.addi", n=2048, seed=12)
    got, ref = _both(["%r = arith.bitcast %a : {T_i32} to {T_f32}"], ["i32"], "f32", [i])
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("c", [1.0e-5, 0.1, 3.0e-8, 1.0e-8, 70000.0, 65519.0, -2.0e-7, 1.0 / 3.0])
@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_scalar_operand_coerced_to_f16(c, dt):
    """A tile times a scalar f16 cannot hold: the scalar rounds to f16 first
    (the reference's np.float16 coercion), for f32 and f16 tiles."""
    x = (np.random.default_rng(13).standard_normal(2048) * 1000).astype(_NP[dt])
    body = [f"%s = arith.constant {c!r} : f32", f"%r = arith.mulf %a, %s : {{T_{dt}}}"]
    _bits_equal(*_both(body, [dt], dt, [x]))
    body = [f"%s = arith.constant {c!r} : f32", f"%r = arith.addf %s, %a : {{T_{dt}}}"]
    _bits_equal(*_both(body, [dt], dt, [x]))


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_remf_bit_exact(dt):
    rng = np.random.default_rng(14)
    a = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-2, 3, 4096)).astype(_NP[dt])
    b = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-2, 2, 4096)).astype(_NP[dt])
    sp = np.array([5.0, -5.0, 5.0, -5.0, 0.0, 7.0, np.inf, 3.0, -3.0, np.nan, -0.0, 1.0], _NP[dt])
    sq = np.array([3.0, 3.0, -3.0, -3.0, 2.0, 0.0, 2.0, np.inf, np.inf, 1.0, 5.0, -np.inf], _NP[dt])
    a[:12], b[:12] = sp, sq
    _bits_equal(*_both([f"%r = arith.remf %a, %b : {{T_{dt}}}"], [dt, dt], dt, [a, b]))


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_fma_bit_exact(dt):
    rng = np.random.default_rng(16)
    a, b, c = ((rng.standard_normal(4096) * 10.0 ** rng.uniform(-3, 3, 4096)).astype(_NP[dt]) for _ in range(3))
    a[:4], b[:4] = 1.0 + 2.0 ** -12, 1.0 + 2.0 ** -12
    c[:4] = -(1.0 + 2.0 ** -11)
    _bits_equal(*_both([f"%r = math.fma %a, %b, %c : {{T_{dt}}}"], [dt, dt, dt], dt, [a, b, c]))


def test_powf_f32_within_ulps_and_f16_within_one_ulp():
    rng = np.random.default_rng(15)
    x = rng.uniform(0.05, 8.0, 4096).astype(np.float32)
    e = rng.uniform(-6, 6, 4096).astype(np.float32)
    got, ref = _both(["%r = math.powf %a, %b : {T_f32}"], ["f32", "f32"], "f32", [x, e])
    ulp = np.spacing(np.abs(ref)).astype(np.float64)
    assert (np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= 2 * ulp).all()
    got, ref = _both(["%r = math.powf %a, %b : {T_f16}"], ["f16", "f16"], "f16", [x.astype(np.float16),
                                                                                  e.astype(np.float16)])
    d = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert d.max() <= 1


@pytest.mark.parametrize("op", ["math.ceil", "math.floor"])
def test_ceil_floor_bit_exact(op):
    x = T.float_cast_operands(n=4096, seed=17)
    _bits_equal(*_both([f"%r = {op} %a : {{T_f32}}"], ["f32"], "f32", [x]))
    _bits_equal(*_both([f"%r = {op} %a : {{T_f16}}"], ["f16"], "f16", [_cases.f16_patterns(4096, seed=18)]))


def test_absi_bit_exact():
    a, _ = T.int_operands("arith.addi", n=2048, seed=19)
    _bits_equal(*_both(["%r = math.absi %a : {T_i32}"], ["i32"], "i32", [a]))
