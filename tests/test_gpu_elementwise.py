"""GPU parity for elementwise arithmetic, transcendentals, compares, selects,
min/max, casts and control flow, against the oracle on the same inputs.

Bars: f16 arithmetic bit-exact (NumPy's f16 ops are correctly rounded, and so
are the kernels' f32-then-round steps); f16 transcendentals within one f16
ulp (north star); f32 transcendentals within a few f32 ulps (ROCm device math
against NumPy's float32 kernels); compares, selects, min/max and casts
bit-exact.  Any NaN matches any NaN.
"""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases

pytestmark = pytest.mark.gpu

_NP = {"f16": np.float16, "f32": np.float32, "bf16": np.uint16, "i1": np.bool_, "i32": np.int32}


def _both(body, ins, out_dt, arrays, cores=4):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    n = len(arrays[0])
    src, fn, names = _cases.elementwise(body, ins, out_dt, n=n, cores=cores)
    kw = dict(zip(names, list(arrays) + [np.zeros(n, _NP[out_dt])]))
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: v.copy() for k, v in kw.items()})["r_ptr"]
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function(fn, **kw)["r_ptr"]
    print(fn, body[-1], g.last_plan.mode, g.last_plan.counts(), flush=True)
    return got, ref


def _bits_equal(got, ref):
    g, r = np.asarray(got), np.asarray(ref)
    if g.dtype.kind == "f":
        nan = np.isnan(g) & np.isnan(r)
        u = {2: np.uint16, 4: np.uint32}[g.dtype.itemsize]
        np.testing.assert_array_equal(np.where(nan, 0, g.view(u)), np.where(nan, 0, r.view(u)))
    else:
        np.testing.assert_array_equal(g, r)


@pytest.mark.parametrize("op", ["arith.addf", "arith.subf", "arith.mulf", "arith.divf"])
def test_f16_binops_bit_exact(op):
    n = 1 << 15
    a, b = _cases.f16_patterns(n, seed=1), _cases.f16_patterns(n, seed=2)
    got, ref = _both([f"%r = {op} %a, %b : {{T_f16}}"], ["f16", "f16"], "f16", [a, b])
    _bits_equal(got, ref)


@pytest.mark.parametrize("op", ["arith.addf", "arith.mulf", "arith.divf"])
def test_bf16_binops_bit_exact(op):
    """bf16 tiles (stored as bit patterns): f32 arithmetic rounded to bf16."""
    from oracle.interp import bf16_bits
    rng = np.random.default_rng(4)
    a = bf16_bits((rng.standard_normal(8192) * 10.0 ** rng.uniform(-20, 20, 8192)).astype(np.float32))
    b = bf16_bits((rng.standard_normal(8192) * 10.0 ** rng.uniform(-20, 20, 8192)).astype(np.float32))
    got, ref = _both([f"%r = {op} %a, %b : {{T_bf16}}"], ["bf16", "bf16"], "bf16", [a, b])
    np.testing.assert_array_equal(got, ref)


_F32_OPS = {"math.exp": (-80, 80), "math.log": (1e-30, 1e30), "math.log2": (1e-30, 1e30),
            "math.log1p": (-0.999, 1e6), "math.tanh": (-12, 12), "math.sin": (-100, 100),
            "math.cos": (-100, 100), "math.erf": (-6, 6), "math.sqrt": (0, 1e30), "math.rsqrt": (1e-30, 1e30)}


@pytest.mark.parametrize("op", sorted(_F32_OPS))
def test_f32_math(op):
    lo, hi = _F32_OPS[op]
    x = (np.geomspace(lo, hi, 8192) if lo > 0 else np.linspace(lo, hi, 8192)).astype(np.float32)
    got, ref = _both([f"%r = {op} %a : {{T_f32}}"], ["f32"], "f32", [x])
    g, r = got.astype(np.float64), ref.astype(np.float64)
    ulp = np.spacing(np.abs(ref)).astype(np.float64)
    # sin / cos near their zeros and erf near 0 (computed as 1 - poly * exp):
    # an absolute floor of a few f32 ulps of 1
    floor = 4.8e-7 if op in ("math.sin", "math.cos", "math.erf") else 0.0
    bad = np.abs(g - r) > 4 * ulp + floor
    assert not bad.any(), (op, x[bad][:5], g[bad][:5], r[bad][:5])


@pytest.mark.parametrize("op", ["math.exp", "math.log", "math.tanh", "math.sin", "math.cos", "math.erf",
                                "math.sqrt", "math.rsqrt", "math.log1p"])
def test_f16_math_within_one_ulp(op):
    lo = 0.01 if op in ("math.log", "math.sqrt", "math.rsqrt") else -8.0
    x = np.linspace(lo, 8.0, 8192).astype(np.float16)
    got, ref = _both([f"%r = {op} %a : {{T_f16}}"], ["f16"], "f16", [x])
    nan = np.isnan(got) | np.isnan(ref)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    d = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    d[nan] = 0
    assert d.max() <= 1, (op, x[d > 1][:5], got[d > 1][:5], ref[d > 1][:5])


@pytest.mark.parametrize("pred", ["oeq", "ogt", "oge", "olt", "ole", "one", "ord", "ueq", "ugt", "uge", "ult",
                                  "ule", "une", "uno", "true", "false"])
def test_cmpf_select_bit_exact(pred):
    vals = np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan, 1e-40, 3.0e38], np.float32)
    a, b = (x.reshape(-1) for x in np.meshgrid(vals, vals))
    a, b = np.tile(a, 41)[:4096], np.tile(b, 41)[:4096]
    got, ref = _both([f"%c = arith.cmpf {pred}, %a, %b : {{T_f32}}",
                      "%r = arith.select %c, %a, %b : {T_i1}, {T_f32}"], ["f32", "f32"], "f32", [a, b])
    _bits_equal(got, ref)


@pytest.mark.parametrize("op", ["arith.maximumf", "arith.minimumf", "arith.maxnumf", "arith.minnumf"])
def test_min_max_bit_exact(op):
    vals = np.array([0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan, 1e-40, 3.0e38], np.float32)
    a, b = (x.reshape(-1) for x in np.meshgrid(vals, vals))
    a, b = np.tile(a, 51)[:4096], np.tile(b, 51)[:4096]
    got, ref = _both([f"%r = {op} %a, %b : {{T_f32}}"], ["f32", "f32"], "f32", [a, b])
    _bits_equal(got, ref)


@pytest.mark.parametrize("to", ["f16", "bf16"])
def test_truncf_bit_exact(to):
    """f32 -> f16 / bf16 over float32 bit patterns at and around the rounding
    ties, overflow, subnormals, infinities and NaN."""
    hi = np.random.default_rng(9).integers(0, 1 << 16, 4096, dtype=np.uint32) << np.uint32(16)
    lows = np.array([0x0000, 0x1000, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x2000, 0x0FFF], np.uint32)
    x = (hi[:, None] | lows[None, :]).reshape(-1)[:16384].view(np.float32)
    got, ref = _both([f"%r = arith.truncf %a : {{T_f32}} to {{T_{to}}}"], ["f32"], to, [x])
    if to == "bf16":
        nan = ((got & 0x7F80) == 0x7F80) & ((got & 0x7F) != 0) & ((ref & 0x7F80) == 0x7F80) & ((ref & 0x7F) != 0)
        np.testing.assert_array_equal(np.where(nan, 0, got), np.where(nan, 0, ref))
    else:
        _bits_equal(got, ref)


@pytest.mark.parametrize("frm", ["f16", "bf16"])
def test_extf_bit_exact(frm):
    bits = np.random.default_rng(10).integers(0, 1 << 16, 8192, dtype=np.uint32).astype(np.uint16)
    x = bits.view(np.float16) if frm == "f16" else bits
    got, ref = _both([f"%r = arith.extf %a : {{T_{frm}}} to {{T_f32}}"], [frm], "f32", [x])
    _bits_equal(got, ref)


_IF_KERNEL = """module {
  func.func @if_kernel(%x_ptr: index, %y_ptr: index) attributes {grid = [8, 1]} {
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %c3 = arith.constant 3 : index
    %B = arith.constant 256 : index
    %off = arith.muli %core_id, %B : index
XVIEW
YVIEW
XTILE
YTILE
    %x = ktdp.load %xt : !ktdp.access_tile<256xindex> -> tensor<256xf16>
    %small = arith.cmpi slt, %core_id, %c3 : index
    scf.if %small {
      %d = arith.addf %x, %x : tensor<256xf16>
      ktdp.store %d, %yt : tensor<256xf16>, !ktdp.access_tile<256xindex>
    } else {
      %e = math.exp %x : tensor<256xf16>
      ktdp.store %e, %yt : tensor<256xf16>, !ktdp.access_tile<256xindex>
    }
    return
  }
}
"""


def test_scf_if_lane_varying_condition():
    """scf.if whose condition differs between cores (cores 0-2 store x + x,
    the others exp(x)): each branch runs on the lanes that take it, all
    cores still together."""
    from ktir_cpu_amd import configs
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src = (_IF_KERNEL.replace("XVIEW", configs._view("x_view", "x_ptr", [2048], [1], "f16"))
           .replace("YVIEW", configs._view("y_view", "y_ptr", [2048], [1], "f16"))
           .replace("XTILE", configs._tile("xt", "x_view", ["%off"], [256], [2048], "f16"))
           .replace("YTILE", configs._tile("yt", "y_view", ["%off"], [256], [2048], "f16")))
    x = np.random.default_rng(2).standard_normal(2048).astype(np.float16)
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function("if_kernel", x_ptr=x.copy(), y_ptr=np.zeros(2048, np.float16))["y_ptr"]
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function("if_kernel", x_ptr=x, y_ptr=np.zeros(2048, np.float16))["y_ptr"]
    assert g.last_plan.mode == "lockstep"
    d = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert d[:768].max() == 0 and d.max() <= 1
    np.testing.assert_array_equal(got[:768], x[:768] + x[:768])


_ACC_KERNEL = """module {
  func.func @acc_kernel(%x_ptr: index, %y_ptr: index) attributes {grid = [6, 1]} {
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %B = arith.constant 512 : index
    %off = arith.muli %core_id, %B : index
XVIEW
YVIEW
XTILE
YTILE
    %x = ktdp.load %xt : !ktdp.access_tile<512xindex> -> tensor<512xf32>
    %y = ktdp.load %yt : !ktdp.access_tile<512xindex> -> tensor<512xf32>
    %s = arith.addf %y, %x : tensor<512xf32>
    ktdp.store %s, %yt : tensor<512xf32>, !ktdp.access_tile<512xindex>
    return
  }
}
"""


def test_cores_accumulating_through_hbm_run_in_core_order():
    """Every core adds its block of x into the same y: cores communicate
    through HBM, so the hazard check sends the run to core-by-core order, and
    the f32 sums come out in the reference's core order, bit for bit."""
    from ktir_cpu_amd import configs
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src = (_ACC_KERNEL.replace("XVIEW", configs._view("x_view", "x_ptr", [3072], [1], "f32"))
           .replace("YVIEW", configs._view("y_view", "y_ptr", [512], [1], "f32"))
           .replace("XTILE", configs._tile("xt", "x_view", ["%off"], [512], [3072], "f32"))
           .replace("YTILE", configs._tile("yt", "y_view", ["%c0"], [512], [512], "f32")))
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(3072) * 10.0 ** rng.uniform(-6, 6, 3072)).astype(np.float32)
    y0 = rng.standard_normal(512).astype(np.float32)
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function("acc_kernel", x_ptr=x.copy(), y_ptr=y0.copy())["y_ptr"]
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function("acc_kernel", x_ptr=x, y_ptr=y0.copy())["y_ptr"]
    assert g.last_plan.mode == "sequential"
    np.testing.assert_array_equal(got, ref)
    want = y0.copy()
    for c in range(6):
        want = (want + x[c * 512:(c + 1) * 512]).astype(np.float32)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n", [1 << 15, 1 << 20])
def test_f16_mulf_keeps_the_sign_of_a_zero_product(n):
    """Products that round to a zero of either sign (tiny operands of mixed
    signs, and signed zeros times finite values): the f16 result keeps the
    sign.  An f32 product narrowed to f16 is otherwise compiled to one
    mixed-precision multiply-add with a +0 addend, which turns -0 into +0."""
    rng = np.random.default_rng(9)
    a = (rng.choice([-1.0, 1.0], n) * rng.uniform(1e-4, 2e-4, n)).astype(np.float16)
    b = (rng.choice([-1.0, 1.0], n) * rng.uniform(1e-4, 2e-4, n)).astype(np.float16)
    a[:4], b[:4] = np.array([-0.0, 0.0, -0.0, 0.0], np.float16), np.array([1.0, -1.0, -2.0, 3.0], np.float16)
    got, ref = _both(["%r = arith.mulf %a, %b : {T_f16}"], ["f16", "f16"], "f16", [a, b])
    assert np.signbit(ref).sum() > n // 4          # the oracle's -0 results
    _bits_equal(got, ref)
