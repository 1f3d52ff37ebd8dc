"""GPU parity for scalars read from tile data (tensor.extract, reductions
over every axis) and the scalar ops, splats and fills that use them, on the
kernels whose oracle results tests/test_oracle_scalar_pins.py pins.

Such a scalar stays on the device (ktir_cpu_amd.executor.DevScalar): the
lockstep walk does not stop to read it, so the plans here run in lockstep
mode, one fused launch per step where the reference pattern allows.  A
scalar that host code must read (here: float64 math on a reduction's Python
float) still takes the core-by-core path; those cases check that the
result is the same.  Scalar arithmetic, splats and fills are bit-exact
against the oracle; transcendentals meet the bars of the same ops on tiles
(tests/test_gpu_elementwise.py)."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases as C
from tests.test_oracle_scalar_pins import (extract_rmsnorm_rows, extract_softmax_closed_form, rows)

pytestmark = pytest.mark.gpu

_NP = {"f16": np.float16, "f32": np.float32}


def _bits_equal(got, ref, what):
    if got.dtype.kind == "f":
        u = {2: np.uint16, 4: np.uint32}[got.dtype.itemsize]
        nan = np.isnan(got) & np.isnan(ref)
        got, ref = np.where(nan, 0, got.view(u)), np.where(nan, 0, ref.view(u))
    np.testing.assert_array_equal(got, ref, err_msg=what)


def _both(src, fn, out, **kw):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})[out]
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function(fn, **kw)[out]
    print("  ", g.last_plan.mode, g.last_plan.counts(), g.last_plan.fallback_reason, flush=True)
    return got, ref, g.last_plan


# (name, body, dtype, out dtype, index of %s, fill, stays on the device[, bar])
# A scalar truncf from f32 to f16 is read on the host: the reference raises
# OverflowError for a value f16 cannot hold (test below).
# bar: bit-exact unless named; "f32ulp": an f32 transcendental of ROCm's
# device library against NumPy's float32 kernel, within 4 f32 ulps;
# "f16ulp": a transcendental rounded to f16, within one f16 ulp (the
# north star's bar; the f16 scalar ops after it are exact)
CHAINS = [
    ("add", "    %r = arith.addf %s, %t : {dt}", "f32", "f32", "%c0", False, True),
    ("sub_f16", "    %r = arith.subf %s, %t : {dt}", "f16", "f16", "%c0", False, True),
    ("mul", "    %r = arith.mulf %s, %t : {dt}", "f32", "f32", "%c0", False, True),
    ("div_const", "    %n = arith.constant 16.0 : {dt}\n    %r = arith.divf %s, %n : {dt}", "f32", "f32", "%c0",
     False, True),
    ("rem", "    %r = arith.remf %s, %t : {dt}", "f32", "f32", "%c0", False, True),
    ("tiny_const", "    %k = arith.constant 1.0e-8 : {dt}\n    %r = arith.addf %s, %k : {dt}", "f32", "f32", "%c0",
     False, True),
    ("max_const", "    %k = arith.constant 0.1 : {dt}\n    %r = arith.maximumf %s, %k : {dt}", "f32", "f32", "%c0",
     False, True),
    ("min_f16_const", "    %k = arith.constant 0.1 : {dt}\n    %r = arith.minimumf %s, %k : {dt}", "f16", "f32",
     "%c0", False, True),
    ("maxnum_mixed", "    %h = arith.truncf %t : f32 to f16\n    %r = arith.maxnumf %s, %h : {dt}", "f32", "f32",
     "%c0", False, False),
    ("trunc_f16_kept", "    %h = arith.truncf %s : f16 to f16\n    %r = arith.addf %h, %t : {dt}", "f16", "f16",
     "%c0", False, True),
    ("exp_f32", "    %r = math.exp %s : {dt}", "f32", "f32", "%c0", False, True, "f32ulp"),
    ("sqrt_f16", "    %a = math.absf %s : {dt}\n    %r = math.sqrt %a : {dt}", "f16", "f16", "%c0", False, True),
    ("rsqrt_chain", "    %a = arith.mulf %s, %s : {dt}\n    %e = arith.constant 1.0e-3 : {dt}\n"
                    "    %b = arith.addf %a, %e : {dt}\n    %r = math.rsqrt %b : {dt}", "f32", "f32", "%c0", False,
     True, "f16ulp"),
    ("neg_abs", "    %a = math.absf %s : {dt}\n    %r = arith.negf %a : {dt}", "f32", "f32", "%c0", False, True),
    ("weak_add", "    %r = arith.addf %u, %t : {dt}", "f32", "f32", "%c0", False, True),
    ("weak_neg", "    %r = arith.negf %u : {dt}", "f16", "f32", "%c0", False, True),
    ("tile_outs_sqrt", "    %r = math.sqrt %v : tensor<1x{dt}>", "f16", "f32", "%c0", False, True),
    ("per_core_index", "    %r = arith.addf %s, %s : {dt}", "f32", "f32", "%i_core", False, True),
    ("splat_i32", "    %r = arith.addf %s, %t : {dt}", "f32", "i32", "%c0", False, True),
    ("splat_bf16", "    %r = math.absf %s : {dt}", "f32", "bf16", "%c0", False, True),
    ("fill_f16", "    %r = math.absf %s : {dt}", "f32", "f16", "%c0", True, True),
    ("tile_times_scalar", "    %rb = arith.mulf %x, %s : tensor<1x16x{dt}>", "f32", "f32", "%c0", False, True),
    ("weak_sqrt_on_host", "    %r = math.sqrt %u : {dt}", "f32", "f32", "%c0", False, False),
]


def _chain_inputs(dt, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((8, 16)) * 10.0 ** rng.integers(-3, 4, (8, 16))
    special = rows((1e-8, 1e-8), (300.0, 300.0), (1 / 3, 3.0), (5.5, -2.0), (np.nan, 1.0), (2049.0, 0.5),
                   (70000.0, 0.0), (-2.75, 0.0))
    x = np.concatenate([x, special])
    return x.astype(_NP[dt])


def _within(got, ref, bar, what):
    if bar == "bits":
        _bits_equal(got, ref, what)
        return
    g, r = got.astype(np.float64), ref.astype(np.float64)
    both_nan = np.isnan(g) & np.isnan(r)
    if bar == "f32ulp":
        ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) * 4
    else:
        ulp = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float64)
    bad = ~both_nan & ~(np.abs(g - r) <= ulp) & ~(g == r)
    assert not bad.any(), (what, g[bad][:8], r[bad][:8])


@pytest.mark.parametrize("name,body,dt,out_dt,idx,fill,on_device,bar",
                         [c + ("bits",) * (8 - len(c)) for c in CHAINS], ids=[c[0] for c in CHAINS])
def test_scalar_chain_against_oracle(name, body, dt, out_dt, idx, fill, on_device, bar):
    from oracle.interp import bf16_bits
    x = _chain_inputs(dt, seed=len(name))
    cores, cols = x.shape
    src, fn = C.scalar_chain(body, dt=dt, out_dt=out_dt, cores=cores, C=cols, idx=idx, fill=fill)
    if out_dt == "bf16":
        y0 = np.zeros((cores, cols), np.uint16)
    else:
        y0 = np.zeros((cores, cols), np.int32 if out_dt == "i32" else _NP[out_dt])
    print(name, dt, out_dt, flush=True)
    with np.errstate(all="ignore"):
        got, ref, plan = _both(src, fn, "y_ptr", x_ptr=x, y_ptr=y0)
    if out_dt == "bf16":
        np.testing.assert_array_equal(got, ref)
        # the element rounded once into bf16
        np.testing.assert_array_equal(got[:, 0], bf16_bits(np.abs(x[:, 0]).astype(np.float32)))
    else:
        _within(got, ref, bar, name)
    assert (plan.mode == "lockstep") == on_device, (plan.mode, plan.fallback_reason)


@pytest.mark.parametrize("rows_,cols,cores", [(64, 256, 8), (4096, 1024, 32)])
def test_softmax_extract_closed_form_and_oracle(rows_, cols, cores):
    """The reference's triton-ktir softmax_fwd form: exact on the closed-form
    rows, bit-exact against the oracle on random rows, one lockstep plan."""
    from ktir_cpu_amd import configs
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    from tests.test_oracle_linalg_pins import broadcast_softmax_rows
    src = configs.softmax_extract(rows_, cols, cores)
    print("softmax_extract", rows_, cols, cores, flush=True)
    g = KTIRInterpreter()
    g.load(src)
    x = broadcast_softmax_rows(rows_, cols).astype(np.float16)
    got = g.execute_function("softmax_fwd", x_ptr=x, y_ptr=np.zeros_like(x), n_rows=rows_)["y_ptr"]
    assert g.last_plan.mode == "lockstep", g.last_plan.fallback_reason
    extract_softmax_closed_form(got, rows_, cols)
    if rows_ <= 64:
        x = (np.random.default_rng(2).standard_normal((rows_, cols)) * 3).astype(np.float16)
        got, ref, plan = _both(src, "softmax_fwd", "y_ptr", x_ptr=x, y_ptr=np.zeros_like(x), n_rows=rows_)
        _bits_equal(got, ref, "softmax_extract")
        assert plan.mode == "lockstep"


def test_softmax_extract_full_reference_size_rows_sampled():
    """At the reference example's own size (4096 x 1024, grid 32), against
    the oracle run on a sample of cores (each core's rows are its own)."""
    from ktir_cpu_amd import configs
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    rows_, cols, cores = 4096, 1024, 32
    src = configs.softmax_extract(rows_, cols, cores)
    x = (np.random.default_rng(3).standard_normal((rows_, cols)) * 3).astype(np.float16)
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function("softmax_fwd", x_ptr=x, y_ptr=np.zeros_like(x), n_rows=rows_)["y_ptr"]
    assert g.last_plan.mode == "lockstep"
    o = OracleInterpreter()
    o.load(src)
    o.cores_to_run = [0, 13, 31]
    ref = o.execute_function("softmax_fwd", x_ptr=x.copy(), y_ptr=np.zeros_like(x), n_rows=rows_)["y_ptr"]
    for c in o.cores_to_run:
        _bits_equal(got[c::cores], ref[c::cores], f"core {c}")


@pytest.mark.parametrize("rows_,cols,cores", [(40, 256, 8), (20, 16, 4)])
def test_rmsnorm_extract_closed_form_and_oracle(rows_, cols, cores):
    from ktir_cpu_amd import configs
    src = configs.rmsnorm_extract(rows_, cols, cores)
    print("rmsnorm_extract", rows_, cols, cores, flush=True)
    x, w, sg = extract_rmsnorm_rows(rows_, cols)
    got, ref, plan = _both(src, "rmsnorm_fwd", "y_ptr", x_ptr=x, w_ptr=w.reshape(1, cols), y_ptr=np.zeros_like(x),
                           n_rows=rows_, eps=0.0)
    np.testing.assert_array_equal(got, (sg[:, None] * w[None, :]).astype(np.float16))
    _bits_equal(got, ref, "closed form")
    assert plan.mode == "lockstep"
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((rows_, cols)) * 2).astype(np.float16)
    got, ref, plan = _both(src, "rmsnorm_fwd", "y_ptr", x_ptr=x, w_ptr=w.reshape(1, cols), y_ptr=np.zeros_like(x),
                           n_rows=rows_, eps=1e-3)
    _bits_equal(got, ref, "random rows")
    assert plan.mode == "lockstep"


def test_extract_index_out_of_range_raises_before_launch():
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn = C.scalar_chain("    %r = arith.addf %s, %t : {dt}", cores=4, C=16, idx="%cC")
    g = KTIRInterpreter()
    g.load(src)
    with pytest.raises(IndexError):
        g.execute_function(fn, x_ptr=np.zeros((4, 16), np.float32), y_ptr=np.zeros((4, 16), np.float32))


def test_scalar_truncf_overflow_raises_like_the_reference():
    """truncf of a scalar that f16 cannot hold raises OverflowError (reference
    ops/arith_ops.py:38-87); 65519 still rounds to 65504."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    body = "    %h = arith.truncf %s : f32 to f16\n    %r = arith.extf %h : f16 to f32"
    src, fn = C.scalar_chain(body, cores=2, C=16)
    for x, raises in ((rows((1.5, 0.0), (70000.0, 0.0)), True), (rows((1.5, 0.0), (65519.0, 0.0)), False)):
        x = x.astype(np.float32)
        kw = dict(x_ptr=x, y_ptr=np.zeros_like(x))
        if raises:
            o = OracleInterpreter()
            o.load(src)
            with pytest.raises(OverflowError):
                o.execute_function(fn, **{k: v.copy() for k, v in kw.items()})
            g = KTIRInterpreter()
            g.load(src)
            with pytest.raises(OverflowError):
                g.execute_function(fn, **kw)
        else:
            got, ref, _ = _both(src, fn, "y_ptr", **kw)
            _bits_equal(got, ref, "truncf")
            assert got[1, 0] == 65504.0


def test_softmax_extract_row_wave_against_oracle():
    """1024-element rows take the row-wave kernel's instantiation for f16
    folds: within 2 f16 ulps of the oracle (its exponential is the hardware
    exp2 rounded to f16, within one f16 ulp of NumPy's), most outputs equal."""
    from ktir_cpu_amd import configs
    rows_, cols, cores = 128, 1024, 16
    src = configs.softmax_extract(rows_, cols, cores)
    x = (np.random.default_rng(5).standard_normal((rows_, cols)) * 3).astype(np.float16)
    got, ref, plan = _both(src, "softmax_fwd", "y_ptr", x_ptr=x, y_ptr=np.zeros_like(x), n_rows=rows_)
    assert plan.mode == "lockstep" and plan.counts() == {"prog": 1}
    d = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert d.max() <= 2, d.max()
    assert (d == 0).mean() > 0.9


def test_rmsnorm_extract_row_wave_bit_exact():
    """2048-element rows: f16 squares, an f16 pairwise sum, the scalar chain
    on the row values and two f16 products, bit for bit."""
    from ktir_cpu_amd import configs
    rows_, cols, cores = 64, 2048, 8
    src = configs.rmsnorm_extract(rows_, cols, cores)
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((rows_, cols)) * 2).astype(np.float16)
    w = rng.uniform(0.5, 1.5, (1, cols)).astype(np.float16)
    got, ref, plan = _both(src, "rmsnorm_fwd", "y_ptr", x_ptr=x, w_ptr=w, y_ptr=np.zeros_like(x), n_rows=rows_,
                           eps=1e-3)
    assert plan.mode == "lockstep" and plan.counts() == {"prog": 1}
    _bits_equal(got, ref, "rmsnorm_extract")


@pytest.mark.parametrize("rows_,cols,blk,cores", [(70, 512, 128, 8), (1151, 8192, 1024, 32)])
def test_layernorm_extract_bit_exact(rows_, cols, blk, cores):
    """The reference's layernorm_fwd form: loop-carried f16 block sums,
    mean and rstd as one-element tensors read by tensor.extract, both
    stored, then the normalised rows; bit for bit against the oracle (on
    sampled cores at the example's own size), within f16 rounding of the
    float64 LayerNorm."""
    from ktir_cpu_amd import configs
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src = configs.layernorm_extract(rows_, cols, blk, cores)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((rows_, cols)) * 2 + 1).astype(np.float16)
    w = rng.uniform(0.5, 1.5, (rows_, cols)).astype(np.float16)
    b = rng.standard_normal((rows_, cols)).astype(np.float16)
    kw = dict(x_ptr=x, y_ptr=np.zeros_like(x), w_ptr=w, b_ptr=b, mean_ptr=np.zeros(rows_, np.float16),
              rstd_ptr=np.zeros(rows_, np.float16), n_cols=cols, eps=1e-5, blk=blk)
    print("layernorm_extract", rows_, cols, blk, cores, flush=True)
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function("layernorm_fwd", **kw)
    print("  ", g.last_plan.mode, g.last_plan.counts(), g.last_plan.fallback_reason, flush=True)
    assert g.last_plan.mode == "lockstep"
    o = OracleInterpreter()
    o.load(src)
    if rows_ > 100:
        o.cores_to_run = [0, 17, 31]
    ref = o.execute_function("layernorm_fwd", **{k: (v.copy() if isinstance(v, np.ndarray) else v)
                                                 for k, v in kw.items()})
    sel = np.concatenate([np.arange(c, rows_, cores) for c in (o.cores_to_run or range(cores))])
    for k in ("y_ptr", "mean_ptr", "rstd_ptr"):
        _bits_equal(got[k][sel], ref[k][sel], k)
    xf = x.astype(np.float64)
    want = (xf - xf.mean(1, keepdims=True)) / np.sqrt(xf.var(1, keepdims=True) + 1e-5) * w + b
    np.testing.assert_allclose(got["y_ptr"].astype(np.float64), want, atol=0.05, rtol=0.02)
