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


# ---------------------------------------------------------------------------
# elementwise arithmetic: closed forms and IEEE definitions
# ---------------------------------------------------------------------------

def _ew(body, ins, out_dt, arrays, n=None):
    n = n or len(arrays[0])
    src, fn, names = _cases.elementwise(body, ins, out_dt, n=n)
    out_np = {"f16": np.float16, "f32": np.float32, "bf16": np.uint16, "i1": np.bool_}[out_dt]
    kw = dict(zip(names, list(arrays) + [np.zeros(n, out_np)]))
    return _exec((src, fn, kw))["r_ptr"]


def _same_f16(got, want):
    """Bit-equal, except that any NaN matches any NaN."""
    g, w = np.asarray(got, np.float16), np.asarray(want, np.float16)
    both_nan = np.isnan(g) & np.isnan(w)
    np.testing.assert_array_equal(np.where(both_nan, 0, g.view(np.uint16)), np.where(both_nan, 0, w.view(np.uint16)))


@pytest.mark.parametrize("op,fn", [("arith.addf", np.add), ("arith.subf", np.subtract),
                                   ("arith.mulf", np.multiply), ("arith.divf", np.divide)])
def test_oracle_f16_binops_correctly_rounded(op, fn):
    """f16 tile arithmetic equals the float64 result rounded once to f16 (round
    to nearest even).  Sums, differences and products of f16 values are exact
    in float64; a float64 quotient of 11-bit significands is never within
    2^-53 of an f16 rounding boundary unless it lies on one, so one rounding of
    it is the correctly rounded quotient.  Swapped operands (sub, div),
    truncation or a rounding in between fail this."""
    n = 1 << 15
    a, b = _cases.f16_patterns(n, seed=1), _cases.f16_patterns(n, seed=2)
    got = _ew([f"%r = {op} %a, %b : {{T_f16}}"], ["f16", "f16"], "f16", [a, b])
    with np.errstate(all="ignore"):
        want = fn(a.astype(np.float64), b.astype(np.float64)).astype(np.float16)
    _same_f16(got, want)


def _bf16_round_exact(x):
    """Round-to-nearest-even of float32 values to bf16, from the two bf16
    neighbours of each value and float64 distances (no bit tricks)."""
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32)
    lo_bits = u & np.uint32(0xFFFF0000)                 # toward zero
    lo = lo_bits.view(np.float32).astype(np.float64)
    mag_hi_bits = (lo_bits & np.uint32(0x7FFF0000)) + np.uint32(0x10000)
    hi = np.where(mag_hi_bits >= 0x7F800000, 2.0 ** 128,
                  (mag_hi_bits | np.uint32(0)).view(np.float32).astype(np.float64))
    hi = np.copysign(hi, x.astype(np.float64))
    xd = x.astype(np.float64)
    d_lo, d_hi = np.abs(xd - lo), np.abs(hi - xd)
    lo_even = ((lo_bits >> np.uint32(16)) & np.uint32(1)) == 0
    take_lo = (d_lo < d_hi) | ((d_lo == d_hi) & lo_even)
    r = np.where(take_lo, lo, hi)
    with np.errstate(over="ignore"):
        r = r.astype(np.float32)                          # 2^128 becomes inf
    return np.where(np.isnan(x), np.float32(np.nan), r)


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
def test_oracle_bf16_round_against_exact_rounding():
    """bf16_round (the oracle's bf16 storage rounding) against round to nearest
    even computed from the neighbours: every high half of a float32 with low
    halves at and around the tie (0x7FFF, 0x8000, 0x8001), 0, 0xFFFF and
    random values; infinities, overflow to infinity and NaN included."""
    from oracle.interp import bf16_round
    hi = np.arange(1 << 16, dtype=np.uint32) << np.uint32(16)
    lows = [0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF] + \
        list(np.random.default_rng(3).integers(0, 1 << 16, 4))
    u = (hi[:, None] | np.asarray(lows, np.uint32)[None, :]).reshape(-1)
    x = u.view(np.float32)
    got, want = bf16_round(x), _bf16_round_exact(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # a signaling NaN whose payload is only in the low half stays a NaN
    snan = np.array([0x7F800001, 0xFF800100], np.uint32).view(np.float32)
    assert np.isnan(bf16_from_bits(bf16_bits(snan))).all()


def test_oracle_erf_within_abramowitz_stegun_bound():
    """math.erf is A&S 7.1.26 (reference ops/math_ops.py:100-106), whose
    absolute error is at most 1.5e-7; evaluated in f32 it stays within 4e-7
    of the exact erf.  A dropped sign, a wrong coefficient or exp(-x) for
    exp(-x^2) is off by far more."""
    import math
    x = np.concatenate([np.linspace(-6, 6, 8191), [0.0]]).astype(np.float32)
    got = _ew(["%r = math.erf %a : {T_f32}"], ["f32"], "f32", [x]).astype(np.float64)
    want = np.array([math.erf(float(v)) for v in x])
    assert np.max(np.abs(got - want)) <= 4e-7


_F32_MATH = [("math.exp", np.exp, (-80, 80)), ("math.log", np.log, (1e-30, 1e30)),
             ("math.log2", np.log2, (1e-30, 1e30)), ("math.log1p", np.log1p, (-0.999, 1e6)),
             ("math.tanh", np.tanh, (-12, 12)), ("math.sin", np.sin, (-100, 100)),
             ("math.cos", np.cos, (-100, 100)), ("math.sqrt", np.sqrt, (0, 1e30))]


@pytest.mark.parametrize("op,f64,rng_", _F32_MATH)
def test_oracle_f32_math_against_float64(op, f64, rng_):
    """f32 transcendentals within 4 f32 ulps of the float64 function (NumPy's
    float32 kernels, which the reference calls, are within a few ulps; a wrong
    function or base is off by orders of magnitude)."""
    lo, hi = rng_
    if lo > 0:
        x = np.geomspace(lo, hi, 4096).astype(np.float32)
    else:
        x = np.linspace(lo, hi, 4096).astype(np.float32)
    got = _ew([f"%r = {op} %a : {{T_f32}}"], ["f32"], "f32", [x]).astype(np.float64)
    want = f64(x.astype(np.float64))
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    tol = 4 * ulp + (1e-6 if op in ("math.sin", "math.cos") else 0.0)
    assert np.all(np.abs(got - want) <= tol), op


@pytest.mark.parametrize("op,f64", [("math.exp", np.exp), ("math.tanh", np.tanh), ("math.sin", np.sin),
                                    ("math.log", np.log), ("math.sqrt", np.sqrt)])
def test_oracle_f16_math_within_one_ulp(op, f64):
    """On f16 tiles the reference evaluates in float32 and rounds to f16, so
    the result is within one f16 ulp of the float64 function."""
    x = np.linspace(0.01 if op in ("math.log", "math.sqrt") else -8, 8, 4096).astype(np.float16)
    got = _ew([f"%r = {op} %a : {{T_f16}}"], ["f16"], "f16", [x]).astype(np.float64)
    want = f64(x.astype(np.float64))
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp), op


_PRED = {"oeq": "E", "ogt": "G", "oge": "GE", "olt": "L", "ole": "LE", "one": "LG", "ord": "LEG",
         "ueq": "EU", "ugt": "GU", "uge": "GEU", "ult": "LU", "ule": "LEU", "une": "LGU", "uno": "U",
         "true": "LEGU", "false": ""}


def _cmp_pairs():
    vals = [0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan, 1e-40, 3.0e38]
    a, b = np.meshgrid(np.array(vals, np.float32), np.array(vals, np.float32))
    a, b = a.reshape(-1), b.reshape(-1)
    reps = 4096 // a.size + 1
    return np.tile(a, reps)[:4096], np.tile(b, reps)[:4096]


@pytest.mark.parametrize("pred", sorted(_PRED))
def test_oracle_cmpf_select_ieee_table(pred):
    """arith.cmpf + arith.select against IEEE 754 relations: every pair of
    values (zeros of both signs, infinities, NaN, subnormals) is less, equal,
    greater or unordered; an ordered predicate is false and an unordered one
    true when a NaN is involved.  select(c, a, b) picks a where c holds."""
    import math
    a, b = _cmp_pairs()
    got = _ew([f"%c = arith.cmpf {pred}, %a, %b : {{T_f32}}",
               "%r = arith.select %c, %a, %b : {T_i1}, {T_f32}"], ["f32", "f32"], "f32", [a, b])

    def rel(x, y):
        x, y = float(x), float(y)
        return "U" if math.isnan(x) or math.isnan(y) else "L" if x < y else "E" if x == y else "G"
    holds = np.array([rel(x, y) in _PRED[pred] for x, y in zip(a, b)])
    want = np.where(holds, a, b)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("op", ["arith.maximumf", "arith.minimumf", "arith.maxnumf", "arith.minnumf"])
def test_oracle_min_max_nan_rules(op):
    """maximumf / minimumf propagate NaN (IEEE 754-2019 maximum, minimum);
    maxnumf / minnumf return the other operand when one is NaN (maxNum,
    minNum).  Values otherwise: the larger / smaller."""
    import math
    a, b = _cmp_pairs()
    got = _ew([f"%r = {op} %a, %b : {{T_f32}}"], ["f32", "f32"], "f32", [a, b]).astype(np.float64)
    for x, y, g in zip(a.astype(np.float64), b.astype(np.float64), got):
        big = op in ("arith.maximumf", "arith.maxnumf")
        if math.isnan(x) or math.isnan(y):
            if op in ("arith.maximumf", "arith.minimumf") or (math.isnan(x) and math.isnan(y)):
                assert math.isnan(g)
            else:
                assert g == (y if math.isnan(x) else x)
        else:
            assert g == (max(x, y) if big else min(x, y))


# ---------------------------------------------------------------------------
# the gather + scatter-add composition, brute force
# ---------------------------------------------------------------------------

def _scatter_add_brute_force(table, idx, out, cores, chunk):
    """Per core in id order, per chunk in order: every position k of the chunk
    reads its destination row as it was before the chunk and its table row,
    adds in f32 and stores; stores go in k order, so a row repeated inside a
    chunk keeps its last position's value (last writer wins) and repeats
    across chunks accumulate one after another."""
    out = out.astype(np.float32).copy()
    per_core = len(idx) // cores
    for c in range(cores):
        for s in range(0, per_core, chunk):
            ks = idx[c * per_core + s: c * per_core + s + chunk]
            before = {int(r): out[r].copy() for r in ks}
            for r in ks:
                r = int(r)
                out[r] = (before[r] + table[r].astype(np.float32)).astype(np.float32)
    return out


@pytest.mark.parametrize("rows,dim,n_idx,cores,chunk,hot", [(64, 8, 64, 2, 8, 64), (200, 16, 96, 4, 8, 5),
                                                           (96, 128, 64, 2, 16, 3)])
def test_oracle_gather_scatter_add_against_brute_force(rows, dim, n_idx, cores, chunk, hot):
    """The config-2 kernel (indirect row gather of the table, indirect row load
    of the output, extf + addf, indirect store) against a per-row Python loop:
    in-chunk duplicates keep the last writer, duplicates across chunks and
    cores accumulate in core and chunk order, with f32 sums.  `hot` bounds the
    index range so duplicates are frequent."""
    rng = np.random.default_rng(rows)
    src, fn, kw = _cases.gather_scatter_add(rows=rows, dim=dim, n_idx=n_idx, cores=cores, chunk=chunk)
    kw["idx_ptr"] = rng.integers(0, hot, n_idx).astype(np.int32)
    kw["out_ptr"] = rng.standard_normal((rows, dim)).astype(np.float32)
    want = _scatter_add_brute_force(kw["table_ptr"], kw["idx_ptr"], kw["out_ptr"], cores, chunk)
    got = _exec((src, fn, kw))["out_ptr"]
    np.testing.assert_array_equal(got, want)
    # a last-writer-wins mistake (accumulating in-chunk repeats) would differ
    assert len(np.unique(kw["idx_ptr"][:chunk])) < chunk or hot >= n_idx


@pytest.mark.parametrize("dim,hot", [(8, 6), (16, 96)])
def test_oracle_scatter_add_two_index_against_brute_force(dim, hot):
    """The same kernel with the source rows named by a second index tensor:
    the updates of one destination row add different table rows, so a wrong
    order (or a wrong source) shows in the f32 sums.  Against a per-row loop:
    each chunk reads its destination rows before any of its stores, the last
    position of a row in a chunk writes, chunks and cores follow in order."""
    src, fn, kw = _cases.scatter_add_two_index(rows=96, dim=dim, n_idx=64, cores=2, chunk=8, seed=dim, hot=hot)
    d, s = kw["idx_ptr"], kw["sidx_ptr"]
    table = kw["table_ptr"].astype(np.float32)
    want = kw["out_ptr"].astype(np.float32).copy()
    per_core = len(d) // 2
    for c in range(2):
        for b in range(c * per_core, (c + 1) * per_core, 8):
            new = {}
            before = {int(r): want[r].copy() for r in d[b:b + 8]}
            for k in range(b, b + 8):
                new[int(d[k])] = (before[int(d[k])] + table[int(s[k])]).astype(np.float32)
            for r, v in new.items():
                want[r] = v
    got = _exec((src, fn, kw))["out_ptr"]
    np.testing.assert_array_equal(got, want)
    # the sources of one destination row differ (else this would not test the order)
    assert any(len(set(s[d == r])) > 1 for r in np.unique(d))


def _splat_kernel(dt, const):
    return f"""module {{
  func.func @splat_kernel(%out_ptr: index) attributes {{grid = [1, 1]}} {{
    %c = arith.constant {const} : {dt}
    %z = arith.constant 0 : index
    %v = ktdp.construct_memory_view %out_ptr, sizes: [4, 8], strides: [8, 1] {{
      coordinate_set = affine_set<(d0, d1) : (d0 >= 0, -d0 + 3 >= 0, d1 >= 0, -d1 + 7 >= 0)>, memory_space = #ktdp.memory_space<global>
    }} : memref<4x8x{dt}>
    %t = tensor.splat %c : tensor<4x8x{dt}>
    %tile = ktdp.construct_access_tile %v[%z, %z] {{
      access_tile_set = affine_set<(d0, d1) : (d0 >= 0, -d0 + 3 >= 0, d1 >= 0, -d1 + 7 >= 0)>,
      access_tile_order = affine_map<(d0, d1) -> (d0, d1)>
    }} : memref<4x8x{dt}> -> !ktdp.access_tile<4x8xindex>
    ktdp.store %t, %tile : tensor<4x8x{dt}>, !ktdp.access_tile<4x8xindex>
    return
  }}
}}
"""


@pytest.mark.parametrize("dt,const,np_dt", [("f32", "2.5", np.float32), ("f16", "0.1", np.float16),
                                            ("i32", "-7", np.int32)])
def test_oracle_splat_takes_shape_and_dtype_from_result_type(dt, const, np_dt):
    """tensor.splat fills the result type's shape with the scalar in the
    result's dtype (reference dialects/tensor_ops.py:57-84): every stored
    element equals np.full of that shape (0.1 rounded once to f16)."""
    o = OracleInterpreter()
    o.load(_splat_kernel(dt, const))
    out = o.execute_function("splat_kernel", out_ptr=np.full((4, 8), 99, np_dt))["out_ptr"]
    want = np.full((4, 8), np_dt(float(const)) if np_dt is not np.int32 else int(const), np_dt)
    assert out.dtype == np_dt
    np.testing.assert_array_equal(out, want)
