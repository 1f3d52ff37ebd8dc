"""GPU parity: the five benchmark kernels through the HIP backend vs the oracle.

Bars (north star): bit-exact for load/store/gather/scatter and integer work;
rtol 1e-2 / atol 1e-3 for reductions, softmax, matmul and attention.
"""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter, bf16_from_bits
from tests import _cases

pytestmark = pytest.mark.gpu


def _run(case):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw = case
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})
    g = KTIRInterpreter()
    g.load(src)
    out = g.execute_function(fn, **kw)
    print(fn, g.last_plan.mode, g.last_plan.counts(), g.last_plan.fallback_reason, flush=True)
    return ref, out, g


@pytest.mark.parametrize("n,block,cores", [(4096, 128, 32), (4096, 128, 1), (1 << 16, 128, 32), (1 << 16, 1024, 64)])
def test_vector_add_bit_exact(n, block, cores):
    ref, out, _ = _run(_cases.vector_add(n, block, cores))
    np.testing.assert_array_equal(out["output_ptr"], ref["output_ptr"])
    np.testing.assert_array_equal(out["x_ptr"], ref["x_ptr"])


def _rmw_kernel(dim):
    """The apply kernel the ordered row RMW takes for f32 rows of `dim` columns."""
    return "rows" if dim % 128 == 0 else "generic"


@pytest.mark.parametrize("dim", [32, 128, 256])
def test_gather_scatter_add_bit_exact(dim):
    ref, out, g = _run(_cases.gather_scatter_add(dim=dim))
    np.testing.assert_array_equal(out["out_ptr"], ref["out_ptr"])
    assert g.last_plan.counts() == {"rmw": 1}
    assert g.last_plan.rmw_variants() == [_rmw_kernel(dim)]


@pytest.mark.parametrize("dim", [32, 128])
@pytest.mark.parametrize("rows", [16, 3])
def test_gather_scatter_add_heavy_duplicates(rows, dim):
    """Many repeats inside one chunk (last writer wins) and long per-row chains
    across chunks and cores (sequential accumulation order)."""
    src, fn, kw = _cases.gather_scatter_add(rows=1024, dim=dim, n_idx=512, cores=4, chunk=32)
    rng = np.random.default_rng(7)
    kw["idx_ptr"] = rng.integers(0, rows, 512).astype(np.int32)
    kw["out_ptr"] = rng.standard_normal((1024, dim)).astype(np.float32)
    ref, out, g = _run((src, fn, kw))
    np.testing.assert_array_equal(out["out_ptr"], ref["out_ptr"])
    assert g.last_plan.rmw_variants() == [_rmw_kernel(dim)]


@pytest.mark.parametrize("dim", [32, 128, 256])
@pytest.mark.parametrize("hot", [None, 24])
def test_scatter_add_two_index_bit_exact(dim, hot):
    """Source rows from a second index tensor: the updates of one destination
    row add different rows, in the reference's order (last writer inside a
    chunk, instance after instance), bit-exact; with `hot`, every destination
    row takes a long chain (the chain path of the row-order kernel)."""
    print(f"[rmw] two-index dim {dim} hot {hot}", flush=True)
    ref, out, g = _run(_cases.scatter_add_two_index(dim=dim, hot=hot))
    np.testing.assert_array_equal(out["out_ptr"], ref["out_ptr"])
    assert g.last_plan.counts() == {"rmw": 1}
    assert g.last_plan.rmw_variants() == [_rmw_kernel(dim)]


@pytest.mark.parametrize("dim", [32, 128])
def test_gather_scatter_add_rows_past_allocation(dim):
    """Indices past the end of the table read zero rows, and a destination
    allocation that ends inside its last row drops the columns past its end
    (reference memory.py:243-305), in both apply kernels."""
    src, fn, kw = _cases.gather_scatter_add(rows=1024, dim=dim, n_idx=512, cores=4, chunk=32)
    rng = np.random.default_rng(11)
    kw["table_ptr"] = kw["table_ptr"][:700].copy()          # rows 700.. of the table view are past its end
    kw["idx_ptr"] = np.concatenate([rng.integers(600, 1024, 500), [1023] * 12]).astype(np.int32)
    kw["out_ptr"] = rng.standard_normal(1024 * dim - 24).astype(np.float32)   # last row ends 24 columns short
    ref, out, g = _run((src, fn, kw))
    np.testing.assert_array_equal(out["out_ptr"], ref["out_ptr"])
    np.testing.assert_array_equal(out["table_ptr"], ref["table_ptr"])
    assert g.last_plan.rmw_variants() == [_rmw_kernel(dim)]


@pytest.mark.parametrize("dim", [32, 128])
def test_blocked_indirect_gather_bit_exact(dim):
    """The unfused blocked-indirect row gather (indirect load, then a plain
    store): bit-exact, and equal to table[idx] (reference
    ops/memory_ops.py:224-486)."""
    src, fn, kw = _cases.gather_rows(dim=dim)
    ref, out, g = _run((src, fn, kw))
    np.testing.assert_array_equal(out["out_ptr"], ref["out_ptr"])
    np.testing.assert_array_equal(out["out_ptr"], kw["table_ptr"][kw["idx_ptr"]])
    assert "rmw" not in g.last_plan.counts()


@pytest.mark.parametrize("dim", [32, 128])
def test_gather_scatter_add_negative_index_raises(dim):
    """A negative index raises IndexError (reference ops/memory_ops.py:378-382)."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw = _cases.gather_scatter_add(rows=1024, dim=dim, n_idx=512, cores=4, chunk=32)
    kw["idx_ptr"][77] = -5
    g = KTIRInterpreter()
    g.load(src)
    with pytest.raises(IndexError):
        g.execute_function(fn, **kw)


@pytest.mark.parametrize("cols", [256, 4096])
def test_softmax(cols):
    ref, out, _ = _run(_cases.softmax(cols=cols))
    np.testing.assert_allclose(out["y_ptr"].astype(np.float32), ref["y_ptr"].astype(np.float32), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("cols", [256, 4096])
def test_rmsnorm(cols):
    ref, out, _ = _run(_cases.rmsnorm(cols=cols))
    np.testing.assert_allclose(out["y_ptr"].astype(np.float32), ref["y_ptr"].astype(np.float32), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("op", ["math.sqrt", "math.rsqrt"])
def test_sqrt_rsqrt_bit_exact(op):
    """f32 sqrt is correctly rounded (as NumPy's) and rsqrt is 1 / sqrt(x) with
    two correct roundings, over thirty decades either side of 1."""
    ref, out, _ = _run(_cases.unary_f32(op))
    np.testing.assert_array_equal(out["y_ptr"], ref["y_ptr"])


def _half_f32(x, dt):
    return bf16_from_bits(x) if dt == "bf16" else x.astype(np.float32)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 1024, 2048, 4096])
def test_softmax_fixed_form(cols, dt):
    """Softmax rows of 512 .. 4096 elements (the fixed-form row kernel), f16 and bf16."""
    ref, out, g = _run(_cases.softmax(rows=48, cols=cols, cores=4, dt=dt))
    assert g.last_plan.counts() == {"prog": 1}
    np.testing.assert_allclose(_half_f32(out["y_ptr"], dt), _half_f32(ref["y_ptr"], dt), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 4096, 256, 3000])
def test_softmax_fixed_form_large_and_non_finite_rows(cols, dt):
    """Rows whose maximum is 2048 or more (the exponent then takes x - m'
    first), rows holding +inf or NaN (a sum that is not finite: the plain
    quotient per element), a row whose maximum (40) only a max over every
    element finds (a smaller one would overflow the f16 exponentials), next to
    ordinary rows; NaN where the oracle has NaN.  256 and 3000 columns take
    the general row kernels."""
    from oracle.interp import bf16_bits
    src, fn, kw = _cases.softmax(rows=48, cols=cols, cores=4, dt=dt)
    x = _half_f32(kw["x_ptr"], dt).astype(np.float64)
    x[1::4] += 3000.0 if dt == "f16" else 1.0e6
    x[2::4] -= 3000.0 if dt == "f16" else 1.0e6
    x[3, 7] = np.inf
    x[7, 1] = np.nan
    x[11, :] = -np.inf
    x[4, 3] = 40.0          # the row max, in the second 32-bit word of its lane's chunk
    kw["x_ptr"] = x.astype(np.float16) if dt == "f16" else bf16_bits(x.astype(np.float32))
    print(f"[softmax] large / non-finite rows {cols} {dt}", flush=True)
    ref, out, g = _run((src, fn, kw))
    if cols in (512, 4096):
        assert g.last_plan.counts() == {"prog": 1}
    got, want = _half_f32(out["y_ptr"], dt), _half_f32(ref["y_ptr"], dt)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_allclose(np.nan_to_num(got), np.nan_to_num(want), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 4096])
def test_softmax_fixed_form_wide_range_relative_error(cols, dt):
    """Rows spanning 30 (exponentials down to e^-30, far below f16's normal
    range): a bf16 output is within rtol 1e-2 of every nonzero reference
    output with no absolute term (the kernel keeps f32 exponentials for
    bf16); an f16 output is within rtol 1e-2 plus one subnormal step 2^-24
    (its f16 exponentials lose relative precision only where the output
    itself is subnormal)."""
    from oracle.interp import bf16_bits
    src, fn, kw = _cases.softmax(rows=48, cols=cols, cores=4, dt=dt)
    rng = np.random.default_rng(21)
    x = rng.uniform(-30.0, 0.0, (48, cols))
    kw["x_ptr"] = x.astype(np.float16) if dt == "f16" else bf16_bits(x.astype(np.float32))
    print(f"[softmax] wide-range rows {cols} {dt}", flush=True)
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts() == {"prog": 1}
    got, want = _half_f32(out["y_ptr"], dt).astype(np.float64), _half_f32(ref["y_ptr"], dt).astype(np.float64)
    if dt == "bf16":
        nz = want != 0
        assert nz.mean() > 0.99
        assert np.all(np.abs(got[nz] - want[nz]) <= 1e-2 * np.abs(want[nz])), \
            np.max(np.abs(got[nz] - want[nz]) / np.abs(want[nz]))
    else:
        assert np.all(np.abs(got - want) <= 1e-2 * np.abs(want) + 2.0 ** -24)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 4096])
def test_rmsnorm_non_finite_and_zero_rows(cols, dt):
    """RMSNorm rows holding +inf or NaN, an all-zero row, and (bf16) values
    whose squares overflow f32: equal to the oracle bit for bit, NaN where it
    has NaN."""
    from oracle.interp import bf16_bits
    src, fn, kw = _cases.rmsnorm(rows=48, cols=cols, cores=4, dt=dt, wide=True)
    x = _half_f32(kw["x_ptr"], dt).astype(np.float64)
    x[2, 5] = np.inf
    x[9, 0] = np.nan
    x[13, :] = 0.0
    if dt == "bf16":
        x[17, 3] = 3.0e38
        x[21, :8] = -2.0e30
    kw["x_ptr"] = x.astype(np.float16) if dt == "f16" else bf16_bits(x.astype(np.float32))
    print(f"[rmsnorm] non-finite rows {cols} {dt}", flush=True)
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts() == {"prog": 1}
    got, want = _half_f32(out["y_ptr"], dt), _half_f32(ref["y_ptr"], dt)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok], want[ok])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 1024, 2048, 4096])
def test_rmsnorm_bit_exact(cols, dt):
    """RMSNorm with magnitudes over eight decades: every step is a correctly
    rounded f32 operation and the sum of squares follows the reference's
    halving order, so the results match bit for bit."""
    ref, out, g = _run(_cases.rmsnorm(rows=48, cols=cols, cores=4, dt=dt, wide=True))
    assert g.last_plan.counts() == {"prog": 1}
    np.testing.assert_array_equal(out["y_ptr"], ref["y_ptr"])


@pytest.fixture
def row_grid_limit():
    """Bound the row kernels' workgroups for one test (reset afterwards)."""
    from ktir_cpu_amd import runtime as rt
    yield rt.set_row_grid_limit
    rt.set_row_grid_limit(0)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 4096])
def test_softmax_fixed_form_many_rows_per_workgroup(cols, dt, row_grid_limit):
    """48 rows on 5 workgroups: every workgroup runs 9 or 10 rows through the
    kernel's two alternating row buffers (odd and even row counts)."""
    row_grid_limit(5)
    ref, out, g = _run(_cases.softmax(rows=48, cols=cols, cores=4, dt=dt))
    assert g.last_plan.counts() == {"prog": 1}
    np.testing.assert_allclose(_half_f32(out["y_ptr"], dt), _half_f32(ref["y_ptr"], dt), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cols", [512, 4096])
def test_rmsnorm_bit_exact_many_rows_per_workgroup(cols, dt, row_grid_limit):
    row_grid_limit(5)
    ref, out, g = _run(_cases.rmsnorm(rows=48, cols=cols, cores=4, dt=dt, wide=True))
    assert g.last_plan.counts() == {"prog": 1}
    np.testing.assert_array_equal(out["y_ptr"], ref["y_ptr"])


@pytest.mark.parametrize("limit", [0, 3])
@pytest.mark.parametrize("cols", [64, 256, 1024, 4096, 8192, 96, 3000])
@pytest.mark.parametrize("combiner", ["arith.addf", "arith.maximumf"])
def test_row_reduce_bit_exact(cols, combiner, limit, row_grid_limit):
    """Row folds reproduce the reference's pairwise-halving order bit for bit
    (power-of-two rows take the register-resident row kernel, the others the
    general row program); with limit 3, 32 rows run on 3 workgroups."""
    row_grid_limit(limit)
    ref, out, _ = _run(_cases.row_reduce(rows=32, cols=cols, combiner=combiner))
    np.testing.assert_array_equal(out["y_ptr"], ref["y_ptr"])


@pytest.mark.parametrize("cols,dt", [(40000, "f32"), (70001, "f32"), (65536, "f16")])
@pytest.mark.parametrize("combiner", ["arith.addf", "arith.maximumf"])
def test_row_reduce_longer_than_lds_bit_exact(cols, dt, combiner):
    """Rows longer than a row program folds in LDS (16384): the first
    halving levels run as elementwise programs on the two halves (an odd
    last element carried, 70001 columns), the rest as the row program; the
    result is the reference's pairwise-halving fold bit for bit."""
    ref, out, _ = _run(_cases.row_reduce(rows=4, cols=cols, rblk=2, combiner=combiner, dt=dt,
                                         decades=6 if dt == "f32" else 2))
    np.testing.assert_array_equal(out["y_ptr"], ref["y_ptr"])


@pytest.mark.parametrize("cols", [256, 4096])
def test_row_reduce_f16_bit_exact(cols):
    ref, out, _ = _run(_cases.row_reduce(rows=16, cols=cols, dt="f16"))
    np.testing.assert_array_equal(out["y_ptr"], ref["y_ptr"])


@pytest.mark.parametrize("cols", [256, 1024, 4096])
@pytest.mark.parametrize("combiner", ["arith.addf", "arith.mulf", "arith.maxnumf", "arith.minnumf", "arith.maximumf"])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_row_reduce_narrow_and_nan_ignoring_folds_bit_exact(dt, combiner, cols):
    """f16 / bf16 folds (every level rounded to the tile's type) and the
    NaN-ignoring max / min, with a NaN in every other row: the row-wave
    kernel's instantiations for such folds (1024 and 4096 columns) and the
    row-chain kernel (256), bit for bit against the oracle."""
    ref, out, _ = _run(_cases.row_reduce(rows=16, cols=cols, dt=dt, combiner=combiner, nans=True,
                                         decades=1 if combiner == "arith.mulf" else 3))
    got, want = out["y_ptr"].view(np.uint16).astype(np.int64), ref["y_ptr"].view(np.uint16).astype(np.int64)
    exp_bits, man_bits = (0x7C00, 0x03FF) if dt == "f16" else (0x7F80, 0x007F)

    def is_nan(b):
        return ((b & exp_bits) == exp_bits) & ((b & man_bits) != 0)

    both = is_nan(got) & is_nan(want)          # any NaN matches any NaN
    if combiner != "arith.addf" and combiner != "arith.mulf":
        # a max / min of -0 and +0: IEEE 754 leaves the sign open; NumPy on x86
        # keeps the first operand for f16 and the second for f32 (its SIMD
        # loop), the kernels give +0 for a max and -0 for a min
        sign = 0x8000
        both |= ((got & ~sign) == 0) & ((want & ~sign) == 0)
    np.testing.assert_array_equal(np.where(both, 0, got), np.where(both, 0, want))
    if combiner in ("arith.maxnumf", "arith.minnumf"):
        assert not is_nan(got).any()


@pytest.mark.parametrize("shape", [(256, 256, 256, 64, 64, 32, 2, 2),      # generic tile path
                                   (256, 256, 512, 128, 128, 64, 2, 2),    # MFMA path, one tile per core
                                   (512, 256, 256, 128, 128, 64, 2, 1),    # MFMA path, 2x2 tiles per core
                                   (256, 256, 192, 128, 128, 64, 2, 2),    # odd number of K steps
                                   (384, 256, 256, 128, 128, 64, 3, 2)])   # 6 tiles: no 2 x 2 grouping
def test_gemm(shape):
    ref, out, g = _run(_cases.gemm(*shape))
    # truncf + store of the K loop's result run in the matmul kernel's epilogue
    assert set(g.last_plan.counts()) == {"mm"}
    np.testing.assert_allclose(out["c_ptr"].astype(np.float32), ref["c_ptr"].astype(np.float32), rtol=1e-2, atol=1e-3)


_MFMA_SHAPES = [(256, 256, 512, 128, 128, 64, 2, 2),    # 256 x 256 blocks
                (256, 256, 192, 128, 128, 64, 2, 2)]    # 128 x 128 tiles (odd K steps)


@pytest.mark.parametrize("shape", _MFMA_SHAPES)
def test_gemm_f32_result(shape):
    """The f32 K-loop sums stored as they are (no truncf) by the matmul
    kernel's epilogue."""
    ref, out, g = _run(_cases.gemm(*shape, out_dt="f32"))
    assert set(g.last_plan.counts()) == {"mm"}
    np.testing.assert_allclose(out["c_ptr"], ref["c_ptr"], rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("shape", _MFMA_SHAPES)
def test_gemm_bf16(shape):
    """bf16 operands (the bf16 MFMA) and a bf16 result written by the
    matmul kernel's epilogue."""
    ref, out, g = _run(_cases.gemm_bf16(*shape))
    assert set(g.last_plan.counts()) == {"mm"}
    np.testing.assert_allclose(bf16_from_bits(out["c_ptr"]), bf16_from_bits(ref["c_ptr"]), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("out_dt", ["f16", "bf16"])
@pytest.mark.parametrize("pad", [3, 8])
def test_gemm_256_block_into_wider_rows(out_dt, pad):
    """C is a 256 x 256 view into rows of 256 + pad elements: with pad 3 the
    rows are not 16-byte aligned, so the 256 x 256 MFMA kernel's epilogue
    takes its direct-store path instead of the LDS-staged one (pad 8 keeps
    the staged path); the padding columns stay untouched."""
    M = N = 256
    if out_dt == "f16":
        src, fn, kw = _cases.gemm(M, N, 512, 128, 128, 64, 2, 2)
    else:
        src, fn, kw = _cases.gemm_bf16(M, N, 512, 128, 128, 64, 2, 2)
    old = f"%c_view = ktdp.construct_memory_view %c_ptr, sizes: [{M}, {N}], strides: [{N}, 1]"
    assert old in src
    src = src.replace(old, f"%c_view = ktdp.construct_memory_view %c_ptr, sizes: [{M}, {N}], strides: [{N + pad}, 1]")
    c = np.full((M, N + pad), 7.0, np.float16)
    kw["c_ptr"] = c if out_dt == "f16" else np.full((M, N + pad), 0x40E0, np.uint16)   # bf16 7.0
    ref, out, g = _run((src, fn, kw))
    assert set(g.last_plan.counts()) == {"mm"}
    got, want = out["c_ptr"], ref["c_ptr"]
    np.testing.assert_array_equal(got[:, N:], want[:, N:])
    f = (lambda x: x.astype(np.float32)) if out_dt == "f16" else bf16_from_bits
    np.testing.assert_allclose(f(got[:, :N]), f(want[:, :N]), rtol=1e-2, atol=1e-3)


def _plant_non_finite(a, b, inf, ninf, nan):
    """Planted values whose products decide the result's non-finite entries
    in any summation order: row 3 of A holds +inf (C row 3 = +-inf by the
    sign of B row 5), row 17 is zero but for one NaN (C row 17 all NaN),
    B[9, 33] = -inf (column 33), and column 70 of B is zero but for +inf at
    k = 100, with A[50, 100] = 0 (C[50, 70] = 0 * inf = NaN)."""
    a[3, 5] = inf
    a[17, :] = 0
    a[17, 40] = nan
    b[9, 33] = ninf
    b[:, 70] = 0
    b[100, 70] = inf
    a[50, 100] = 0


def _check_non_finite(o, r):
    np.testing.assert_array_equal(np.isnan(o), np.isnan(r))
    np.testing.assert_array_equal(np.isposinf(o), np.isposinf(r))
    np.testing.assert_array_equal(np.isneginf(o), np.isneginf(r))
    fin = np.isfinite(r)
    assert np.isnan(r).any() and np.isinf(r).any() and fin.mean() > 0.9
    np.testing.assert_allclose(o[fin], r[fin], rtol=1e-2, atol=1e-3)


@pytest.mark.filterwarnings("ignore:invalid value encountered in matmul")
@pytest.mark.parametrize("shape,out_dt", [((256, 256, 256, 64, 64, 32, 2, 2), "f16"),   # generic tile path
                                          (_MFMA_SHAPES[0], "f16"), (_MFMA_SHAPES[0], "f32"),
                                          (_MFMA_SHAPES[1], "f32")])
def test_gemm_non_finite_inputs(shape, out_dt):
    """+-inf and NaN operands: the result is NaN, +inf or -inf exactly where
    the oracle's is (those follow from the products alone, whatever the
    order of the sums), and within tolerance elsewhere."""
    src, fn, kw = _cases.gemm(*shape, out_dt=out_dt)
    _plant_non_finite(kw["a_ptr"], kw["b_ptr"], np.inf, -np.inf, np.nan)
    ref, out, g = _run((src, fn, kw))
    assert set(g.last_plan.counts()) == {"mm"}
    _check_non_finite(out["c_ptr"].astype(np.float32), ref["c_ptr"].astype(np.float32))


@pytest.mark.filterwarnings("ignore:invalid value encountered in matmul")
@pytest.mark.parametrize("shape", _MFMA_SHAPES)
def test_gemm_bf16_non_finite_inputs(shape):
    src, fn, kw = _cases.gemm_bf16(*shape)
    _plant_non_finite(kw["a_ptr"], kw["b_ptr"], 0x7F80, 0xFF80, 0x7FC0)
    ref, out, g = _run((src, fn, kw))
    assert set(g.last_plan.counts()) == {"mm"}
    _check_non_finite(bf16_from_bits(out["c_ptr"]), bf16_from_bits(ref["c_ptr"]))


def test_flash_attention_generic_path():
    """D = 32, 64-row blocks: not the fused kernel's shape, op-by-op launches."""
    ref, out, g = _run(_cases.flash_attention())
    assert "attn" not in g.last_plan.counts()
    np.testing.assert_allclose(bf16_from_bits(out["o_ptr"]), bf16_from_bits(ref["o_ptr"]), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("args", [dict(S=512, D=128, blk=128),
                                  dict(S=512, D=128, blk=128, dt="f16"),
                                  dict(B=2, H=2, S=384, D=128, blk=128, causal=False),
                                  dict(B=1, H=3, S=1024, D=128, blk=128, seed=3)])
def test_flash_attention_fused(args):
    """The whole KV loop in one fused MFMA launch (causal and full, bf16 and f16)."""
    ref, out, g = _run(_cases.flash_attention(**args))
    assert g.last_plan.counts().get("attn") == 1
    f = bf16_from_bits if args.get("dt", "bf16") == "bf16" else (lambda x: x.astype(np.float32))
    np.testing.assert_allclose(f(out["o_ptr"]), f(ref["o_ptr"]), rtol=1e-2, atol=1e-3)
    for k in ("q_ptr", "k_ptr", "v_ptr"):
        np.testing.assert_array_equal(out[k], ref[k])


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_flash_attention_fused_without_pairs(dt, monkeypatch):
    """A launch that names no lane pairs (as a C-ABI caller may) runs one
    query block per workgroup, with the same f16 P @ V rule."""
    from ktir_cpu_amd import fusion
    monkeypatch.setattr(fusion, "_pp_pairs", lambda *a, **k: np.zeros(0, np.int32))
    ref, out, g = _run(_cases.flash_attention(S=512, D=128, blk=128, dt=dt))
    assert g.last_plan.counts().get("attn") == 1
    f = bf16_from_bits if dt == "bf16" else (lambda x: x.astype(np.float32))
    np.testing.assert_allclose(f(out["o_ptr"]), f(ref["o_ptr"]), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("big", [3.0e5, -7.0e4])
def test_flash_attention_fused_v_beyond_f16(big):
    """A V value f16 cannot hold sends P @ V of the launch to the bf16 hi + lo
    kernel (the f16 copy of V is not used); results still match."""
    from oracle.interp import bf16_bits
    src, fn, kw = _cases.flash_attention(S=512, D=128, blk=128)
    v = bf16_from_bits(kw["v_ptr"])
    v[0, 1, 300, 5] = big
    kw["v_ptr"] = bf16_bits(v)
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts().get("attn") == 1
    np.testing.assert_allclose(bf16_from_bits(out["o_ptr"]), bf16_from_bits(ref["o_ptr"]), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("fill,sign,dt", [("-1.0e4", 1, "bf16"), ("-1.0e4", 1, "f16"), ("0xFF800000", -1, "bf16"),
                                          ("-3.0", -1, "f16")])
def test_flash_attention_fused_other_fill_or_scale(fill, sign, dt):
    """A finite mask fill value or a negative scale (the two-group kernel
    takes only -inf and scale > 0) still runs as one fused launch, on the
    one-lane-per-workgroup kernel, and matches the oracle."""
    src, fn, kw = _cases.flash_attention(S=512, D=128, blk=128, dt=dt)
    src = src.replace("%neg_inf = arith.constant 0xFF800000 : f32",
                      f"%neg_inf = arith.constant 0xFF800000 : f32\n    %fill = arith.constant {fill} : f32")
    src = src.replace("%r = arith.select %keep, %sv, %neg_inf : f32", "%r = arith.select %keep, %sv, %fill : f32")
    kw["scale"] = sign * kw["scale"]
    print(f"[attn] fill {fill} scale sign {sign} {dt}", flush=True)
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts().get("attn") == 1
    f = bf16_from_bits if dt == "bf16" else (lambda x: x.astype(np.float32))
    np.testing.assert_allclose(f(out["o_ptr"]), f(ref["o_ptr"]), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_flash_attention_fused_non_finite_inputs(dt):
    """A NaN in one query row and an infinity in one key: NaN exactly where
    the oracle has NaN (the NaN row; the rows whose maximum the infinite key
    sets), the other rows within tolerance."""
    from oracle.interp import bf16_bits
    src, fn, kw = _cases.flash_attention(S=512, D=128, blk=128, dt=dt)
    f = bf16_from_bits if dt == "bf16" else (lambda x: x.astype(np.float32))
    back = (lambda x: bf16_bits(x.astype(np.float32))) if dt == "bf16" else (lambda x: x.astype(np.float16))
    q, k = f(kw["q_ptr"]).copy(), f(kw["k_ptr"]).copy()
    q[0, 1, 200, 7] = np.nan
    k[0, 0, 300, 3] = np.inf
    kw["q_ptr"], kw["k_ptr"] = back(q), back(k)
    print(f"[attn] non-finite inputs {dt}", flush=True)
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts().get("attn") == 1
    got, want = f(out["o_ptr"]), f(ref["o_ptr"])
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    assert np.isnan(want).any()
    ok = ~np.isnan(want)
    np.testing.assert_allclose(got[ok], want[ok], rtol=1e-2, atol=1e-3)


def test_flash_attention_replay_reuses_v_copy():
    """Replays of a prepared bf16 attention reuse the f16 copy of V while no
    host write has reached the arena; a new V written through memory.hbm
    makes the next replay convert again, and its result is the oracle's for
    the new V; reset_inputs restores the first result."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    from oracle.interp import bf16_bits
    src, fn, kw = _cases.flash_attention(S=512, D=128, blk=128)
    print("[attn] replay with the f16 copy of V", flush=True)
    g = KTIRInterpreter()
    g.load(src)
    prep = g.prepare(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})
    out0 = prep.outputs()["o_ptr"]
    attn = [d for k, d, _ in prep.plan.launches if k == "attn"]
    assert len(attn) == 1 and len(prep.plan.v16) == 1
    assert next(iter(prep.plan.v16.values())).ok
    prep.run()
    assert attn[0].v16_ready == 1
    np.testing.assert_array_equal(prep.outputs()["o_ptr"], out0)
    # a different V through the interpreter's HBM (a host write into the arena)
    v2 = bf16_bits(bf16_from_bits(kw["v_ptr"])[..., ::-1] * 0.5)
    a = next(x for x in prep.arena.allocs if x.name == "v_ptr")
    g.memory.hbm.write(a.addr // 128, v2.reshape(-1))
    prep.run()
    assert attn[0].v16_ready == 0
    o = OracleInterpreter()
    o.load(src)
    kw2 = dict(kw, v_ptr=v2, o_ptr=np.zeros_like(kw["o_ptr"]))
    ref2 = o.execute_function(fn, **kw2)["o_ptr"]
    out2 = prep.outputs()["o_ptr"]
    np.testing.assert_allclose(bf16_from_bits(out2), bf16_from_bits(ref2), rtol=1e-2, atol=1e-3)
    assert not np.array_equal(out2, out0)
    prep.run()
    assert attn[0].v16_ready == 1
    np.testing.assert_array_equal(prep.outputs()["o_ptr"], out2)
    prep.reset_inputs()
    prep.run()
    assert attn[0].v16_ready == 0
    np.testing.assert_array_equal(prep.outputs()["o_ptr"], out0)


def test_flash_attention_unfused_epilogue():
    """An epilogue other than acc / l stays a separate program after the fused loop."""
    src, fn, kw = _cases.flash_attention(S=256, D=128, blk=128)
    src = src.replace("%q_ = arith.divf %av, %lv : f32", "%q_ = arith.mulf %av, %lv : f32")
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts() == {"attn": 1, "prog": 1}
    np.testing.assert_allclose(bf16_from_bits(out["o_ptr"]), bf16_from_bits(ref["o_ptr"]), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("cols", [256, 1024])
@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_row_product_fold_keeps_the_sign_of_zero(dt, cols):
    """Row products that are zeros of either sign: -0 times ones, +0 times
    one -1, one -0 with one -1, and a row of -0s with one +0, bit for bit
    (the sign is the parity of the negative factors, whatever the order)."""
    src, fn, kw = _cases.row_reduce(rows=8, cols=cols, rblk=4, dt=dt, combiner="arith.mulf")
    x = np.ones((8, cols), np.float32)
    x[1, 0] = -0.0
    x[2, 0], x[2, 1] = 0.0, -1.0
    x[3, 5], x[3, 6] = -0.0, -1.0
    x[4], x[4, 3] = -0.0, 0.0
    if dt == "bf16":
        from oracle.interp import bf16_bits
        kw["x_ptr"] = bf16_bits(x)
    else:
        kw["x_ptr"] = x.astype(kw["x_ptr"].dtype)
    ref, out, _ = _run((src, fn, kw))
    u = np.uint32 if dt == "f32" else np.uint16
    np.testing.assert_array_equal(out["y_ptr"].view(u), ref["y_ptr"].view(u))
    bits = ref["y_ptr"].view(u).astype(np.int64)
    assert list((bits[[1, 2, 3, 4]] >> (31 if dt == "f32" else 15)) & 1) == [1, 1, 0, 1]


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_flash_attention_epilogue_reciprocal_within_one_ulp(dt):
    """O = acc / l as acc times the correctly rounded 1 / l, against the
    oracle's division, on scores that make every probability exactly 1 or 0:
    query i is one-hot on dimension i % 7, key j is 200 on dimension j % 7,
    so query i's kept keys (j <= i, j = i mod 7) score 200 and the others 0
    (exp(-200) is 0 in f32).  Then l is the count k_i = i // 7 + 1 and acc
    the exact sum of their integer V rows, so the only difference left is
    the epilogue's rounding: at most one output ulp, none where k_i is a
    power of two (1 / k_i exact)."""
    from oracle.interp import bf16_bits
    B, H, S, D = 1, 2, 512, 128
    src, fn, kw = _cases.flash_attention(B=B, H=H, S=S, D=D, blk=128, dt=dt)
    rng = np.random.default_rng(11)
    q = np.zeros((B, H, S, D), np.float32)
    k = np.zeros((B, H, S, D), np.float32)
    idx = np.arange(S)
    q[:, :, idx, idx % 7] = 1.0
    k[:, :, idx, idx % 7] = 200.0
    v = rng.integers(-8, 9, (B, H, S, D)).astype(np.float32)
    enc = bf16_bits if dt == "bf16" else (lambda a: a.astype(np.float16))
    kw.update(q_ptr=enc(q), k_ptr=enc(k), v_ptr=enc(v), o_ptr=np.zeros_like(enc(q)), scale=1.0)
    ref, out, g = _run((src, fn, kw))
    assert g.last_plan.counts().get("attn") == 1
    u = np.int32
    got = out["o_ptr"].view(np.int16).astype(u)
    want = ref["o_ptr"].view(np.int16).astype(u)
    d = np.abs(got - want)
    assert d.max() <= 1, d.max()
    kcount = idx // 7 + 1
    pow2 = (kcount & (kcount - 1)) == 0
    assert (d[..., pow2, :] == 0).all()
    # the exact quotients, rounded once: the oracle holds them
    exact = np.zeros((B, H, S, D))
    for i in range(S):
        keep = (idx <= i) & (idx % 7 == i % 7)
        exact[:, :, i] = v[:, :, keep].sum(axis=2) / keep.sum()
    want_exact = enc(exact.astype(np.float32)).view(np.int16).astype(u)
    np.testing.assert_array_equal(want, want_exact)
