"""GPU parity for the paged attention, single-tile f16 attention and rotary
embedding forms of the reference's examples, on the kernels whose oracle
results tests/test_oracle_example_pins.py pins against closed forms (and
against the example files themselves).

Bars: RoPE is f16 multiply / add / subtract only, so bit-exact; the two
attention forms meet the north star's rtol 1e-2 / atol 1e-3 (matmul and
softmax), the f16 one with every intermediate rounded to f16 as the oracle
does."""
import numpy as np
import pytest

from ktir_cpu_amd import configs
from oracle.interp import OracleInterpreter
from tests.test_oracle_example_pins import (PA_ARGS, PA_CASES, PA_FN, paged_inputs, rope_inputs, sdpa_inputs)

pytestmark = pytest.mark.gpu


def _both(src, fn, kw, out):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    o = OracleInterpreter()
    o.load(src)
    ref = o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})[out]
    g = KTIRInterpreter()
    g.load(src)
    got = g.execute_function(fn, **kw)[out]
    print("  ", g.last_plan.mode, g.last_plan.counts(), g.last_plan.fallback_reason, flush=True)
    return got, ref, g.last_plan


@pytest.mark.parametrize("gen,inp,args", [c[1:] for c in PA_CASES], ids=[c[0] for c in PA_CASES])
def test_paged_attention_within_tolerance(gen, inp, args):
    kw = dict(paged_inputs(**inp), **args)
    got, ref, plan = _both(configs.paged_attention(**gen), PA_FN, kw, "output_ptr")
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)
    # the output tiles of an odd batch start sit off the 2-row grid but are
    # disjoint: the lanes still run together, the KV loop as one launch
    assert plan.mode == "lockstep"
    # the KV loop is one launch whose epilogue also divides by l and stores
    # the output; the other launch copies the Q tile
    assert plan.counts() == {"prog": 1, "pattn": 1}


def test_paged_attention_many_tokens_within_tolerance():
    """64 tokens of one sequence over a 512-block cache: 32 x 8 cores, each
    through 40 pages of the table (640 keys)."""
    gen = dict(tokens=64, q_heads=32, kv_heads=8, head=128, page=16, blocks=512, max_pages=64, block_q=2)
    kw = dict(paged_inputs(tokens=64, blocks=512, max_pages=64, seed=7),
              **dict(PA_ARGS, num_tiles=40, context_len=576, block_table_offset=3))
    got, ref, plan = _both(configs.paged_attention(**gen), PA_FN, kw, "output_ptr")
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)
    assert plan.counts().get("pattn") == 1


PA_SHAPES = [
    # matrix-core form: head sizes 32 and 256, 16 rows per core (4 tokens x 4 heads)
    ("d32", dict(head=32), dict(head=32), {}),
    ("d256", dict(tokens=8, q_heads=8, kv_heads=2, head=256, blocks=32, max_pages=8),
     dict(tokens=8, q_heads=8, kv_heads=2, head=256, blocks=32, max_pages=8), {}),
    ("rows16", dict(block_q=4), {}, {}),
    # f32-FMA form: pages of 32 keys, 32 rows per core (8 tokens x 4 heads)
    ("page32", dict(page=32, blocks=32, max_pages=8), dict(page=32, blocks=32, max_pages=8),
     dict(num_tiles=4, context_len=100)),
    ("rows32", dict(tokens=16, block_q=8), dict(tokens=16), {}),
]


@pytest.mark.parametrize("gen,inp,args", [c[1:] for c in PA_SHAPES], ids=[c[0] for c in PA_SHAPES])
def test_paged_attention_shapes_within_tolerance(gen, inp, args):
    """Shapes on either side of the matrix-core form's limits (pages of 16
    keys, at most 16 query rows per core, D in {32, 64, 128, 256}): both the
    MFMA kernel and the f32 FMA kernel against the oracle."""
    kw = dict(paged_inputs(seed=11, **inp), **dict(PA_ARGS, **args))
    got, ref, plan = _both(configs.paged_attention(**gen), PA_FN, kw, "output_ptr")
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)
    assert plan.counts().get("pattn") == 1


@pytest.mark.parametrize("n,d,rows", [(32, 64, 32), (256, 128, 64)])
def test_sdpa_f16_within_tolerance(n, d, rows):
    kw = sdpa_inputs(n, d, seed=n)
    got, ref, _ = _both(configs.sdpa_f16(n, d, rows), "sdpa_kernel_2d", kw, "output_ptr")
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("zero", [False, True], ids=["normal", "zero_input"])
def test_rope_example_size_bit_exact(zero):
    """The example's size: 40 heads x 4096 positions x 128, grid [4, 2]."""
    kw = rope_inputs(zero=zero)
    got, ref, plan = _both(configs.rope(), "rope_fwd_kernel", kw, "out_ptr")
    np.testing.assert_array_equal(got.view(np.uint16), ref.view(np.uint16))
    assert plan.mode == "lockstep"


def test_rope_odd_grid_bit_exact():
    H, S, D = 6, 768, 64
    kw = rope_inputs(H, S, D, seed=9)
    got, ref, _ = _both(configs.rope(H, S, D, grid_s=3, grid_h=3, tile=128), "rope_fwd_kernel", kw, "out_ptr")
    np.testing.assert_array_equal(got.view(np.uint16), ref.view(np.uint16))


from tests import _cases as C  # noqa: E402
from tests.test_oracle_example_pins import _bits  # noqa: E402


@pytest.mark.parametrize("index,dim1_start", [((3, 7), 5), ((15, 0, 9), 32)])
def test_indexed_add_bit_exact(index, dim1_start):
    src, fn, kw = C.indexed_add(index=index, dim1_start=dim1_start)
    got, ref, _ = _both(src, fn, kw, "output_ptr")
    np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("write,pages", [(False, None), (True, None), (True, [3, 7, 3, 1, 0, 7, 2, 5])],
                         ids=["copy", "write", "write_repeated_pages"])
def test_paged_tensor_bit_exact(write, pages):
    src, fn, kw = C.paged_tensor(write=write, pages=pages)
    got, ref, _ = _both(src, fn, kw, "y_ptr")
    np.testing.assert_array_equal(_bits(got), _bits(ref))


def test_expert_gather_bit_exact():
    src, fn, kw = C.expert_gather()
    got, ref, _ = _both(src, fn, kw, "out_ptr")
    np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("outer,inner", [(2, 2), (5, 3)])
def test_nested_yield(outer, inner):
    src, fn, kw = C.nested_yield(outer, inner)
    got, ref, _ = _both(src, fn, kw, "out")
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, np.full(4, float(outer), np.float32))


@pytest.mark.parametrize("rows,cols,cores", [(2, 4096, 1), (8, 16384, 4), (3, 262144, 2)])
def test_softmax_wide_within_tolerance(rows, cols, cores):
    """The f16 row softmax of examples/ktir/softmax_wide.mlir, up to its own
    262144-element rows."""
    src, fn, kw = C.softmax_wide(rows, cols, cores)
    got, ref, _ = _both(src, fn, kw, "output_ptr")
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_scalar_broadcast_bit_exact(dt):
    src, fn, kw = C.scalar_broadcast(dt=dt)
    got, ref, _ = _both(src, fn, kw, "out_ptr")
    np.testing.assert_array_equal(got, ref)
    assert np.all(got == kw["in_ptr"][0, 0])


def _bf16_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_paged_attention_bf16_within_tolerance():
    from oracle.interp import bf16_bits
    kw = {k: (bf16_bits(v.astype(np.float32)) if k != "block_tables_ptr" else v) for k, v in paged_inputs().items()}
    got, ref, plan = _both(configs.paged_attention(dt="bf16"), PA_FN, dict(kw, **PA_ARGS), "output_ptr")
    np.testing.assert_allclose(_bf16_f32(got), _bf16_f32(ref), rtol=1e-2, atol=1e-3)
    assert plan.counts().get("pattn") == 1


def test_paged_attention_without_mask_within_tolerance():
    kw = dict(paged_inputs(seed=3), **PA_ARGS)
    got, ref, plan = _both(configs.paged_attention(causal=False), PA_FN, kw, "output_ptr")
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)
    assert plan.counts().get("pattn") == 1


def test_paged_attention_no_tiles_gives_zero():
    """num_tiles = 0: the loop does not run; acc / L = 0 / 1."""
    kw = dict(paged_inputs(), **dict(PA_ARGS, num_tiles=0))
    got, ref, _ = _both(configs.paged_attention(), PA_FN, kw, "output_ptr")
    np.testing.assert_array_equal(got, ref)
    assert not np.any(got)


def test_paged_attention_page_past_the_cache_reads_zero():
    """A table entry beyond the cache's blocks: its K and V rows read as
    zeros (the reference's zero-pad on over-read), on both paths."""
    kw = paged_inputs()
    kw["block_tables_ptr"][0, 3] = 64 + 5
    got, ref, _ = _both(configs.paged_attention(), PA_FN, dict(kw, **PA_ARGS), "output_ptr")
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), rtol=1e-2, atol=1e-3)


def test_paged_attention_negative_page_raises():
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    kw = paged_inputs()
    kw["block_tables_ptr"][0, 2] = -1
    args = dict(kw, **PA_ARGS)
    o = OracleInterpreter()
    o.load(configs.paged_attention())
    with pytest.raises(IndexError):
        o.execute_function(PA_FN, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in args.items()})
    g = KTIRInterpreter()
    g.load(configs.paged_attention())
    with pytest.raises(IndexError):
        g.execute_function(PA_FN, **args)
