"""Oracle pins for three kernel forms of the reference's examples, written by
this package's own generators (ktir_cpu_amd.configs): paged attention
(examples/triton-ktir/paged_attention.mlir), single-tile f16 attention
(examples/triton-ktir/sdpa_2d.mlir) and rotary embedding
(examples/latency/rope_fwd_4x2.mlir).

Each is checked against its closed form the way the reference's own tests
check the example files (tests/test_examples.py:506-628 and 1080-1190):
softmax(Q K^T * scale) V with the causal mask of the paged form, f16 RoPE
rotation.  Where the reference checkout is present, the generator's text at
the example's parameters also gives the same bits as the example file on the
oracle, which shows the generated kernel is the example's computation."""
import os

import numpy as np
import pytest

from ktir_cpu_amd import configs
from oracle.interp import OracleInterpreter

EXAMPLES = "/root/reference/examples"
PA_FN = "kernel_unified_attention_spyre_2d"
PA_ARGS = dict(cur_batch_start_index=0, block_table_offset=0, num_tiles=8, context_len=120,
               scale=0.08838834764831843)


def oracle(src, fn, kw):
    o = OracleInterpreter()
    o.load(src)
    return o.execute_function(fn, **{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()})


# ---------------------------------------------------------------------------
# inputs and closed forms
# ---------------------------------------------------------------------------

def paged_inputs(tokens=8, q_heads=32, kv_heads=8, head=128, page=16, blocks=64, max_pages=16, seed=42):
    """The reference test's inputs (tests/test_examples.py:521-525) at its
    shapes: standard normal f16 query and caches, page table uniform over the
    cache's blocks (so pages may repeat)."""
    rng = np.random.default_rng(seed)
    return dict(output_ptr=np.zeros((tokens, q_heads, head), np.float16),
                query_ptr=rng.standard_normal((tokens, q_heads, head)).astype(np.float16),
                key_cache_ptr=rng.standard_normal((blocks, page, kv_heads, head)).astype(np.float16),
                value_cache_ptr=rng.standard_normal((blocks, page, kv_heads, head)).astype(np.float16),
                block_tables_ptr=rng.integers(0, blocks, size=(1, max_pages), dtype=np.int32))


def paged_closed_form(kw, args, tokens=8, block_q=2):
    """Attention of the `tokens` query tokens the grid covers (from the batch
    start on) against the keys of
    pages block_tables[0, offset : offset + num_tiles], in float64: token t
    (relative to the batch start) sees key positions 0 .. context_len + t.
    Rows the grid does not cover keep the output's initial contents."""
    q = kw["query_ptr"].astype(np.float64)
    q_heads = q.shape[1]
    kc, vc = kw["key_cache_ptr"].astype(np.float64), kw["value_cache_ptr"].astype(np.float64)
    kv_heads, page = kc.shape[2], kc.shape[1]
    g = q_heads // kv_heads
    start, off, nt = args["cur_batch_start_index"], args["block_table_offset"], args["num_tiles"]
    pages = kw["block_tables_ptr"][0, off:off + nt]
    out = kw["output_ptr"].astype(np.float64).copy()
    pos = np.arange(nt * page)
    for h in range(q_heads):
        K = np.concatenate([kc[p, :, h // g] for p in pages])
        V = np.concatenate([vc[p, :, h // g] for p in pages])
        for t in range(tokens // block_q * block_q):
            s = (K @ q[start + t, h]) * args["scale"]
            s[pos > args["context_len"] + t] = -np.inf
            w = np.exp(s - s.max())
            out[start + t, h] = w @ V / w.sum()
    return out


def sdpa_inputs(n=32, d=64, seed=42):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((n, d)).astype(np.float16) for _ in range(3))
    return dict(q_ptr=q, k_ptr=k, v_ptr=v, output_ptr=np.zeros((n, d), np.float16))


def sdpa_closed_form(kw):
    """The reference test's closed form (tests/test_examples.py:615-621):
    f32 softmax of Q K^T / 8, probabilities rounded to f16, times V."""
    q, k, v = (kw[n].astype(np.float32) for n in ("q_ptr", "k_ptr", "v_ptr"))
    s = (q @ k.T) * np.float32(0.125)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p = (p / p.sum(axis=1, keepdims=True)).astype(np.float16)
    return (p.astype(np.float32) @ v).astype(np.float16)


def rope_inputs(heads=40, seq=4096, head=128, seed=42, zero=False):
    """Standard normal f16 x and the standard RoPE tables (base 10000), as
    the reference test builds them (tests/test_examples.py:1096-1104)."""
    rng = np.random.default_rng(seed)
    x = np.zeros((heads * seq, head), np.float16) if zero else \
        rng.standard_normal((heads * seq, head)).astype(np.float16)
    freq = 10000.0 ** (-np.arange(head // 2, dtype=np.float64) * 2.0 / head)
    ang = np.outer(np.arange(seq, dtype=np.float64), freq)
    return dict(x_ptr=x, cos_ptr=np.cos(ang).astype(np.float16), sin_ptr=np.sin(ang).astype(np.float16),
                out_ptr=np.zeros_like(x))


def rope_closed_form(kw, heads, seq):
    """Half-layout rotation in f16 arithmetic: each product and the sum or
    difference rounded to f16 (f16 tile ops are exact-then-rounded)."""
    x, c, s = kw["x_ptr"], kw["cos_ptr"], kw["sin_ptr"]
    h = x.shape[1] // 2
    x1, x2 = x[:, :h].reshape(heads, seq, h), x[:, h:].reshape(heads, seq, h)
    y = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)
    return y.reshape(heads * seq, 2 * h)


def _bits(a):
    return a.view({2: np.uint16, 4: np.uint32}[a.dtype.itemsize])


# ---------------------------------------------------------------------------
# paged attention
# ---------------------------------------------------------------------------

PA_CASES = [
    # (id, generator kwargs, input kwargs, args)
    ("example", {}, {}, PA_ARGS),
    # a short context: the diagonal key is one of at most 16 a token sees,
    # so a mask off by one position moves the output far beyond tolerance
    ("short_context", {}, {}, dict(PA_ARGS, num_tiles=2, context_len=4)),
    # a later batch start in a longer query array, a later page-table column
    ("offsets", dict(tokens=8, max_pages=24, total_tokens=20), dict(tokens=20, max_pages=24),
     dict(PA_ARGS, cur_batch_start_index=9, block_table_offset=5, num_tiles=7, context_len=97)),
    # 4 query tokens per core, 2 query heads per KV head, head size 64
    ("bq4_g2_d64", dict(tokens=16, q_heads=8, kv_heads=4, head=64, page=16, blocks=32, max_pages=8, block_q=4),
     dict(tokens=16, q_heads=8, kv_heads=4, head=64, page=16, blocks=32, max_pages=8),
     dict(PA_ARGS, num_tiles=8, context_len=100, scale=0.125)),
]


@pytest.mark.parametrize("gen,inp,args", [c[1:] for c in PA_CASES], ids=[c[0] for c in PA_CASES])
def test_paged_attention_matches_closed_form(gen, inp, args):
    kw = paged_inputs(**inp)
    got = oracle(configs.paged_attention(**gen), PA_FN, dict(kw, **args))["output_ptr"]
    want = paged_closed_form(kw, args, gen.get("tokens", 8), gen.get("block_q", 2))
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got.astype(np.float64), want, rtol=1e-2, atol=2e-3)


def test_paged_attention_closed_form_catches_a_shifted_mask():
    """The short-context case fails if the mask admits one more key: the
    closed form itself is sensitive to the diagonal."""
    args = dict(PA_ARGS, num_tiles=2, context_len=4)
    kw = paged_inputs()
    got = oracle(configs.paged_attention(), PA_FN, dict(kw, **args))["output_ptr"].astype(np.float64)
    shifted = paged_closed_form(kw, dict(args, context_len=5))
    assert np.abs(got - shifted).max() > 0.05


@pytest.mark.skipif(not os.path.isdir(EXAMPLES), reason="reference example kernels not present")
def test_paged_attention_generator_is_the_example():
    kw = dict(paged_inputs(), **PA_ARGS)
    mine = oracle(configs.paged_attention(), PA_FN, kw)["output_ptr"]
    ex = oracle(os.path.join(EXAMPLES, "triton-ktir/paged_attention.mlir"), PA_FN, kw)["output_ptr"]
    np.testing.assert_array_equal(_bits(mine), _bits(ex))


# ---------------------------------------------------------------------------
# single-tile f16 attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,d,rows", [(32, 64, 32), (128, 64, 32)])
def test_sdpa_f16_matches_closed_form(n, d, rows):
    kw = sdpa_inputs(n, d)
    got = oracle(configs.sdpa_f16(n, d, rows), "sdpa_kernel_2d", kw)["output_ptr"]
    np.testing.assert_allclose(got.astype(np.float32), sdpa_closed_form(kw).astype(np.float32), rtol=1e-2, atol=1e-2)


def test_sdpa_f16_uniform_when_keys_are_zero():
    """K = 0: every score is 0, each probability 1/n exactly in f16 for n a
    power of two, and the output row is the mean of V's rows."""
    kw = sdpa_inputs(32, 64)
    kw["k_ptr"][:] = 0
    got = oracle(configs.sdpa_f16(), "sdpa_kernel_2d", kw)["output_ptr"]
    want = (kw["v_ptr"].astype(np.float64).mean(axis=0)).astype(np.float16)
    np.testing.assert_allclose(got.astype(np.float32), np.broadcast_to(want, got.shape).astype(np.float32),
                               rtol=0, atol=2e-3)


@pytest.mark.skipif(not os.path.isdir(EXAMPLES), reason="reference example kernels not present")
def test_sdpa_f16_generator_is_the_example():
    kw = sdpa_inputs()
    mine = oracle(configs.sdpa_f16(), "sdpa_kernel_2d", kw)["output_ptr"]
    ex = oracle(os.path.join(EXAMPLES, "triton-ktir/sdpa_2d.mlir"), "sdpa_kernel_2d", kw)["output_ptr"]
    np.testing.assert_array_equal(_bits(mine), _bits(ex))


# ---------------------------------------------------------------------------
# rotary embedding
# ---------------------------------------------------------------------------

def test_rope_f16_closed_form_bit_exact():
    H, S, D = 4, 512, 64
    kw = rope_inputs(H, S, D, seed=3)
    got = oracle(configs.rope(H, S, D, grid_s=2, grid_h=2, tile=128), "rope_fwd_kernel", kw)["out_ptr"]
    np.testing.assert_array_equal(_bits(got), _bits(rope_closed_form(kw, H, S)))


def test_rope_closed_form_catches_swapped_halves():
    """A rotation by -angle (sin's sign swapped) is a plausible slip; the
    closed form tells it apart from the kernel's result."""
    H, S, D = 2, 256, 64
    kw = rope_inputs(H, S, D, seed=4)
    got = oracle(configs.rope(H, S, D, grid_s=1, grid_h=1, tile=128), "rope_fwd_kernel", kw)["out_ptr"]
    flipped = rope_closed_form(dict(kw, sin_ptr=-kw["sin_ptr"]), H, S)
    assert not np.array_equal(_bits(got), _bits(flipped))


def test_rope_zero_input_gives_zero():
    H, S, D = 4, 512, 64
    kw = rope_inputs(H, S, D, zero=True)
    got = oracle(configs.rope(H, S, D, grid_s=2, grid_h=2, tile=128), "rope_fwd_kernel", kw)["out_ptr"]
    assert not np.any(got)


@pytest.mark.skipif(not os.path.isdir(EXAMPLES), reason="reference example kernels not present")
def test_rope_generator_is_the_example():
    kw = rope_inputs()
    mine = oracle(configs.rope(), "rope_fwd_kernel", kw)["out_ptr"]
    ex = oracle(os.path.join(EXAMPLES, "latency/rope_fwd_4x2.mlir"), "rope_fwd_kernel", kw)["out_ptr"]
    np.testing.assert_array_equal(_bits(mine), _bits(ex))


# ---------------------------------------------------------------------------
# indirect forms: indexed add (i64 index), paged tensor copy and write,
# expert gather; nested loops with iter_args
# ---------------------------------------------------------------------------

from tests import _cases as C  # noqa: E402


def paged_copy_closed_form(kw, P):
    x, idx = kw["x_ptr"], kw["idx_ptr"]
    out = np.zeros_like(kw["y_ptr"])
    for b in range(idx.shape[0]):
        for t in range(idx.shape[1] * P):
            out[b, t] = x[idx[b, t // P], :, t % P]
    return out


def paged_write_closed_form(kw, P):
    """Later (b, h, t, d) points win where two pages repeat: the reference's
    last writer in variables-space order (memory.py:290)."""
    x, idx = kw["x_ptr"], kw["idx_ptr"]
    out = kw["y_ptr"].copy()
    for b in range(idx.shape[0]):
        for h in range(x.shape[2]):
            for t in range(idx.shape[1] * P):
                out[idx[b, t // P], h, t % P] = x[b, t, h]
    return out


def test_indexed_add_closed_form():
    src, fn, kw = C.indexed_add()
    got = oracle(src, fn, kw)["output_ptr"]
    s = kw["dim1_start"]
    np.testing.assert_array_equal(_bits(got), _bits(kw["x_ptr"][kw["index_ptr"]][:, s:s + 32] + kw["y_ptr"]))


@pytest.mark.skipif(not os.path.isdir(EXAMPLES), reason="reference example kernels not present")
def test_indexed_add_generator_is_the_example():
    """At the example's shapes (x [128, 64, 8, 128], grid [2, 8], 32 rows
    from dim1_start) with the reference test's index (3, 7)."""
    src, fn, kw = C.indexed_add(rows=128, d1=64, heads=8, D=128, width=32, index=(3, 7), dim1_start=0)
    mine = oracle(src, fn, kw)["output_ptr"]
    ex = oracle(os.path.join(EXAMPLES, "triton-ktir/indexed_add.mlir"), fn, kw)["output_ptr"]
    np.testing.assert_array_equal(_bits(mine), _bits(ex))


@pytest.mark.parametrize("write", [False, True], ids=["copy", "write"])
def test_paged_tensor_closed_form(write):
    src, fn, kw = C.paged_tensor(write=write)
    got = oracle(src, fn, kw)["y_ptr"]
    want = (paged_write_closed_form if write else paged_copy_closed_form)(kw, 64)
    np.testing.assert_array_equal(_bits(got), _bits(want))


def test_paged_tensor_write_repeated_page_last_writer():
    """A page named twice in the table: the later table entry's rows win."""
    pages = [3, 7, 3, 1, 0, 7, 2, 5]
    src, fn, kw = C.paged_tensor(write=True, pages=pages)
    got = oracle(src, fn, kw)["y_ptr"]
    np.testing.assert_array_equal(_bits(got), _bits(paged_write_closed_form(kw, 64)))
    first_wins = kw["y_ptr"].copy()
    x, idx = kw["x_ptr"], kw["idx_ptr"]
    for b in reversed(range(idx.shape[0])):
        for h in range(x.shape[2]):
            for t in reversed(range(idx.shape[1] * 64)):
                first_wins[idx[b, t // 64], h, t % 64] = x[b, t, h]
    assert not np.array_equal(_bits(got), _bits(first_wins))


def test_expert_gather_closed_form():
    src, fn, kw = C.expert_gather()
    got = oracle(src, fn, kw)["out_ptr"]
    np.testing.assert_array_equal(_bits(got), _bits(kw["x_ptr"][kw["idx_ptr"]]))


def test_nested_yield_value():
    """The reference test's value (tests/test_examples.py:1197-1209): 2.0."""
    src, fn, kw = C.nested_yield()
    np.testing.assert_array_equal(oracle(src, fn, kw)["out"], np.full(4, 2.0, np.float32))
    src, fn, kw = C.nested_yield(outer=5, inner=3)
    np.testing.assert_array_equal(oracle(src, fn, kw)["out"], np.full(4, 5.0, np.float32))
