"""Seeded inputs for the five benchmark kernels at sizes the oracle finishes
in seconds (the same generators run at full size in bench.py)."""
import math

import numpy as np

from ktir_cpu_amd import configs
from oracle.interp import bf16_bits


def vector_add(n=4096, block=128, cores=32, seed=42):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float16)
    y = rng.standard_normal(n).astype(np.float16)
    return (configs.vector_add(n, block, cores), "add_kernel",
            dict(x_ptr=x, y_ptr=y, output_ptr=np.zeros(n, np.float16), BLOCK_SIZE=block))


def gather_scatter_add(rows=1024, dim=32, n_idx=512, cores=4, chunk=32, seed=42, dup_frac=0.1):
    rng = np.random.default_rng(seed)
    table = rng.standard_normal((rows, dim)).astype(np.float16)
    n_dup = int(n_idx * dup_frac)
    uniq = rng.choice(rows, n_idx - n_dup, replace=False)
    dup = rng.choice(uniq, n_dup)
    idx = rng.permutation(np.concatenate([uniq, dup])).astype(np.int32)
    return (configs.gather_scatter_add(rows, dim, n_idx, cores, chunk), "gather_scatter_add",
            dict(table_ptr=table, idx_ptr=idx, out_ptr=np.zeros((rows, dim), np.float32)))


def scatter_add_two_index(rows=1024, dim=32, n_idx=512, cores=4, chunk=32, seed=42, hot=None):
    """out[didx[i], :] = out[didx[i], :] + extf(table[sidx[i], :]): the
    gather + scatter-add kernel with its source rows named by a second index
    tensor, so updates of one destination row add different rows and their
    order shows in the f32 sums.  `hot`: destination indices drawn from
    [0, hot) (long chains)."""
    rng = np.random.default_rng(seed)
    src = configs.gather_scatter_add(rows, dim, n_idx, cores, chunk)
    sig = "%table_ptr: index, %idx_ptr: index, %out_ptr: index)"
    assert src.count(sig) == 1
    src = src.replace(sig, "%table_ptr: index, %idx_ptr: index, %out_ptr: index, %sidx_ptr: index)")
    view = configs._view("idx_view", "idx_ptr", [n_idx], [1], "i32")
    assert src.count(view) == 1
    src = src.replace(view, view + "\n" + configs._view("sidx_view", "sidx_ptr", [n_idx], [1], "i32"))
    g = "%table_view[ind(%idx_view[%row0 + %r]), (%c)]"
    assert src.count(g) == 1
    src = src.replace(g, "%table_view[ind(%sidx_view[%row0 + %r]), (%c)]")
    table = rng.standard_normal((rows, dim)).astype(np.float16)
    didx = rng.integers(0, hot or rows, n_idx).astype(np.int32)
    sidx = rng.integers(0, rows, n_idx).astype(np.int32)
    out = rng.standard_normal((rows, dim)).astype(np.float32)
    return src, "gather_scatter_add", dict(table_ptr=table, idx_ptr=didx, out_ptr=out, sidx_ptr=sidx)


def _half(x, dt):
    """f32 values as the element type's storage: f16 values, or bf16 bit patterns."""
    return x.astype(np.float16) if dt == "f16" else bf16_bits(x.astype(np.float32))


def softmax(rows=64, cols=256, cores=8, rblk=4, seed=42, dt="f16"):
    rng = np.random.default_rng(seed)
    x = _half(rng.standard_normal((rows, cols)) * 2, dt)
    return configs.softmax(rows, cols, cores, rblk, dt), "softmax_kernel", dict(x_ptr=x, y_ptr=np.zeros_like(x))


def rmsnorm(rows=64, cols=256, cores=8, rblk=4, seed=42, dt="f16", wide=False):
    """`wide`: magnitudes spread over eight decades, so that the order of the
    sum of squares shows in the result bits."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)) * 2
    if wide:
        x = x * 10.0 ** rng.uniform(-4, 3.5, (rows, cols))
    x = _half(x, dt)
    w = _half(rng.uniform(0.5, 1.5, cols), dt)
    return (configs.rmsnorm(rows, cols, cores, rblk, dt), "rmsnorm_kernel",
            dict(x_ptr=x, w_ptr=w, y_ptr=np.zeros_like(x), eps=1e-6))


def gemm(M=256, N=256, K=256, bm=64, bn=64, bk=32, gm=2, gn=2, seed=42, out_dt="f16"):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((M, K)) * K ** -0.5).astype(np.float16)
    b = (rng.standard_normal((K, N)) * K ** -0.5).astype(np.float16)
    return (configs.gemm(M, N, K, bm, bn, bk, gm, gn, out_dt), "gemm_kernel",
            dict(a_ptr=a, b_ptr=b, c_ptr=np.zeros((M, N), np.float16 if out_dt == "f16" else np.float32)))


def gemm_bf16(M=256, N=256, K=512, bm=128, bn=128, bk=64, gm=2, gn=2, seed=7):
    """The tiled GEMM with bf16 operands and a bf16 result (the f32 K-loop
    sums rounded once by the store's truncf)."""
    rng = np.random.default_rng(seed)
    a = bf16_bits((rng.standard_normal((M, K)) * K ** -0.5).astype(np.float32))
    b = bf16_bits((rng.standard_normal((K, N)) * K ** -0.5).astype(np.float32))
    src = configs.gemm(M, N, K, bm, bn, bk, gm, gn).replace("f16", "bf16")
    return src, "gemm_kernel", dict(a_ptr=a, b_ptr=b, c_ptr=np.zeros((M, N), np.uint16))


def flash_attention(B=1, H=2, S=256, D=32, blk=64, seed=42, dt="bf16", causal=True):
    rng = np.random.default_rng(seed)
    if dt == "bf16":
        q, k, v = (bf16_bits(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    else:
        q, k, v = (rng.standard_normal((B, H, S, D)).astype(np.float16) for _ in range(3))
    return (configs.flash_attention(B, H, S, D, blk, dt=dt, causal=causal), "flash_attention",
            dict(q_ptr=q, k_ptr=k, v_ptr=v, o_ptr=np.zeros_like(q), scale=1.0 / math.sqrt(D)))


def row_reduce(rows=32, cols=4096, rblk=4, combiner="arith.addf", dt="f32", seed=5, nans=False, decades=6):
    """out[r] = fold of x[r, :] with `combiner` (the reference's pairwise-halving
    linalg.reduce), one core per rblk-row block; values spread over 2 x
    `decades` decades so the summation order shows in the result bits;
    `nans` puts a NaN in every other row."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * 10.0 ** rng.uniform(-decades, decades, (rows, cols))).astype(np.float32)
    if nans:
        # a NaN in every other row: the NaN-ignoring folds skip it, the others propagate it
        x[::2, rng.integers(0, cols, rows // 2 + rows % 2)] = np.nan
    if dt == "f16":
        x = x.astype(np.float16)
    elif dt == "bf16":
        from oracle.interp import bf16_bits
        x = bf16_bits(x)
    cores = rows // rblk
    T, V = configs._t([rblk, cols], dt), configs._t([rblk], dt)
    ninf = {"f32": "0xFF800000", "f16": "0xFC00", "bf16": "0xFF80"}[dt]
    pinf = {"f32": "0x7F800000", "f16": "0x7C00", "bf16": "0x7F80"}[dt]
    init = {"arith.addf": "0.0", "arith.maximumf": ninf, "arith.maxnumf": ninf, "arith.minnumf": pinf,
            "arith.mulf": "1.0"}[combiner]
    src = f"""module {{
  func.func @row_reduce(%x_ptr: index, %y_ptr: index) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %RB = arith.constant {rblk} : index
    %init = arith.constant {init} : {dt}
{configs._view("x_view", "x_ptr", [rows, cols], [cols, 1], dt)}
{configs._view("y_view", "y_ptr", [rows], [1], dt)}
    %row = arith.muli %core_id, %RB : index
{configs._tile("x_acc", "x_view", ["%row", "%c0"], [rblk, cols], [rows, cols], dt)}
    %x = ktdp.load %x_acc : !ktdp.access_tile<{rblk}x{cols}xindex> -> {T}
    %i = tensor.splat %init : {V}
    %r = linalg.reduce {{ {combiner} }} ins(%x : {T}) outs(%i : {V}) dimensions = [1]
{configs._tile("y_acc", "y_view", ["%row"], [rblk], [rows], dt)}
    ktdp.store %r, %y_acc : {V}, !ktdp.access_tile<{rblk}xindex>
    return
  }}
}}
"""
    return src, "row_reduce", dict(x_ptr=x, y_ptr=np.zeros(rows, x.dtype))


def unary_f32(op="math.sqrt", n=1 << 14, block=512, cores=32, seed=11):
    """out = op(x) on f32 values spread over many decades (x > 0)."""
    rng = np.random.default_rng(seed)
    x = (10.0 ** rng.uniform(-30, 30, n)).astype(np.float32)
    bpc = n // (cores * block)
    assert bpc * cores * block == n
    T = configs._t([block], "f32")
    src = f"""module {{
  func.func @unary_kernel(%x_ptr: index, %y_ptr: index) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %bpc = arith.constant {bpc} : index
    %B = arith.constant {block} : index
{configs._view("x_view", "x_ptr", [n], [1], "f32")}
{configs._view("y_view", "y_ptr", [n], [1], "f32")}
    %first = arith.muli %core_id, %bpc : index
    scf.for %b = %c0 to %bpc step %c1 : index {{
      %blk = arith.addi %first, %b : index
      %off = arith.muli %blk, %B : index
{configs._tile("x_tile", "x_view", ["%off"], [block], [n], "f32", "      ")}
      %x = ktdp.load %x_tile : !ktdp.access_tile<{block}xindex> -> {T}
      %y = {op} %x : {T}
{configs._tile("y_tile", "y_view", ["%off"], [block], [n], "f32", "      ")}
      ktdp.store %y, %y_tile : {T}, !ktdp.access_tile<{block}xindex>
      scf.yield
    }}
    return
  }}
}}
"""
    return src, "unary_kernel", dict(x_ptr=x, y_ptr=np.zeros_like(x))


def elementwise(body, ins, out_dt, n=4096, cores=4, name="ew_kernel"):
    """One tile per core: load each input (`ins`: list of dtypes, SSA names
    %a, %b, %c, ...), run `body` (KTIR lines over those names and the tile
    type `T<dt>` written as {T_dt}), store %r (dtype `out_dt`) to the output.
    Returns (src, fn, arg-name list)."""
    blk = n // cores
    assert blk * cores == n
    names = "abcdefg"[:len(ins)]
    args = ", ".join([f"%{x}_ptr: index" for x in names] + ["%r_ptr: index"])
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             f"    %B = arith.constant {blk} : index",
             "    %off = arith.muli %core_id, %B : index"]
    at = f"!ktdp.access_tile<{blk}xindex>"
    for x, dt in zip(names, ins):
        lines.append(configs._view(f"{x}_view", f"{x}_ptr", [n], [1], dt))
        lines.append(configs._tile(f"{x}_t", f"{x}_view", ["%off"], [blk], [n], dt))
        lines.append(f"    %{x} = ktdp.load %{x}_t : {at} -> {configs._t([blk], dt)}")
    types = {f"T_{dt}": configs._t([blk], dt) for dt in ("f16", "bf16", "f32", "i1", "i32", "i64")}
    lines += ["    " + ln.format(**types) for ln in body]
    lines.append(configs._view("r_view", "r_ptr", [n], [1], out_dt))
    lines.append(configs._tile("r_t", "r_view", ["%off"], [blk], [n], out_dt))
    lines.append(f"    ktdp.store %r, %r_t : {configs._t([blk], out_dt)}, {at}")
    src = (f"module {{\n  func.func @{name}({args}) attributes {{grid = [{cores}, 1]}} {{\n"
           + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, name, [f"{x}_ptr" for x in names] + ["r_ptr"]


def f16_patterns(n, seed=0, specials=True):
    """`n` f16 values: random bit patterns (all exponents, subnormals
    included), plus zeros, infinities and NaN when `specials`."""
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    v = bits.view(np.float16).copy()
    if specials:
        v[:8] = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 65504.0], np.float16)
    else:
        v[~np.isfinite(v)] = np.float16(1.5)
    return v


def gather_rows(rows=2048, dim=128, n_idx=1024, cores=8, chunk=64, seed=3):
    """Plain blocked-indirect row gather: out[i, :] = table[idx[i], :] (f16),
    chunk by chunk, no read-modify-write (the unfused indirect load path)."""
    rng = np.random.default_rng(seed)
    table = rng.standard_normal((rows, dim)).astype(np.float16)
    idx = rng.integers(0, rows, n_idx).astype(np.int32)
    per_core = n_idx // cores
    nch = per_core // chunk
    vss = f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {chunk - 1} >= 0, d1 >= 0, -d1 + {dim - 1} >= 0)>"
    T = configs._t([chunk, dim], "f16")
    src = f"""module {{
  func.func @gather_rows(%table_ptr: index, %idx_ptr: index, %out_ptr: index) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %nch = arith.constant {nch} : index
    %per_core = arith.constant {per_core} : index
    %chunk = arith.constant {chunk} : index
{configs._view("table_view", "table_ptr", [rows, dim], [dim, 1], "f16")}
{configs._view("idx_view", "idx_ptr", [n_idx], [1], "i32")}
{configs._view("out_view", "out_ptr", [n_idx, dim], [dim, 1], "f16")}
    %core_base = arith.muli %core_id, %per_core : index
    scf.for %ch = %c0 to %nch step %c1 : index {{
      %ch_off = arith.muli %ch, %chunk : index
      %row0 = arith.addi %core_base, %ch_off : index
      %g_tile = ktdp.construct_indirect_access_tile intermediate_variables(%r, %c)
          %table_view[ind(%idx_view[%row0 + %r]), (%c)] {{
        variables_space_set = {vss},
        variables_space_order = affine_map<(d0, d1) -> (d0, d1)>
      }} : memref<{rows}x{dim}xf16>, memref<{n_idx}xi32> -> !ktdp.access_tile<{chunk}x{dim}xindex>
      %g = ktdp.load %g_tile : !ktdp.access_tile<{chunk}x{dim}xindex> -> {T}
{configs._tile("o_tile", "out_view", ["%row0", "%c0"], [chunk, dim], [n_idx, dim], "f16", "      ")}
      ktdp.store %g, %o_tile : {T}, !ktdp.access_tile<{chunk}x{dim}xindex>
      scf.yield
    }}
    return
  }}
}}
"""
    return src, "gather_rows", dict(table_ptr=table, idx_ptr=idx, out_ptr=np.zeros((n_idx, dim), np.float16))


# ---------------------------------------------------------------------------
# distributed memory views (two partitions of a 4 x 4 f16 tensor)
# ---------------------------------------------------------------------------

# (id, p0, p1, access shape, access indices); a partition is
# (rows (first, last), cols (first, last), space, strides, element address).
# The layouts and expected slices are the reference's test table
# (tests/test_distributed_view.py:207-470): the tensor is arange(16) and
# the result is its access-tile slice.
DIST_CASES = [
    ("row_hbm_hbm_full", ((0, 1), (0, 3), "HBM", (4, 1), 0), ((2, 3), (0, 3), "HBM", (4, 1), 4096), (4, 4), (0, 0)),
    ("row_hbm_hbm_partial_p1_pruned", ((0, 1), (0, 3), "HBM", (4, 1), 0), ((2, 3), (0, 3), "HBM", (4, 1), 4096),
     (2, 4), (0, 0)),
    ("row_hbm_hbm_subtile_nonzero", ((0, 1), (0, 3), "HBM", (4, 1), 0), ((2, 3), (0, 3), "HBM", (4, 1), 4096),
     (2, 2), (1, 1)),
    ("row_hbm_lx_col_packed_full", ((0, 1), (0, 3), "HBM", (4, 1), 0), ((2, 3), (0, 3), "LX", (1, 4), 4096),
     (4, 4), (0, 0)),
    ("row_lx_hbm_col_packed_full", ((0, 1), (0, 3), "LX", (1, 4), 0), ((2, 3), (0, 3), "HBM", (4, 1), 4096),
     (4, 4), (0, 0)),
    ("row_hbm_lx_subtile_nonzero", ((0, 1), (0, 3), "HBM", (4, 1), 0), ((2, 3), (0, 3), "LX", (1, 4), 4096),
     (2, 2), (1, 1)),
    ("row_hbm_hbm_unequal_full", ((0, 0), (0, 3), "HBM", (4, 1), 0), ((1, 3), (0, 3), "HBM", (4, 1), 4096),
     (4, 4), (0, 0)),
    ("row_hbm_hbm_unequal_partial_p0_pruned", ((0, 0), (0, 3), "HBM", (4, 1), 0),
     ((1, 3), (0, 3), "HBM", (4, 1), 4096), (2, 4), (1, 0)),
    ("col_hbm_hbm_full", ((0, 3), (0, 1), "HBM", (2, 1), 0), ((0, 3), (2, 3), "HBM", (2, 1), 4096), (4, 4), (0, 0)),
    ("col_hbm_hbm_partial_p1_pruned", ((0, 3), (0, 1), "HBM", (2, 1), 0), ((0, 3), (2, 3), "HBM", (2, 1), 4096),
     (4, 2), (0, 0)),
    ("col_hbm_hbm_subtile_nonzero", ((0, 3), (0, 1), "HBM", (2, 1), 0), ((0, 3), (2, 3), "HBM", (2, 1), 4096),
     (2, 2), (1, 1)),
    ("col_hbm_lx_col_packed_full", ((0, 3), (0, 1), "HBM", (2, 1), 0), ((0, 3), (2, 3), "LX", (1, 4), 4096),
     (4, 4), (0, 0)),
    ("mixed_left_block_only", ((0, 3), (0, 1), "HBM", (2, 1), 0), ((2, 3), (2, 3), "HBM", (2, 1), 4096),
     (4, 2), (0, 0)),
    ("mixed_bottom_left_only", ((0, 3), (0, 1), "HBM", (2, 1), 0), ((2, 3), (2, 3), "HBM", (2, 1), 4096),
     (2, 2), (2, 0)),
    ("mixed_lx_left_hbm_right_bottom_only", ((0, 3), (0, 1), "LX", (1, 4), 0), ((2, 3), (2, 3), "HBM", (2, 1), 4096),
     (2, 2), (2, 0)),
]
DIST_OUT = 8192      # element address of the output (f16)


def _box_set(r0, r1, c0, c1):
    return f"affine_set<(d0, d1) : (d0 - {r0} >= 0, -d0 + {r1} >= 0, d1 - {c0} >= 0, -d1 + {c1} >= 0)>"


def _space(sp, ct=None):
    if sp == "HBM":
        return "#ktdp.memory_space<global>"
    return "#ktdp.memory_space<ct_local>" if ct is None else f"#ktdp.memory_space<ct_local, ct_id = {ct}>"


def dist_copy(p0, p1, ashape, idx, gshape=(4, 4)):
    """Load an access tile of a two-partition distributed view at literal
    element addresses and store it to a contiguous output at DIST_OUT."""
    parts = []
    for k, (rows, cols, sp, st, addr) in enumerate((p0, p1)):
        nr, nc = rows[1] - rows[0] + 1, cols[1] - cols[0] + 1
        parts.append(f"""    %a{k} = arith.constant {addr} : index
    %P{k} = ktdp.construct_memory_view %a{k}, sizes: [{nr}, {nc}], strides: [{st[0]}, {st[1]}] {{
      coordinate_set = {_box_set(rows[0], rows[1], cols[0], cols[1])}, memory_space = {_space(sp)}
    }} : memref<{nr}x{nc}xf16>""")
    m = lambda p: f"memref<{p[0][1] - p[0][0] + 1}x{p[1][1] - p[1][0] + 1}xf16>"
    acs = _box_set(0, ashape[0] - 1, 0, ashape[1] - 1)
    G = f"memref<{gshape[0]}x{gshape[1]}xf16>"
    return f"""module {{
  func.func @dist_copy() attributes {{grid = [1, 1]}} {{
    %c0 = arith.constant 0 : index
    %i0 = arith.constant {idx[0]} : index
    %i1 = arith.constant {idx[1]} : index
{parts[0]}
{parts[1]}
    %A = ktdp.construct_distributed_memory_view (%P0, %P1 : {m(p0)}, {m(p1)}) : {G}
    %ob = arith.constant {DIST_OUT} : index
    %B = ktdp.construct_memory_view %ob, sizes: [{ashape[0]}, {ashape[1]}], strides: [{ashape[1]}, 1] {{
      coordinate_set = {acs}, memory_space = #ktdp.memory_space<global>
    }} : memref<{ashape[0]}x{ashape[1]}xf16>
    %at = ktdp.construct_access_tile %A[%i0, %i1] {{
      access_tile_set = {acs}, access_tile_order = affine_map<(d0, d1) -> (d0, d1)>
    }} : {G} -> !ktdp.access_tile<{ashape[0]}x{ashape[1]}xindex>
    %bt = ktdp.construct_access_tile %B[%c0, %c0] {{
      access_tile_set = {acs}, access_tile_order = affine_map<(d0, d1) -> (d0, d1)>
    }} : memref<{ashape[0]}x{ashape[1]}xf16> -> !ktdp.access_tile<{ashape[0]}x{ashape[1]}xindex>
    %v = ktdp.load %at : !ktdp.access_tile<{ashape[0]}x{ashape[1]}xindex> -> tensor<{ashape[0]}x{ashape[1]}xf16>
    ktdp.store %v, %bt : tensor<{ashape[0]}x{ashape[1]}xf16>, !ktdp.access_tile<{ashape[0]}x{ashape[1]}xindex>
    return
  }}
}}
"""


def strided_block(block, strides):
    """The memory image of a 2-D block laid out with element `strides`
    (holes zero), as the reference's test seeds partitions."""
    r, c = np.indices(block.shape)
    offs = (r * strides[0] + c * strides[1]).reshape(-1)
    buf = np.zeros(int(offs.max()) + 1, dtype=block.dtype)
    buf[offs] = block.reshape(-1)
    return buf


def dist_copy_2core():
    """A 192 x 64 f16 tensor over three partitions: rows 0..95 in HBM
    (row-major), rows 96..127 in core 0's LX (column-major, ct_id = 0), rows
    128..191 in core 1's LX (row-major, ct_id = 1).  Core c copies rows
    96c .. 96c + 95 to the output, so core 1 reads core 0's LX."""
    sets = [_box_set(0, 95, 0, 63), _box_set(96, 127, 0, 63), _box_set(128, 191, 0, 63)]
    acs = _box_set(0, 95, 0, 63)
    return f"""module {{
  func.func @dist_rows() attributes {{grid = [2, 1]}} {{
    %core = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %c96 = arith.constant 96 : index
    %row = arith.muli %core, %c96 : index
    %ah = arith.constant 0 : index
    %al0 = arith.constant 12288 : index
    %al1 = arith.constant 16384 : index
    %ab = arith.constant 24576 : index
    %H = ktdp.construct_memory_view %ah, sizes: [96, 64], strides: [64, 1] {{
      coordinate_set = {sets[0]}, memory_space = {_space("HBM")}
    }} : memref<96x64xf16>
    %L0 = ktdp.construct_memory_view %al0, sizes: [32, 64], strides: [1, 32] {{
      coordinate_set = {sets[1]}, memory_space = {_space("LX", 0)}
    }} : memref<32x64xf16>
    %L1 = ktdp.construct_memory_view %al1, sizes: [64, 64], strides: [64, 1] {{
      coordinate_set = {sets[2]}, memory_space = {_space("LX", 1)}
    }} : memref<64x64xf16>
    %A = ktdp.construct_distributed_memory_view (%H, %L0, %L1 : memref<96x64xf16>, memref<32x64xf16>, memref<64x64xf16>) : memref<192x64xf16>
    %B = ktdp.construct_memory_view %ab, sizes: [192, 64], strides: [64, 1] {{
      coordinate_set = {_box_set(0, 191, 0, 63)}, memory_space = {_space("HBM")}
    }} : memref<192x64xf16>
    %at = ktdp.construct_access_tile %A[%row, %c0] {{
      access_tile_set = {acs}, access_tile_order = affine_map<(d0, d1) -> (d0, d1)>
    }} : memref<192x64xf16> -> !ktdp.access_tile<96x64xindex>
    %bt = ktdp.construct_access_tile %B[%row, %c0] {{
      access_tile_set = {acs}, access_tile_order = affine_map<(d0, d1) -> (d0, d1)>
    }} : memref<192x64xf16> -> !ktdp.access_tile<96x64xindex>
    %v = ktdp.load %at : !ktdp.access_tile<96x64xindex> -> tensor<96x64xf16>
    ktdp.store %v, %bt : tensor<96x64xf16>, !ktdp.access_tile<96x64xindex>
    return
  }}
}}
"""


DIST_IN = 8192       # element address of the stored tile's source (f16)


def dist_store(p0, p1, ashape, idx, gshape=(4, 4)):
    """Load a contiguous tile from DIST_IN and store it through an access
    tile of a two-partition distributed view (partitions as in dist_copy)."""
    src = dist_copy(p0, p1, ashape, idx, gshape).replace("@dist_copy", "@dist_store")
    src = src.replace(f"%ob = arith.constant {DIST_OUT} : index", f"%ob = arith.constant {DIST_IN} : index")
    t = f"!ktdp.access_tile<{ashape[0]}x{ashape[1]}xindex>"
    r = f"tensor<{ashape[0]}x{ashape[1]}xf16>"
    src = src.replace(f"    %v = ktdp.load %at : {t} -> {r}\n    ktdp.store %v, %bt : {r}, {t}\n",
                      f"    %v = ktdp.load %bt : {t} -> {r}\n    ktdp.store %v, %at : {r}, {t}\n")
    assert "ktdp.store %v, %at" in src
    return src


def lx_exchange(n=256, out=4096):
    """Two cores: each loads n f16 from its own LX (byte 0) and stores them
    into core 1's LX (ct_id = 1) and to HBM at element out + n * core.  Core
    0 runs first in the reference, so core 1 loads what core 0 stored."""
    box = f"affine_set<(d0) : (d0 >= 0, -d0 + {n - 1} >= 0)>"
    tile = f"!ktdp.access_tile<{n}xindex>"
    return f"""module {{
  func.func @lx_exchange() attributes {{grid = [2, 1]}} {{
    %core = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %cn = arith.constant {n} : index
    %ob = arith.constant {out} : index
    %off = arith.muli %core, %cn : index
    %own = ktdp.construct_memory_view %c0, sizes: [{n}], strides: [1] {{
      coordinate_set = {box}, memory_space = {_space("LX")}
    }} : memref<{n}xf16>
    %to1 = ktdp.construct_memory_view %c0, sizes: [{n}], strides: [1] {{
      coordinate_set = {box}, memory_space = {_space("LX", 1)}
    }} : memref<{n}xf16>
    %hv = ktdp.construct_memory_view %ob, sizes: [{2 * n}], strides: [1] {{
      coordinate_set = affine_set<(d0) : (d0 >= 0, -d0 + {2 * n - 1} >= 0)>, memory_space = {_space("HBM")}
    }} : memref<{2 * n}xf16>
    %ta = ktdp.construct_access_tile %own[%c0] {{
      access_tile_set = {box}, access_tile_order = affine_map<(d0) -> (d0)>
    }} : memref<{n}xf16> -> {tile}
    %tb = ktdp.construct_access_tile %to1[%c0] {{
      access_tile_set = {box}, access_tile_order = affine_map<(d0) -> (d0)>
    }} : memref<{n}xf16> -> {tile}
    %tc = ktdp.construct_access_tile %hv[%off] {{
      access_tile_set = {box}, access_tile_order = affine_map<(d0) -> (d0)>
    }} : memref<{2 * n}xf16> -> {tile}
    %v = ktdp.load %ta : {tile} -> tensor<{n}xf16>
    ktdp.store %v, %tb : tensor<{n}xf16>, {tile}
    ktdp.store %v, %tc : tensor<{n}xf16>, {tile}
    return
  }}
}}
"""


def ring_reduce(n_cores=4, cols=128, group_size=None, strided=False, combiner="add", iters=0, dtype="f16",
                only_core0=False):
    """Every core loads its row of a [n_cores, cols] tensor, the rows are
    combined across each group with ktdp.inter_tile_produce /
    inter_tile_reduce, and every core stores its group's result to its own
    output row.  Groups: `group_size` consecutive cores, or with `strided`
    n_cores / group_size groups g = {g, g + G, g + 2G, ...}.  `combiner`:
    "add" (linalg.add) or "max" (arith.maximumf).  With `iters` > 0 the
    reduce sits in an scf.for whose iter_arg accumulates the results.  With
    `only_core0` just core 0 reaches the reduce (the others skip it), which
    the reference reports as a deadlock."""
    gs = n_cores if group_size is None else group_size
    ng = n_cores // gs
    if strided:
        pset = (f"affine_set<(i)[g] : ((i - g) mod {ng} == 0, i - g >= 0, -i + g + {n_cores - ng} >= 0)>")
    else:
        pset = f"affine_set<(i)[g] : (i - {gs}*g >= 0, -i + {gs}*g + {gs - 1} >= 0)>"
    groups = f"affine_set<(g) : (g >= 0, -g + {ng - 1} >= 0)>"
    T = f"tensor<1x{cols}x{dtype}>"
    fut = f"!ktdp.tile_future<{T}, groups = {groups}>"
    row = f"affine_set<(d0, d1) : (d0 >= 0, -d0 >= 0, d1 >= 0, -d1 + {cols - 1} >= 0)>"
    idm = "affine_map<(d0, d1) -> (d0, d1)>"
    if combiner == "add":
        comb = (f"        %init = tensor.empty() : {T}\n"
                f"        %r = linalg.add ins(%lhs, %rhs : {T}, {T}) outs(%init : {T}) -> {T}\n")
    else:
        comb = f"        %r = arith.maximumf %lhs, %rhs : {T}\n"
    reduce_ops = f"""    %fut = ktdp.inter_tile_produce producer_tiles_per_group = {pset}
        : {T} -> {fut}
    {{
      ^bb0(%gid: index):
        ktdp.yield_partial %partial : {T}
    }}
    %e = tensor.empty() : {T}
    %id = linalg.fill ins(%z : {dtype}) outs(%e : {T}) -> {T}
    %red = ktdp.inter_tile_reduce(%fut) consumer_tiles_per_group = {pset}, identity(%id : {T})
        : {fut} -> {T}
    {{
      ^bb0(%lhs: {T}, %rhs: {T}):
{comb}        ktdp.yield_reduced %r : {T}
    }}
"""
    if iters:
        body = f"""    %z0 = arith.constant dense<0.0> : {T}
    %c1 = arith.constant 1 : index
    %cit = arith.constant {iters} : index
    %res = scf.for %it = %c0 to %cit step %c1 iter_args(%acc = %z0) -> ({T}) {{
{reduce_ops}      %nx = arith.addf %acc, %red : {T}
      scf.yield %nx : {T}
    }}
"""
    else:
        body = reduce_ops + "    %res = arith.addf %red, %zt : " + T + "\n"
    if only_core0:
        body = body.replace("    %fut = ktdp.inter_tile_produce", "    %is0 = arith.cmpi eq, %pid, %c0 : index\n"
                            "    scf.if %is0 {\n    %fut = ktdp.inter_tile_produce") + "    }\n"
        body = body.replace("    %res = arith.addf %red, %zt", "    %unused = arith.addf %red, %zt") + \
            "    %res = arith.addf %partial, %zt : " + T + "\n"
    return f"""module {{
  func.func @ring_reduce(%in_ptr: index, %out_ptr: index) attributes {{grid = [{n_cores}]}} {{
    %c0 = arith.constant 0 : index
    %cols = arith.constant {cols} : index
    %z = arith.constant 0.0 : {dtype}
    %zt = arith.constant dense<0.0> : {T}
    %pid = ktdp.get_compute_tile_id : index
    %offs = arith.muli %pid, %cols : index
    %rp = arith.addi %in_ptr, %offs : index
    %wp = arith.addi %out_ptr, %offs : index
    %rv = ktdp.construct_memory_view %rp, sizes: [1, {cols}], strides: [{cols}, 1] {{
      coordinate_set = {row}, memory_space = #ktdp.memory_space<global>
    }} : memref<1x{cols}x{dtype}>
    %ra = ktdp.construct_access_tile %rv[%c0, %c0] {{
      access_tile_set = {row}, access_tile_order = {idm}
    }} : memref<1x{cols}x{dtype}> -> !ktdp.access_tile<1x{cols}xindex>
    %partial = ktdp.load %ra : !ktdp.access_tile<1x{cols}xindex> -> {T}
{body}    %wv = ktdp.construct_memory_view %wp, sizes: [1, {cols}], strides: [{cols}, 1] {{
      coordinate_set = {row}, memory_space = #ktdp.memory_space<global>
    }} : memref<1x{cols}x{dtype}>
    %wa = ktdp.construct_access_tile %wv[%c0, %c0] {{
      access_tile_set = {row}, access_tile_order = {idm}
    }} : memref<1x{cols}x{dtype}> -> !ktdp.access_tile<1x{cols}xindex>
    ktdp.store %res, %wa : {T}, !ktdp.access_tile<1x{cols}xindex>
    return
  }}
}}
"""


def rmsnorm_2x2(rows=16, H=256):
    """RMSNorm over a [rows, H] f16 tensor on a 2 x 2 grid: core (c, r)
    owns columns c*H/2 .. and rows r*rows/2 ..; each row's sum of squares
    (f32) is folded across the two column partners with inter_tile_reduce.

    X is a distributed view whose left half is the argument X0 (HBM) and
    whose right half sits in core 1's LX at byte 0 (ct_id = 1, row-major),
    so cores 1 and 3 read core 1's scratchpad; W is one [1, H] tensor seen
    through two partitions; Y's halves are the separate arguments Y0, Y1."""
    h = H // 2
    rh = rows // 2
    T16, T32, V32 = f"tensor<1x{h}xf16>", f"tensor<1x{h}xf32>", "tensor<1xf32>"
    cset = lambda c0, c1, r1: f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {r1} >= 0, d1 - {c0} >= 0, -d1 + {c1} >= 0)>"
    blk = f"affine_set<(d0, d1) : (d0 >= 0, -d0 >= 0, d1 >= 0, -d1 + {h - 1} >= 0)>"
    idm = "affine_map<(d0, d1) -> (d0, d1)>"
    pset = "affine_set<(i)[g] : (i - 2*g >= 0, -i + 2*g + 1 >= 0)>"
    fut = f"!ktdp.tile_future<{V32}, groups = affine_set<(g) : (g >= 0, -g + 1 >= 0)>>"
    G, M = f"memref<{rows}x{H}xf16>", f"memref<{rows}x{h}xf16>"
    WG, WM = f"memref<1x{H}xf16>", f"memref<1x{h}xf16>"
    at = f"!ktdp.access_tile<1x{h}xindex>"

    def part(name, ptr, shape, cs, space):
        return (f"    %{name} = ktdp.construct_memory_view {ptr}, sizes: [{shape[0]}, {shape[1]}], "
                f"strides: [{shape[2]}, 1] {{\n      coordinate_set = {cs}, memory_space = {space}\n    }} : "
                f"memref<{shape[0]}x{shape[1]}xf16>")

    def tile(name, view, idx, mem):
        return (f"      %{name} = ktdp.construct_access_tile %{view}[{idx}] {{\n"
                f"        access_tile_set = {blk}, access_tile_order = {idm}\n      }} : {mem} -> {at}")

    hbm, lx1 = "#ktdp.memory_space<global>", "#ktdp.memory_space<ct_local, ct_id = 1>"
    return f"""module {{
  func.func @rmsnorm_2x2(%X0: index, %W: index, %Y0: index, %Y1: index, %eps: f16) attributes {{grid = [2, 2]}} {{
    %col_id, %row_id = ktdp.get_compute_tile_id : index, index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %ch = arith.constant {h} : index
    %crh = arith.constant {rh} : index
    %zero = arith.constant 0.0 : f32
    %nf = arith.constant {float(H)} : f32
    %row_start = arith.muli %row_id, %crh : index
    %row_end = arith.addi %row_start, %crh : index
    %col = arith.muli %col_id, %ch : index
    %W1 = arith.addi %W, %ch : index
{part("X_p0", "%X0", (rows, h, h), cset(0, h - 1, rows - 1), hbm)}
{part("X_p1", "%c0", (rows, h, h), cset(h, H - 1, rows - 1), lx1)}
    %X = ktdp.construct_distributed_memory_view (%X_p0, %X_p1 : {M}, {M}) : {G}
{part("W_p0", "%W", (1, h, H), cset(0, h - 1, 0), hbm)}
{part("W_p1", "%W1", (1, h, H), cset(h, H - 1, 0), hbm)}
    %Wv = ktdp.construct_distributed_memory_view (%W_p0, %W_p1 : {WM}, {WM}) : {WG}
{part("Y_p0", "%Y0", (rows, h, h), cset(0, h - 1, rows - 1), hbm)}
{part("Y_p1", "%Y1", (rows, h, h), cset(h, H - 1, rows - 1), hbm)}
    %Y = ktdp.construct_distributed_memory_view (%Y_p0, %Y_p1 : {M}, {M}) : {G}
{tile("w_t", "Wv", "%c0, %col", WG).replace("      ", "    ", 1)}
    %w = ktdp.load %w_t : {at} -> {T16}
    %wf = arith.extf %w : {T16} to {T32}
    scf.for %row = %row_start to %row_end step %c1 {{
{tile("x_t", "X", "%row, %col", G)}
      %x = ktdp.load %x_t : {at} -> {T16}
      %xf = arith.extf %x : {T16} to {T32}
      %sq = arith.mulf %xf, %xf : {T32}
      %ss_init = tensor.splat %zero : {V32}
      %ss = linalg.reduce {{ arith.addf }} ins(%sq : {T32}) outs(%ss_init : {V32}) dimensions = [1]
      %fut = ktdp.inter_tile_produce producer_tiles_per_group = {pset}
          : {V32} -> {fut}
      {{
        ^bb0(%gid: index):
          ktdp.yield_partial %ss : {V32}
      }}
      %id_init = tensor.empty() : {V32}
      %add_id = linalg.fill ins(%zero : f32) outs(%id_init : {V32}) -> {V32}
      %full = ktdp.inter_tile_reduce(%fut) consumer_tiles_per_group = {pset}, identity(%add_id : {V32})
          : {fut} -> {V32}
      {{
        ^bb0(%lhs: {V32}, %rhs: {V32}):
          %init = tensor.empty() : {V32}
          %sum = linalg.add ins(%lhs, %rhs : {V32}, {V32}) outs(%init : {V32}) -> {V32}
          ktdp.yield_reduced %sum : {V32}
      }}
      %s = tensor.extract %full[%c0] : {V32}
      %ms = arith.divf %s, %nf : f32
      %mse = arith.addf %ms, %eps : f32
      %rstd = math.rsqrt %mse : f32
      %rb = tensor.splat %rstd : {T32}
      %xn = arith.mulf %xf, %rb : {T32}
      %yf = arith.mulf %xn, %wf : {T32}
      %y = arith.truncf %yf : {T32} to {T16}
{tile("y_t", "Y", "%row, %col", G)}
      ktdp.store %y, %y_t : {T16}, {at}
      scf.yield
    }}
    return
  }}
}}
"""


def splitk_pv(K=1024, N=128, nx=2, ny=4):
    """Decode P @ V split over a [nx, ny] grid (the reference's
    examples/sdsc/sdpa_pv_ksplit.mlir shape of problem, written here): core
    (x, y) multiplies P[0, yK/ny ..] (1 x K/ny, f16) by V[yK/ny .., xN/nx ..]
    in f32, rounds the 1 x N/nx partial to f16, and the partials of the cores
    with the same x -- the strided group {x, x + nx, x + 2 nx, ...} of linear
    ids -- are summed by inter_tile_reduce (an f16 combiner); core (x, 0)
    stores C[0, xN/nx ..]."""
    kb, nb = K // ny, N // nx
    T = lambda s, dt: f"tensor<{s[0]}x{s[1]}x{dt}>"
    pset = f"affine_set<(i)[g] : ((i - g) mod {nx} == 0, i - g >= 0, -i + g + {nx * ny - nx} >= 0)>"
    groups = f"affine_set<(g) : (g >= 0, -g + {nx - 1} >= 0)>"
    fut = f"!ktdp.tile_future<{T((1, nb), 'f16')}, groups = {groups}>"
    box = lambda r, c: f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {r - 1} >= 0, d1 >= 0, -d1 + {c - 1} >= 0)>"
    idm = "affine_map<(d0, d1) -> (d0, d1)>"
    hbm = "#ktdp.memory_space<global>"

    def view(name, ptr, shape, strides):
        return (f"    %{name} = ktdp.construct_memory_view %{ptr}, sizes: [{shape[0]}, {shape[1]}], strides: "
                f"[{strides[0]}, {strides[1]}] {{\n      coordinate_set = {box(*shape)}, memory_space = {hbm}\n"
                f"    }} : memref<{shape[0]}x{shape[1]}xf16>")

    def tile(name, v, idx, shape, vshape):
        return (f"    %{name} = ktdp.construct_access_tile %{v}[{idx}] {{\n      access_tile_set = {box(*shape)}, "
                f"access_tile_order = {idm}\n    }} : memref<{vshape[0]}x{vshape[1]}xf16> -> "
                f"!ktdp.access_tile<{shape[0]}x{shape[1]}xindex>")
    return f"""module {{
  func.func @splitk_pv(%p_ptr: index, %v_ptr: index, %c_ptr: index) attributes {{grid = [{nx}, {ny}]}} {{
    %x, %y = ktdp.get_compute_tile_id : index, index
    %c0 = arith.constant 0 : index
    %ckb = arith.constant {kb} : index
    %cnb = arith.constant {nb} : index
    %k0 = arith.muli %y, %ckb : index
    %n0 = arith.muli %x, %cnb : index
{view("pv", "p_ptr", (1, K), (K, 1))}
{view("vv", "v_ptr", (K, N), (N, 1))}
{view("cv", "c_ptr", (1, N), (N, 1))}
{tile("pt", "pv", "%c0, %k0", (1, kb), (1, K))}
{tile("vt", "vv", "%k0, %n0", (kb, nb), (K, N))}
    %p = ktdp.load %pt : !ktdp.access_tile<1x{kb}xindex> -> {T((1, kb), 'f16')}
    %v = ktdp.load %vt : !ktdp.access_tile<{kb}x{nb}xindex> -> {T((kb, nb), 'f16')}
    %pf = arith.extf %p : {T((1, kb), 'f16')} to {T((1, kb), 'f32')}
    %vf = arith.extf %v : {T((kb, nb), 'f16')} to {T((kb, nb), 'f32')}
    %zf = arith.constant 0.0 : f32
    %acc0 = tensor.splat %zf : {T((1, nb), 'f32')}
    %prod = linalg.matmul ins(%pf, %vf : {T((1, kb), 'f32')}, {T((kb, nb), 'f32')}) outs(%acc0 : {T((1, nb), 'f32')}) -> {T((1, nb), 'f32')}
    %part = arith.truncf %prod : {T((1, nb), 'f32')} to {T((1, nb), 'f16')}
    %fut = ktdp.inter_tile_produce producer_tiles_per_group = {pset}
        : {T((1, nb), 'f16')} -> {fut}
    {{
      ^bb0(%gid: index):
        ktdp.yield_partial %part : {T((1, nb), 'f16')}
    }}
    %z = arith.constant 0.0 : f16
    %e = tensor.empty() : {T((1, nb), 'f16')}
    %id = linalg.fill ins(%z : f16) outs(%e : {T((1, nb), 'f16')}) -> {T((1, nb), 'f16')}
    %red = ktdp.inter_tile_reduce(%fut) consumer_tiles_per_group = {pset}, identity(%id : {T((1, nb), 'f16')})
        : {fut} -> {T((1, nb), 'f16')}
    {{
      ^bb0(%lhs: {T((1, nb), 'f16')}, %rhs: {T((1, nb), 'f16')}):
        %init = tensor.empty() : {T((1, nb), 'f16')}
        %s = linalg.add ins(%lhs, %rhs : {T((1, nb), 'f16')}, {T((1, nb), 'f16')}) outs(%init : {T((1, nb), 'f16')}) -> {T((1, nb), 'f16')}
        ktdp.yield_reduced %s : {T((1, nb), 'f16')}
    }}
    %is0 = arith.cmpi eq, %y, %c0 : index
    scf.if %is0 {{
{tile("ct", "cv", "%c0, %n0", (1, nb), (1, N)).replace("    ", "      ", 1)}
      ktdp.store %red, %ct : {T((1, nb), 'f16')}, !ktdp.access_tile<1x{nb}xindex>
    }}
    return
  }}
}}
"""


def ffn_swiglu_4core(seq=4, d=256, f=1024, cores=4):
    """SwiGLU feed-forward with the hidden dimension split over `cores`
    cores (the shape of problem of the reference's ffn_swiglu_4core
    example, written here): x [seq, d] is read by every core; core c owns
    columns c*f/cores .. of W_gate and W_up and the matching rows of W_down,
    computes h = silu(x W_gate_c) * (x W_up_c) and its partial h W_down_c
    (f16 matmuls, f32 accumulation inside), the partials are summed by
    inter_tile_reduce, and core 0 adds the residual x and stores."""
    fc = f // cores
    T = lambda r, c: f"tensor<{r}x{c}xf16>"
    box = lambda r, c: f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {r - 1} >= 0, d1 >= 0, -d1 + {c - 1} >= 0)>"
    idm = "affine_map<(d0, d1) -> (d0, d1)>"
    hbm = "#ktdp.memory_space<global>"
    pset = f"affine_set<(i)[g] : (i - {cores}*g >= 0, -i + {cores}*g + {cores - 1} >= 0)>"
    fut = f"!ktdp.tile_future<{T(seq, d)}, groups = affine_set<(g) : (g == 0)>>"

    def view(name, ptr, shape):
        return (f"    %{name} = ktdp.construct_memory_view %{ptr}, sizes: [{shape[0]}, {shape[1]}], strides: "
                f"[{shape[1]}, 1] {{\n      coordinate_set = {box(*shape)}, memory_space = {hbm}\n    }} : "
                f"memref<{shape[0]}x{shape[1]}xf16>")

    def load(name, v, idx, shape, vshape):
        return (f"    %{name}_t = ktdp.construct_access_tile %{v}[{idx}] {{\n      access_tile_set = {box(*shape)}, "
                f"access_tile_order = {idm}\n    }} : memref<{vshape[0]}x{vshape[1]}xf16> -> "
                f"!ktdp.access_tile<{shape[0]}x{shape[1]}xindex>\n"
                f"    %{name} = ktdp.load %{name}_t : !ktdp.access_tile<{shape[0]}x{shape[1]}xindex> -> "
                f"{T(*shape)}")
    return f"""module {{
  func.func @ffn_swiglu(%x_ptr: index, %wg_ptr: index, %wu_ptr: index, %wd_ptr: index, %out_ptr: index)
      attributes {{grid = [{cores}]}} {{
    %c = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %cfc = arith.constant {fc} : index
    %col = arith.muli %c, %cfc : index
    %one = arith.constant 1.0 : f16
    %zero = arith.constant 0.0 : f16
{view("xv", "x_ptr", (seq, d))}
{view("wgv", "wg_ptr", (d, f))}
{view("wuv", "wu_ptr", (d, f))}
{view("wdv", "wd_ptr", (f, d))}
{view("ov", "out_ptr", (seq, d))}
{load("x", "xv", "%c0, %c0", (seq, d), (seq, d))}
{load("wg", "wgv", "%c0, %col", (d, fc), (d, f))}
{load("wu", "wuv", "%c0, %col", (d, fc), (d, f))}
{load("wd", "wdv", "%col, %c0", (fc, d), (f, d))}
    %g0 = tensor.splat %zero : {T(seq, fc)}
    %gate = linalg.matmul ins(%x, %wg : {T(seq, d)}, {T(d, fc)}) outs(%g0 : {T(seq, fc)}) -> {T(seq, fc)}
    %u0 = tensor.splat %zero : {T(seq, fc)}
    %up = linalg.matmul ins(%x, %wu : {T(seq, d)}, {T(d, fc)}) outs(%u0 : {T(seq, fc)}) -> {T(seq, fc)}
    %ng = arith.negf %gate : {T(seq, fc)}
    %en = math.exp %ng : {T(seq, fc)}
    %ones = tensor.splat %one : {T(seq, fc)}
    %den = arith.addf %ones, %en : {T(seq, fc)}
    %silu = arith.divf %gate, %den : {T(seq, fc)}
    %h = arith.mulf %silu, %up : {T(seq, fc)}
    %p0 = tensor.splat %zero : {T(seq, d)}
    %part = linalg.matmul ins(%h, %wd : {T(seq, fc)}, {T(fc, d)}) outs(%p0 : {T(seq, d)}) -> {T(seq, d)}
    %fut = ktdp.inter_tile_produce producer_tiles_per_group = {pset}
        : {T(seq, d)} -> {fut}
    {{
      ^bb0(%gid: index):
        ktdp.yield_partial %part : {T(seq, d)}
    }}
    %e = tensor.empty() : {T(seq, d)}
    %id = linalg.fill ins(%zero : f16) outs(%e : {T(seq, d)}) -> {T(seq, d)}
    %sum = ktdp.inter_tile_reduce(%fut) consumer_tiles_per_group = {pset}, identity(%id : {T(seq, d)})
        : {fut} -> {T(seq, d)}
    {{
      ^bb0(%lhs: {T(seq, d)}, %rhs: {T(seq, d)}):
        %init = tensor.empty() : {T(seq, d)}
        %s = linalg.add ins(%lhs, %rhs : {T(seq, d)}, {T(seq, d)}) outs(%init : {T(seq, d)}) -> {T(seq, d)}
        ktdp.yield_reduced %s : {T(seq, d)}
    }}
    %y = arith.addf %sum, %x : {T(seq, d)}
    %is0 = arith.cmpi eq, %c, %c0 : index
    scf.if %is0 {{
      %o_t = ktdp.construct_access_tile %ov[%c0, %c0] {{
        access_tile_set = {box(seq, d)}, access_tile_order = {idm}
      }} : memref<{seq}x{d}xf16> -> !ktdp.access_tile<{seq}x{d}xindex>
      ktdp.store %y, %o_t : {T(seq, d)}, !ktdp.access_tile<{seq}x{d}xindex>
    }}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# linalg.reduce over other axes, several axes and all axes; linalg.generic
# with reduction iterators; linalg.batch_matmul
# ---------------------------------------------------------------------------

def _nd_box(shape):
    dims = ", ".join(f"d{i}" for i in range(len(shape)))
    cons = ", ".join(f"d{i} >= 0, -d{i} + {s - 1} >= 0" for i, s in enumerate(shape))
    return f"affine_set<({dims}) : ({cons})>", f"affine_map<({dims}) -> ({dims})>"


def _core_tile(name, view, shape, full, dt, row="%row0"):
    """Access tile of `shape` at row `row` of a view of shape `full`."""
    idx = [row] + ["%c0"] * (len(shape) - 1)
    return configs._tile(name, view, idx, list(shape), list(full), dt)


def reduce_kernel(shape=(3, 4, 2), dims=(0, 2), dt="f32", init=0.0, combiner="arith.addf", cores=2,
                  region=False):
    """Each core loads its `shape` block of x (blocks stacked on axis 0),
    reduces it over `dims` (None: every axis, to a scalar) with outs
    initialised to `init`, and stores the result (a scalar through a
    one-element tensor.splat).  `region` writes the combiner as an explicit
    region instead of the shorthand."""
    nd = len(shape)
    full = (shape[0] * cores,) + tuple(shape[1:])
    rshape = tuple(s for i, s in enumerate(shape) if dims is not None and i not in dims)
    rfull = (rshape[0] * cores,) + rshape[1:] if rshape else (cores,)
    T = configs._t(list(shape), dt)
    if region:
        comb = (f"(%in: {dt}, %acc: {dt}) {{\n        %cmb = {combiner} %in, %acc : {dt}\n"
                f"        linalg.yield %cmb : {dt}\n      }}")
        head, tail = "", f"\n      {comb}"
    else:
        head, tail = f" {{ {combiner} }}", ""
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %c_rows = arith.constant {shape[0]} : index",
             "    %row0 = arith.muli %core_id, %c_rows : index",
             f"    %c_orows = arith.constant {rshape[0] if rshape else 1} : index",
             "    %orow0 = arith.muli %core_id, %c_orows : index",
             configs._view("x_view", "x_ptr", list(full), list(_cstr(full)), dt),
             configs._view("y_view", "y_ptr", list(rfull), list(_cstr(rfull)), dt),
             _core_tile("xt", "x_view", shape, full, dt),
             f"    %x = ktdp.load %xt : !ktdp.access_tile<{'x'.join(map(str, shape))}xindex> -> {T}",
             f"    %iv = arith.constant {init!r} : {dt}"]
    if dims is None or not rshape:
        dd = "" if dims is None else f" dimensions = {list(dims)}"
        lines += [f"    %init = tensor.splat %iv : tensor<{dt}>",
                  f"    %s = linalg.reduce{head} ins(%x : {T}) outs(%init : tensor<{dt}>){dd}{tail}",
                  f"    %r = tensor.splat %s : tensor<1x{dt}>",
                  configs._tile("yt", "y_view", ["%core_id"], [1], [cores], dt),
                  f"    ktdp.store %r, %yt : tensor<1x{dt}>, !ktdp.access_tile<1xindex>"]
    else:
        R = configs._t(list(rshape), dt)
        lines += [f"    %init = tensor.splat %iv : {R}",
                  f"    %r = linalg.reduce{head} ins(%x : {T}) outs(%init : {R}) dimensions = {list(dims)}{tail}",
                  _core_tile("yt", "y_view", rshape, rfull, dt, row="%orow0"),
                  f"    ktdp.store %r, %yt : {R}, !ktdp.access_tile<{'x'.join(map(str, rshape))}xindex>"]
    src = (f"module {{\n  func.func @reduce_kernel(%x_ptr: index, %y_ptr: index) attributes {{grid = [{cores}, 1]}} {{\n"
           + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "reduce_kernel", full, rfull


def _cstr(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= s
    return tuple(reversed(st))


def generic_contraction(M=3, N=4, K=5, dt="f32", cores=2, combiner="arith.addf"):
    """C = A @ B + C0 written as a linalg.generic with a reduction iterator
    (the reference's tests/test_dialects_exec.py:1222-1277 contraction), one
    (M, K) @ (K, N) block per core."""
    a_full, b_full, c_full = (M * cores, K), (K * cores, N), (M * cores, N)
    TA, TB, TC = (configs._t(list(s), dt) for s in ((M, K), (K, N), (M, N)))
    mul = "arith.mulf" if dt.startswith(("f", "b")) else "arith.muli"
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %cm = arith.constant {M} : index", f"    %ck = arith.constant {K} : index",
             "    %am = arith.muli %core_id, %cm : index", "    %bk = arith.muli %core_id, %ck : index",
             configs._view("a_view", "a_ptr", list(a_full), [K, 1], dt),
             configs._view("b_view", "b_ptr", list(b_full), [N, 1], dt),
             configs._view("c_view", "c_ptr", list(c_full), [N, 1], dt),
             configs._tile("at", "a_view", ["%am", "%c0"], [M, K], list(a_full), dt),
             configs._tile("bt", "b_view", ["%bk", "%c0"], [K, N], list(b_full), dt),
             configs._tile("ct", "c_view", ["%am", "%c0"], [M, N], list(c_full), dt),
             f"    %a = ktdp.load %at : !ktdp.access_tile<{M}x{K}xindex> -> {TA}",
             f"    %b = ktdp.load %bt : !ktdp.access_tile<{K}x{N}xindex> -> {TB}",
             f"    %c = ktdp.load %ct : !ktdp.access_tile<{M}x{N}xindex> -> {TC}",
             "    %r = linalg.generic {indexing_maps = [affine_map<(d0, d1, d2) -> (d0, d2)>, "
             "affine_map<(d0, d1, d2) -> (d2, d1)>, affine_map<(d0, d1, d2) -> (d0, d1)>],",
             '                         iterator_types = ["parallel", "parallel", "reduction"]}',
             f"        ins(%a, %b : {TA}, {TB}) outs(%c : {TC}) {{",
             f"      ^bb0(%aa: {dt}, %bb: {dt}, %cc: {dt}):",
             f"        %mul = {mul} %aa, %bb : {dt}",
             f"        %acc = {combiner} %mul, %cc : {dt}",
             f"        linalg.yield %acc : {dt}",
             f"    }} -> {TC}",
             f"    ktdp.store %r, %ct : {TC}, !ktdp.access_tile<{M}x{N}xindex>"]
    src = (f"module {{\n  func.func @generic_red(%a_ptr: index, %b_ptr: index, %c_ptr: index) "
           f"attributes {{grid = [{cores}, 1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "generic_red", a_full, b_full, c_full


def generic_stick_contraction(cores=2):
    """The stickified contraction of the reference's issue-174 test
    (tests/test_dialects_exec.py:1279-1330): iteration (d0..d4) = (n_stick 1,
    m 4, k_stick 2, k_elem 4, n_elem 4), reductions over d2 and d3, A read
    through a permuted map (d2, d1, d3) and W through the computed map
    (d0, d2 * 4 + d3, d4).  One block per core."""
    a_s, w_s, c_s = (2, 4, 4), (1, 8, 4), (1, 4, 4)
    full = {k: (s[0] * cores,) + s[1:] for k, s in (("a", a_s), ("w", w_s), ("c", c_s))}
    T = {k: configs._t(list(s), "f32") for k, s in (("a", a_s), ("w", w_s), ("c", c_s))}
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index", "    %c1 = arith.constant 1 : index",
             "    %c2 = arith.constant 2 : index",
             "    %r2 = arith.muli %core_id, %c2 : index"]
    for k, s, r in (("a", a_s, "%r2"), ("w", w_s, "%core_id"), ("c", c_s, "%core_id")):
        lines.append(configs._view(f"{k}_view", f"{k}_ptr", list(full[k]), list(_cstr(full[k])), "f32"))
        lines.append(configs._tile(f"{k}t", f"{k}_view", [r, "%c0", "%c0"], list(s), list(full[k]), "f32"))
        lines.append(f"    %{k} = ktdp.load %{k}t : !ktdp.access_tile<{'x'.join(map(str, s))}xindex> -> {T[k]}")
    lines += ["    %r = linalg.generic {indexing_maps = [affine_map<(d0, d1, d2, d3, d4) -> (d2, d1, d3)>, "
              "affine_map<(d0, d1, d2, d3, d4) -> (d0, d2 * 4 + d3, d4)>, "
              "affine_map<(d0, d1, d2, d3, d4) -> (d0, d1, d4)>],",
              '                         iterator_types = ["parallel", "parallel", "reduction", "reduction", '
              '"parallel"]}',
              f"        ins(%a, %w : {T['a']}, {T['w']}) outs(%c : {T['c']}) {{",
              "      ^bb0(%aa: f32, %ww: f32, %cc: f32):",
              "        %mul = arith.mulf %aa, %ww : f32",
              "        %acc = arith.addf %mul, %cc : f32",
              "        linalg.yield %acc : f32",
              f"    }} -> {T['c']}",
              f"    ktdp.store %r, %ct : {T['c']}, !ktdp.access_tile<1x4x4xindex>"]
    src = (f"module {{\n  func.func @stick_red(%a_ptr: index, %w_ptr: index, %c_ptr: index) "
           f"attributes {{grid = [{cores}, 1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "stick_red", full


def batch_matmul(Bt=3, M=16, N=32, K=64, dt="f16", out_dt="f32", cores=2):
    """C = C0 + A @ B per batch with linalg.batch_matmul, one (Bt, M, K) x
    (Bt, K, N) block per core (blocks stacked on the batch axis)."""
    a_full, b_full, c_full = (Bt * cores, M, K), (Bt * cores, K, N), (Bt * cores, M, N)
    TA, TB = configs._t([Bt, M, K], dt), configs._t([Bt, K, N], dt)
    TC = configs._t([Bt, M, N], out_dt)
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %cb = arith.constant {Bt} : index",
             "    %b0 = arith.muli %core_id, %cb : index",
             configs._view("a_view", "a_ptr", list(a_full), list(_cstr(a_full)), dt),
             configs._view("b_view", "b_ptr", list(b_full), list(_cstr(b_full)), dt),
             configs._view("c_view", "c_ptr", list(c_full), list(_cstr(c_full)), out_dt),
             configs._tile("at", "a_view", ["%b0", "%c0", "%c0"], [Bt, M, K], list(a_full), dt),
             configs._tile("bt", "b_view", ["%b0", "%c0", "%c0"], [Bt, K, N], list(b_full), dt),
             configs._tile("ct", "c_view", ["%b0", "%c0", "%c0"], [Bt, M, N], list(c_full), out_dt),
             f"    %a = ktdp.load %at : !ktdp.access_tile<{Bt}x{M}x{K}xindex> -> {TA}",
             f"    %b = ktdp.load %bt : !ktdp.access_tile<{Bt}x{K}x{N}xindex> -> {TB}",
             f"    %c = ktdp.load %ct : !ktdp.access_tile<{Bt}x{M}x{N}xindex> -> {TC}",
             f"    %r = linalg.batch_matmul ins(%a, %b : {TA}, {TB}) outs(%c : {TC}) -> {TC}",
             f"    ktdp.store %r, %ct : {TC}, !ktdp.access_tile<{Bt}x{M}x{N}xindex>"]
    src = (f"module {{\n  func.func @bmm(%a_ptr: index, %b_ptr: index, %c_ptr: index) "
           f"attributes {{grid = [{cores}, 1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "bmm", a_full, b_full, c_full


# ---------------------------------------------------------------------------
# general indirect path: direct_expr subscripts, a permuted
# variables_space_order, its error paths
# ---------------------------------------------------------------------------

def _box2(m, k):
    return f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {m - 1} >= 0, d1 >= 0, -d1 + {k - 1} >= 0)>"


def iat_direct_expr(cores=2, rows=64, cols=128, E=4, M=60):
    """Y[e, m] = X[IDX[e], 2 m + 1] (the reference's direct_expr case,
    tests/test_blocked_indirect_fast_path.py:360-391), E index rows per core."""
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %ce = arith.constant {E} : index",
             "    %e0 = arith.muli %core_id, %ce : index",
             configs._view("x_view", "x_ptr", [rows, cols], [cols, 1], "f16"),
             configs._view("i_view", "i_ptr", [E * cores], [1], "i32"),
             configs._view("y_view", "y_ptr", [E * cores, M], [M, 1], "f16"),
             "    %g = ktdp.construct_indirect_access_tile intermediate_variables(%e, %m)",
             "        %x_view[ind(%i_view[%e0 + %e]), (2 * %m + 1)] {",
             f"      variables_space_set = {_box2(E, M)},",
             "      variables_space_order = affine_map<(d0, d1) -> (d0, d1)>",
             f"    }} : memref<{rows}x{cols}xf16>, memref<{E * cores}xi32> -> !ktdp.access_tile<{E}x{M}xindex>",
             f"    %v = ktdp.load %g : !ktdp.access_tile<{E}x{M}xindex> -> tensor<{E}x{M}xf16>",
             configs._tile("yt", "y_view", ["%e0", "%c0"], [E, M], [E * cores, M], "f16"),
             f"    ktdp.store %v, %yt : tensor<{E}x{M}xf16>, !ktdp.access_tile<{E}x{M}xindex>"]
    src = (f"module {{\n  func.func @iat_expr(%x_ptr: index, %i_ptr: index, %y_ptr: index) "
           f"attributes {{grid = [{cores}, 1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "iat_expr"


def iat_permuted(M=4, K=8, rows=16, cols=16, cores=2, scatter=False, vso="(d1, d0)", store_shape=None):
    """Two-index gather (or scatter) Y[m, k] <-> X[I1[m, k], I2[m, k]] over an
    M x K variable space visited in the order of `vso` (a permutation of
    (d0, d1)); each core uses its own M rows of I1 / I2 / Y.  A scatter
    stores Y's tile (of `store_shape`, default M x K) through the IAT."""
    ss = store_shape or (M, K)
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %cm = arith.constant {M} : index",
             "    %m0 = arith.muli %core_id, %cm : index",
             configs._view("x_view", "x_ptr", [rows, cols], [cols, 1], "f16"),
             configs._view("i1_view", "i1_ptr", [M * cores, K], [K, 1], "i32"),
             configs._view("i2_view", "i2_ptr", [M * cores, K], [K, 1], "i32"),
             configs._view("y_view", "y_ptr", [M * cores, K], [K, 1], "f16"),
             "    %g = ktdp.construct_indirect_access_tile intermediate_variables(%m, %k)",
             "        %x_view[ind(%i1_view[%m0 + %m, %k]), ind(%i2_view[%m0 + %m, %k])] {",
             f"      variables_space_set = {_box2(M, K)},",
             f"      variables_space_order = affine_map<(d0, d1) -> {vso}>",
             f"    }} : memref<{rows}x{cols}xf16>, memref<{M * cores}x{K}xi32>, memref<{M * cores}x{K}xi32> "
             f"-> !ktdp.access_tile<{M}x{K}xindex>"]
    yt = configs._tile("yt", "y_view", ["%m0", "%c0"], [M, K], [M * cores, K], "f16")
    if scatter:
        T = configs._t(list(ss), "f16")
        lines += [yt, f"    %v0 = ktdp.load %yt : !ktdp.access_tile<{M}x{K}xindex> -> {configs._t([M, K], 'f16')}"]
        if tuple(ss) != (M, K):
            lines.append(f"    %v = tensor.collapse_shape %v0 [[0, 1]] : {configs._t([M, K], 'f16')} into "
                         f"{configs._t([M * K], 'f16')}")
            T = configs._t([M * K], "f16")
        else:
            lines.append(f"    %v = arith.addf %v0, %v0 : {T}")
        lines.append(f"    ktdp.store %v, %g : {T}, !ktdp.access_tile<{M}x{K}xindex>")
    else:
        lines += [f"    %v = ktdp.load %g : !ktdp.access_tile<{M}x{K}xindex> -> tensor<{M}x{K}xf16>", yt,
                  f"    ktdp.store %v, %yt : tensor<{M}x{K}xf16>, !ktdp.access_tile<{M}x{K}xindex>"]
    src = (f"module {{\n  func.func @iat_perm(%x_ptr: index, %i1_ptr: index, %i2_ptr: index, %y_ptr: index) "
           f"attributes {{grid = [{cores}, 1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "iat_perm"


# ---------------------------------------------------------------------------
# memory views with SSA sizes / strides and symbolic coordinate sets
# ---------------------------------------------------------------------------

def dyn_vector_add(block=1024, cores=1, dt="f32"):
    """out = x + y over views whose size is the i32 argument n (a symbolic
    coordinate set bound to it), with a fixed `block`-element access tile per
    core: positions past the n-element allocations read zero and their
    writes are dropped (after examples/triton-ktir/vector_add_dynamic_ktir.mlir)."""
    T = configs._t([block], dt)
    view = lambda name, ptr: (f"    %{name} = ktdp.construct_memory_view %{ptr}, sizes: [%n], strides: [1] {{\n"
                              f"      coordinate_set = affine_set<(d0)[s0] : (d0 >= 0, -d0 + s0 - 1 >= 0)>, "
                              f"memory_space = #ktdp.memory_space<global>\n    }} : memref<?x{dt}>")
    tile = lambda name, v: (f"    %{name} = ktdp.construct_access_tile %{v}[%off] {{\n"
                            f"      access_tile_set = affine_set<(d0) : (d0 >= 0, -d0 + {block - 1} >= 0)>,\n"
                            f"      access_tile_order = affine_map<(d0) -> (d0)>\n"
                            f"    }} : memref<?x{dt}> -> !ktdp.access_tile<{block}xindex>")
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             f"    %cb = arith.constant {block} : index",
             "    %off = arith.muli %core_id, %cb : index",
             "    %n = arith.index_cast %n_elements : i32 to index",
             view("x_view", "x_ptr"), view("y_view", "y_ptr"), view("o_view", "out_ptr"),
             tile("xt", "x_view"), tile("yt", "y_view"), tile("ot", "o_view"),
             f"    %x = ktdp.load %xt : !ktdp.access_tile<{block}xindex> -> {T}",
             f"    %y = ktdp.load %yt : !ktdp.access_tile<{block}xindex> -> {T}",
             f"    %o = arith.addf %x, %y : {T}",
             f"    ktdp.store %o, %ot : {T}, !ktdp.access_tile<{block}xindex>"]
    src = (f"module {{\n  func.func @add_dyn(%x_ptr: index, %y_ptr: index, %out_ptr: index, %n_elements: i32) "
           f"attributes {{grid = [{cores}, 1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "add_dyn"


def dyn_distributed_copy(rows=64, tile_cols=32, merge_rows=False):
    """B = A where A is two partitions with a symbolic column extent s0 (an
    i32 argument) and SSA row strides, composed into one distributed view;
    B's view has SSA size and stride 2 s0 (or, with merge_rows, the two
    partitions split the rows and share the symbolic columns).  A loop
    with an SSA trip count walks rows x tile_cols tiles across the global
    domain (after examples/rfc/distributed-view-copy-dynamic.mlir)."""
    if merge_rows:
        p0 = f"affine_set<(d0, d1)[s0] : (d0 >= 0, -d0 + {rows - 1} >= 0, d1 >= 0, -d1 + s0 - 1 >= 0)>"
        p1 = (f"affine_set<(d0, d1)[s0] : (d0 - {rows} >= 0, -d0 + {2 * rows - 1} >= 0, d1 >= 0, "
              f"-d1 + s0 - 1 >= 0)>")
        bset = f"affine_set<(d0, d1)[s0] : (d0 >= 0, -d0 + {2 * rows - 1} >= 0, d1 >= 0, -d1 + s0 - 1 >= 0)>"
        grows, bsize, bstride, ub, row_tiles = 2 * rows, f"[{2 * rows}, %s0]", "[%s0, 1]", "%s0", 2
    else:
        p0 = f"affine_set<(d0, d1)[s0] : (d0 >= 0, -d0 + {rows - 1} >= 0, d1 >= 0, -d1 + s0 - 1 >= 0)>"
        p1 = f"affine_set<(d0, d1)[s0] : (d0 >= 0, -d0 + {rows - 1} >= 0, d1 - s0 >= 0, -d1 + 2*s0 - 1 >= 0)>"
        bset = f"affine_set<(d0, d1)[s0] : (d0 >= 0, -d0 + {rows - 1} >= 0, d1 >= 0, -d1 + s0 - 1 >= 0)>"
        grows, bsize, bstride, ub, row_tiles = rows, "[%s0x2]", "[%s0x2, 1]", "%s0x2", 1
    tset = f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {rows - 1} >= 0, d1 >= 0, -d1 + {tile_cols - 1} >= 0)>"
    mt = f"memref<{rows}x?xf16>"
    gt = f"memref<{grows}x?xf16>"
    bs = f"[{rows}, %s0x2]" if not merge_rows else f"[{2 * rows}, %s0]"
    lines = ["    %c0 = arith.constant 0 : index", "    %c1 = arith.constant 1 : index",
             "    %c2 = arith.constant 2 : index", f"    %ct = arith.constant {tile_cols} : index",
             f"    %crows = arith.constant {rows} : index",
             "    %s0 = arith.index_cast %s0_in : i32 to index",
             "    %s0x2 = arith.muli %s0, %c2 : index",
             f"    %a0 = ktdp.construct_memory_view %a0_ptr, sizes: [{rows}, %s0], strides: [%s0, 1] {{",
             f"      coordinate_set = {p0}, memory_space = #ktdp.memory_space<global>", f"    }} : {mt}",
             f"    %a1 = ktdp.construct_memory_view %a1_ptr, sizes: [{rows}, %s0], strides: [%s0, 1] {{",
             f"      coordinate_set = {p1}, memory_space = #ktdp.memory_space<global>", f"    }} : {mt}",
             f"    %a = ktdp.construct_distributed_memory_view (%a0, %a1 : {mt}, {mt}) : {gt}",
             f"    %b = ktdp.construct_memory_view %b_ptr, sizes: {bs}, strides: {bstride if merge_rows else '[%s0x2, 1]'} {{",
             f"      coordinate_set = {bset}, memory_space = #ktdp.memory_space<global>", f"    }} : {gt}",
             f"    scf.for %r = %c0 to %c{row_tiles} step %c1 {{" if merge_rows else "    scf.for %r = %c0 to %c1 step %c1 {",
             "      %roff = arith.muli %r, %crows : index",
             f"      scf.for %off = %c0 to {ub} step %ct {{",
             "        %at = ktdp.construct_access_tile %a[%roff, %off] {",
             f"          access_tile_set = {tset}, access_tile_order = affine_map<(d0, d1) -> (d0, d1)>",
             f"        }} : {gt} -> !ktdp.access_tile<{rows}x{tile_cols}xindex>",
             "        %bt = ktdp.construct_access_tile %b[%roff, %off] {",
             f"          access_tile_set = {tset}, access_tile_order = affine_map<(d0, d1) -> (d0, d1)>",
             f"        }} : {gt} -> !ktdp.access_tile<{rows}x{tile_cols}xindex>",
             f"        %d = ktdp.load %at : !ktdp.access_tile<{rows}x{tile_cols}xindex> -> tensor<{rows}x{tile_cols}xf16>",
             f"        ktdp.store %d, %bt : tensor<{rows}x{tile_cols}xf16>, !ktdp.access_tile<{rows}x{tile_cols}xindex>",
             "      }", "    }"]
    if merge_rows:
        lines.insert(0, "    %c2r = arith.constant 2 : index")
        lines = [ln.replace("%c2 step %c1", "%c2r step %c1") for ln in lines]
    src = (f"module {{\n  func.func @dyn_copy(%a0_ptr: index, %a1_ptr: index, %b_ptr: index, %s0_in: i32) "
           f"attributes {{grid = [1]}} {{\n" + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "dyn_copy"


# ---------------------------------------------------------------------------
# tensor.extract_slice / insert_slice / generate / from_elements / reshape
# ---------------------------------------------------------------------------

def tensor_ops(cores=4, R=4, C=16):
    """Each core loads its R x C f32 block X of x and stores:
    a = X[1:3, 2:10] (extract_slice, static);
    b = X[k, 1:14:3] (extract_slice, dynamic row k = core mod R, stride 3,
        rank-reduced to 5 elements);
    c = zeros with a inserted at [2, k2 : k2 + 8] (insert_slice, dynamic
        column k2 = 2 (core mod 4));
    g = (i >= j) as f16 over R x C (tensor.generate yielding cmpi);
    r = X reshaped to (R C / 32) x 32 through a from_elements shape tensor."""
    T = configs._t([R, C], "f32")
    rr = R * C // 32
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %cR = arith.constant {R} : index",
             "    %c2 = arith.constant 2 : index", "    %c4 = arith.constant 4 : index",
             f"    %crr = arith.constant {rr} : index", "    %c32 = arith.constant 32 : index",
             "    %row0 = arith.muli %core_id, %cR : index",
             "    %k = arith.remui %core_id, %cR : index",
             "    %m4 = arith.remui %core_id, %c4 : index",
             "    %k2 = arith.muli %m4, %c2 : index",
             "    %zero = arith.constant 0.0 : f32"]
    outs = {"x": ([R * cores, C], "f32"), "a": ([2 * cores, 8], "f32"), "b": ([5 * cores], "f32"),
            "c": ([R * cores, C], "f32"), "g": ([R * cores, C], "f16"), "r": ([rr * cores, 32], "f32")}
    for n, (shape, dt) in outs.items():
        lines.append(configs._view(f"{n}_view", f"{n}_ptr", shape, list(_cstr(shape)), dt))
    lines += [configs._tile("xt", "x_view", ["%row0", "%c0"], [R, C], [R * cores, C], "f32"),
              f"    %x = ktdp.load %xt : !ktdp.access_tile<{R}x{C}xindex> -> {T}",
              f"    %a = tensor.extract_slice %x[1, 2] [2, 8] [1, 1] : {T} to tensor<2x8xf32>",
              f"    %b = tensor.extract_slice %x[%k, 1] [1, 5] [1, 3] : {T} to tensor<5xf32>",
              f"    %z = tensor.splat %zero : {T}",
              f"    %c = tensor.insert_slice %a into %z[2, %k2] [2, 8] [1, 1] : tensor<2x8xf32> into {T}",
              "    %g = tensor.generate {",
              "    ^bb0(%i: index, %j: index):",
              "      %cmp = arith.cmpi sge, %i, %j : index",
              "      tensor.yield %cmp : i1",
              f"    }} : tensor<{R}x{C}xf16>",
              "    %shape = tensor.from_elements %crr, %c32 : tensor<2xindex>",
              f"    %r = tensor.reshape %x(%shape) : ({T}, tensor<2xindex>) -> tensor<{rr}x32xf32>",
              "    %a0 = arith.muli %core_id, %c2 : index",
              "    %c5 = arith.constant 5 : index",
              "    %b0 = arith.muli %core_id, %c5 : index",
              "    %r0 = arith.muli %core_id, %crr : index",
              configs._tile("at", "a_view", ["%a0", "%c0"], [2, 8], [2 * cores, 8], "f32"),
              configs._tile("bt", "b_view", ["%b0"], [5], [5 * cores], "f32"),
              configs._tile("ct", "c_view", ["%row0", "%c0"], [R, C], [R * cores, C], "f32"),
              configs._tile("gt", "g_view", ["%row0", "%c0"], [R, C], [R * cores, C], "f16"),
              configs._tile("rt", "r_view", ["%r0", "%c0"], [rr, 32], [rr * cores, 32], "f32"),
              "    ktdp.store %a, %at : tensor<2x8xf32>, !ktdp.access_tile<2x8xindex>",
              "    ktdp.store %b, %bt : tensor<5xf32>, !ktdp.access_tile<5xindex>",
              f"    ktdp.store %c, %ct : {T}, !ktdp.access_tile<{R}x{C}xindex>",
              f"    ktdp.store %g, %gt : tensor<{R}x{C}xf16>, !ktdp.access_tile<{R}x{C}xindex>",
              f"    ktdp.store %r, %rt : tensor<{rr}x32xf32>, !ktdp.access_tile<{rr}x32xindex>"]
    args = ", ".join(f"%{n}_ptr: index" for n in outs)
    src = (f"module {{\n  func.func @tensor_ops({args}) attributes {{grid = [{cores}, 1]}} {{\n"
           + "\n".join(lines) + "\n    return\n  }\n}\n")
    rng = np.random.default_rng(17)
    kw = {f"{n}_ptr": (rng.standard_normal(shape).astype(np.float32) if n == "x"
              else np.zeros(shape, np.float16 if dt == "f16" else np.float32)) for n, (shape, dt) in outs.items()}
    return src, "tensor_ops", kw


# ---------------------------------------------------------------------------
# scalars read from tile data (tensor.extract, reductions over every axis)
# ---------------------------------------------------------------------------

def scalar_chain(body, dt="f32", out_dt="f32", cores=4, C=16, idx="%c0", fill=False):
    """Each core loads row `core_id` of x (cores x C, `dt`) and reads three
    scalars from it: %s = x[core, idx] and %t = x[core, C - 1]
    (tensor.extract: NumPy scalars of the tile's type) and %u, the sum of
    the row (linalg.reduce over every axis into a 0-d outs: a Python
    float); %v is the same sum reduced into a tensor<1x..> outs, which the
    reference holds as a one-element tile.  `body`
    ({dt} is replaced by `dt`) computes the scalar %r, which tensor.splat
    (linalg.fill with `fill`) spreads over the core's row of y (cores x C,
    `out_dt`); a body that defines the tile %rb itself stores that."""
    T, O = configs._t([1, C], dt), configs._t([1, C], out_dt)
    at = f"!ktdp.access_tile<1x{C}xindex>"
    lines = ["    %core_id = ktdp.get_compute_tile_id : index",
             "    %c0 = arith.constant 0 : index",
             f"    %cC = arith.constant {C} : index",
             f"    %cl = arith.constant {C - 1} : index",
             "    %i_core = arith.remui %core_id, %cC : index",
             configs._view("x_view", "x_ptr", [cores, C], [C, 1], dt),
             configs._view("y_view", "y_ptr", [cores, C], [C, 1], out_dt),
             configs._tile("xt", "x_view", ["%core_id", "%c0"], [1, C], [cores, C], dt),
             f"    %x = ktdp.load %xt : {at} -> {T}",
             f"    %s = tensor.extract %x[%c0, {idx}] : {T}",
             f"    %t = tensor.extract %x[%c0, %cl] : {T}",
             f"    %z = arith.constant 0.0 : {dt}",
             f"    %u_e = tensor.empty() : tensor<{dt}>",
             f"    %u_init = linalg.fill ins(%z : {dt}) outs(%u_e : tensor<{dt}>) -> tensor<{dt}>",
             f"    %u = linalg.reduce {{ arith.addf }} ins(%x : {T}) outs(%u_init : tensor<{dt}>)",
             f"    %v_init = tensor.splat %z : tensor<1x{dt}>",
             f"    %v = linalg.reduce {{ arith.addf }} ins(%x : {T}) outs(%v_init : tensor<1x{dt}>)",
             body.replace("{dt}", dt)]
    if "%rb =" not in body:
        if fill:
            lines += [f"    %e = tensor.empty() : {O}",
                      f"    %rb = linalg.fill ins(%r : {dt}) outs(%e : {O}) -> {O}"]
        else:
            lines.append(f"    %rb = tensor.splat %r : {O}")
    lines += [configs._tile("yt", "y_view", ["%core_id", "%c0"], [1, C], [cores, C], out_dt),
              f"    ktdp.store %rb, %yt : {O}, {at}"]
    src = (f"module {{\n  func.func @scalar_chain(%x_ptr: index, %y_ptr: index) attributes {{grid = [{cores}, 1]}} {{\n"
           + "\n".join(lines) + "\n    return\n  }\n}\n")
    return src, "scalar_chain"


# ---------------------------------------------------------------------------
# indirect forms of the reference's examples (pointer arguments and sizes of
# our choosing; the structure of examples/triton-ktir/indexed_add.mlir,
# examples/rfc/paged-tensor-copy.mlir, paged-tensor-write.mlir, and the
# X[IDX[e], m, n] / page-table gathers of the reference's
# tests/test_blocked_indirect_fast_path.py:234-360)
# ---------------------------------------------------------------------------

def _vsets(shape):
    dims = ", ".join(f"d{i}" for i in range(len(shape)))
    cons = ", ".join(f"d{i} >= 0, -d{i} + {s - 1} >= 0" for i, s in enumerate(shape))
    return f"affine_set<({dims}) : ({cons})>", f"affine_map<({dims}) -> ({dims})>"


def indexed_add(rows=16, d1=64, heads=8, D=128, width=32, seed=0, index=(3, 7), dim1_start=5):
    """out[g0, :, g1, :] = x[index[g0], s : s + width, g1, :] + y[g0, :, g1, :]
    (f16) with an i64 index tensor, grid [len(index), heads]: the x tile is an
    indirect access tile whose other subscripts are SSA + variable
    expressions (dim1_start + d1, g1 + d2)."""
    G0 = len(index)
    xs, ys = [rows, d1, heads, D], [G0, width, heads, D]
    st = lambda sh: [int(np.prod(sh[i + 1:])) for i in range(len(sh))]
    at4 = f"!ktdp.access_tile<1x{width}x1x{D}xindex>"
    T4 = configs._t([1, width, 1, D], "f16")
    vss, vso = _vsets([1, width, 1, D])
    src = f"""module {{
  func.func @indexed_add_kernel(%x_ptr: index, %y_ptr: index, %index_ptr: index, %output_ptr: index,
      %dim1_start: index) attributes {{grid = [{G0}, {heads}]}} {{
    %g0, %g1 = ktdp.get_compute_tile_id : index, index
    %c0 = arith.constant 0 : index
{configs._view("i_view", "index_ptr", [G0], [1], "i64")}
{configs._view("x_view", "x_ptr", xs, st(xs), "f16")}
{configs._view("y_view", "y_ptr", ys, st(ys), "f16")}
{configs._view("o_view", "output_ptr", ys, st(ys), "f16")}
    %x_tile = ktdp.construct_indirect_access_tile intermediate_variables(%e0, %e1, %e2, %e3)
        %x_view[ind(%i_view[%g0 + %e0]), (%dim1_start + %e1), (%g1 + %e2), (%e3)] {{
      variables_space_set = {vss},
      variables_space_order = {vso}
    }} : memref<{'x'.join(map(str, xs))}xf16>, memref<{G0}xi64> -> {at4}
{configs._tile("y_tile", "y_view", ["%g0", "%c0", "%g1", "%c0"], [1, width, 1, D], ys, "f16")}
    %x = ktdp.load %x_tile : {at4} -> {T4}
    %y = ktdp.load %y_tile : {at4} -> {T4}
    %o = arith.addf %x, %y : {T4}
{configs._tile("o_tile", "o_view", ["%g0", "%c0", "%g1", "%c0"], [1, width, 1, D], ys, "f16")}
    ktdp.store %o, %o_tile : {T4}, {at4}
    return
  }}
}}
"""
    rng = np.random.default_rng(seed)
    kw = dict(x_ptr=rng.standard_normal(xs).astype(np.float16), y_ptr=rng.standard_normal(ys).astype(np.float16),
              index_ptr=np.asarray(index, np.int64), output_ptr=np.zeros(ys, np.float16), dim1_start=dim1_start)
    return src, "indexed_add_kernel", kw


def paged_tensor(write=False, Nb=2, Ntkv=256, Ptkv=64, Nhkv=4, Ndkv=64, Npages=24, seed=1, pages=None):
    """The page-table copy of examples/rfc/paged-tensor-copy.mlir (write
    False): Y[b, tkv, h, d] = X[Idx[b, tkv // Ptkv], h, tkv % Ptkv, d], the
    gather an indirect access tile whose index and direct subscripts use
    floordiv / mod of one variable, the store an access tile whose order
    permutes (b, h, tkv, d) to Y's (b, tkv, h, d) layout; or its scatter dual
    (paged-tensor-write.mlir, write True): Y[Idx[b, tkv // Ptkv], h,
    tkv % Ptkv, d] = X[b, tkv, h, d].  One core; f16; Idx i32 [Nb, Ntkv / Ptkv]."""
    npg = Ntkv // Ptkv
    paged = [Npages, Nhkv, Ptkv, Ndkv]
    flat = [Nb, Ntkv, Nhkv, Ndkv]
    st = lambda sh: [int(np.prod(sh[i + 1:])) for i in range(len(sh))]
    tile = [Nb, Nhkv, Ntkv, Ndkv]
    vss, vso = _vsets(tile)
    perm = "affine_map<(d0, d1, d2, d3) -> (d0, d2, d1, d3)>"
    at = f"!ktdp.access_tile<{'x'.join(map(str, tile))}xindex>"
    T = configs._t(tile, "f16")
    src_view, dst_view = ("X_view", "Y_view")
    iat = f"""    %P_tile = ktdp.construct_indirect_access_tile intermediate_variables(%b, %h, %t, %d)
        %{'Y' if write else 'X'}_view[ind(%I_view[%b, %t floordiv {Ptkv}]), (%h), (%t mod {Ptkv}), (%d)] {{
      variables_space_set = {vss},
      variables_space_order = {vso}
    }} : memref<{'x'.join(map(str, paged))}xf16>, memref<{Nb}x{npg}xi32> -> {at}"""
    ftile = f"""    %F_tile = ktdp.construct_access_tile %{'X' if write else 'Y'}_view[%c0, %c0, %c0, %c0] {{
      access_tile_set = {vss},
      access_tile_order = {perm}
    }} : memref<{'x'.join(map(str, flat))}xf16> -> {at}"""
    body = (f"    %v = ktdp.load %F_tile : {at} -> {T}\n    ktdp.store %v, %P_tile : {T}, {at}" if write else
            f"    %v = ktdp.load %P_tile : {at} -> {T}\n    ktdp.store %v, %F_tile : {T}, {at}")
    name = "paged_tensor_write_1core" if write else "paged_tensor_copy_1core"
    src = f"""module {{
  func.func @{name}(%x_ptr: index, %idx_ptr: index, %y_ptr: index) {{
    %c0 = arith.constant 0 : index
{configs._view("I_view", "idx_ptr", [Nb, npg], [npg, 1], "i32")}
{configs._view("X_view", "x_ptr", flat if write else paged, st(flat if write else paged), "f16")}
{configs._view("Y_view", "y_ptr", paged if write else flat, st(paged if write else flat), "f16")}
{iat}
{ftile}
{body}
    return
  }}
}}
"""
    rng = np.random.default_rng(seed)
    if pages is None:
        pages = rng.permutation(Npages)[:Nb * npg]
    idx = np.asarray(pages, np.int32).reshape(Nb, npg)
    x = rng.standard_normal(flat if write else paged).astype(np.float16)
    y = np.zeros(paged if write else flat, np.float16)
    return src, name, dict(x_ptr=x, idx_ptr=idx, y_ptr=y)


def expert_gather(E=32, M=8, N=64, sel=(0, 5, 9, 17, 22, 31), cores=2):
    """X[IDX[e], m, n] (the reference's tests/test_blocked_indirect_fast_path.py:234-258
    MoE pattern): each core gathers len(sel) // cores experts' [M, N] blocks
    of an f16 weight tensor through an i32 index tensor and stores them."""
    k = len(sel) // cores
    xs, os_ = [E, M, N], [len(sel), M, N]
    st = lambda sh: [int(np.prod(sh[i + 1:])) for i in range(len(sh))]
    vss, vso = _vsets([k, M, N])
    at = f"!ktdp.access_tile<{k}x{M}x{N}xindex>"
    T = configs._t([k, M, N], "f16")
    src = f"""module {{
  func.func @expert_gather(%x_ptr: index, %idx_ptr: index, %out_ptr: index) attributes {{grid = [{cores}, 1]}} {{
    %core = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %ck = arith.constant {k} : index
    %e0 = arith.muli %core, %ck : index
{configs._view("i_view", "idx_ptr", [len(sel)], [1], "i32")}
{configs._view("x_view", "x_ptr", xs, st(xs), "f16")}
{configs._view("o_view", "out_ptr", os_, st(os_), "f16")}
    %g = ktdp.construct_indirect_access_tile intermediate_variables(%e, %m, %n)
        %x_view[ind(%i_view[%e0 + %e]), (%m), (%n)] {{
      variables_space_set = {vss},
      variables_space_order = {vso}
    }} : memref<{E}x{M}x{N}xf16>, memref<{len(sel)}xi32> -> {at}
    %v = ktdp.load %g : {at} -> {T}
{configs._tile("o_tile", "o_view", ["%e0", "%c0", "%c0"], [k, M, N], os_, "f16")}
    ktdp.store %v, %o_tile : {T}, {at}
    return
  }}
}}
"""
    rng = np.random.default_rng(2)
    return src, "expert_gather", dict(x_ptr=rng.standard_normal(xs).astype(np.float16),
                                      idx_ptr=np.asarray(sel, np.int32), out_ptr=np.zeros(os_, np.float16))


def nested_yield(outer=2, inner=2, n=4):
    """Nested scf.for loops with iter_args (the structure of the reference's
    examples/ktir/nested_yield.ktir): the outer loop adds 1 per trip, the
    inner loop's own sum is computed and discarded; the result, stored, is
    `outer` in every element."""
    T = configs._t([n], "f32")
    src = f"""module {{
  func.func @nested_yield(%out: index) attributes {{grid = [1]}} {{
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %cI = arith.constant {outer} : index
    %cJ = arith.constant {inner} : index
    %fone = arith.constant 1.0 : f32
    %fzero = arith.constant 0.0 : f32
    %one = tensor.splat %fone : {T}
    %zero = tensor.splat %fzero : {T}
{configs._view("o_view", "out", [n], [1], "f32")}
    %sum = scf.for %i = %c0 to %cI step %c1 iter_args(%acc = %zero) -> ({T}) {{
      %next = arith.addf %acc, %one : {T}
      %inner = scf.for %j = %c0 to %cJ step %c1 iter_args(%iacc = %zero) -> ({T}) {{
        %t = arith.addf %iacc, %one : {T}
        scf.yield %t : {T}
      }}
      scf.yield %next : {T}
    }}
{configs._tile("o_tile", "o_view", ["%c0"], [n], [n], "f32")}
    ktdp.store %sum, %o_tile : {T}, !ktdp.access_tile<{n}xindex>
    return
  }}
}}
"""
    return src, "nested_yield", dict(out=np.zeros(n, np.float32))


def softmax_wide(rows=2, cols=4096, cores=1):
    """The row softmax of the reference's examples/ktir/softmax_wide.mlir:
    rows [start, min(start + chunk, R)) per core, a whole row per step in
    f16, `maxnumf` row max and sum read by tensor.extract.  At its own width
    (262144) one row's tile exceeds the 2 MiB LX scratchpad and the run
    raises the reference's overflow error."""
    chunk = -(-rows // cores)
    T = configs._t([1, cols], "f16")
    at = f"!ktdp.access_tile<1x{cols}xindex>"
    src = f"""module {{
  func.func @softmax_kernel(%output_ptr: index, %input_ptr: index) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c_chunk = arith.constant {chunk} : index
    %c_R = arith.constant {rows} : index
    %c1 = arith.constant 1 : index
    %start = arith.muli %core_id, %c_chunk : index
    %end_raw = arith.addi %start, %c_chunk : index
    %cmp = arith.cmpi slt, %end_raw, %c_R : index
    %end = arith.select %cmp, %end_raw, %c_R : index
{configs._view("in_view", "input_ptr", [rows, cols], [cols, 1], "f16")}
{configs._view("out_view", "output_ptr", [rows, cols], [cols, 1], "f16")}
    scf.for %row = %start to %end step %c1 : index {{
      %c0 = arith.constant 0 : index
{configs._tile("in_acc", "in_view", ["%row", "%c0"], [1, cols], [rows, cols], "f16", "      ")}
      %x = ktdp.load %in_acc : {at} -> {T}
      %neg_inf = arith.constant 0xFC00 : f16
      %max_init = tensor.splat %neg_inf : tensor<1xf16>
      %row_max = linalg.reduce {{ arith.maxnumf }} ins(%x : {T}) outs(%max_init : tensor<1xf16>) dimensions = [1]
      %m = tensor.extract %row_max[%c0] : tensor<1xf16>
      %mb = tensor.splat %m : {T}
      %d = arith.subf %x, %mb : {T}
      %e = math.exp %d : {T}
      %zero = arith.constant 0.0 : f16
      %sum_init = tensor.splat %zero : tensor<1xf16>
      %sum = linalg.reduce {{ arith.addf }} ins(%e : {T}) outs(%sum_init : tensor<1xf16>) dimensions = [1]
      %s = tensor.extract %sum[%c0] : tensor<1xf16>
      %sb = tensor.splat %s : {T}
      %y = arith.divf %e, %sb : {T}
{configs._tile("out_acc", "out_view", ["%row", "%c0"], [1, cols], [rows, cols], "f16", "      ")}
      ktdp.store %y, %out_acc : {T}, {at}
      scf.yield
    }}
    return
  }}
}}
"""
    rng = np.random.default_rng(5)
    return src, "softmax_kernel", dict(output_ptr=np.zeros((rows, cols), np.float16),
                                       input_ptr=rng.standard_normal((rows, cols)).astype(np.float16))


def scalar_broadcast(shape=(4, 64), dt="f16"):
    """The reference's examples/ktir/scalar_broadcast.mlir: a 1x1 tile
    collapsed to a 0-d tensor and broadcast over every dimension of the
    output (linalg.broadcast dimensions [0, 1])."""
    T = configs._t(list(shape), dt)
    src = f"""module {{
  func.func @scalar_broadcast(%in_ptr: index, %out_ptr: index) attributes {{grid = [1]}} {{
    %c0 = arith.constant 0 : index
{configs._view("in_view", "in_ptr", [1, 1], [1, 1], dt)}
{configs._tile("in_tile", "in_view", ["%c0", "%c0"], [1, 1], [1, 1], dt)}
    %in = ktdp.load %in_tile : !ktdp.access_tile<1x1xindex> -> {configs._t([1, 1], dt)}
    %s = tensor.collapse_shape %in [] : {configs._t([1, 1], dt)} into tensor<{dt}>
    %init = tensor.empty() : {T}
    %b = linalg.broadcast ins(%s : tensor<{dt}>) outs(%init : {T}) dimensions = [0, 1]
{configs._view("out_view", "out_ptr", list(shape), [shape[1], 1], dt)}
{configs._tile("out_tile", "out_view", ["%c0", "%c0"], list(shape), list(shape), dt)}
    ktdp.store %b, %out_tile : {T}, !ktdp.access_tile<{shape[0]}x{shape[1]}xindex>
    return
  }}
}}
"""
    npdt = np.float16 if dt == "f16" else np.float32
    return src, "scalar_broadcast", dict(in_ptr=np.array([[-3.25]], npdt), out_ptr=np.zeros(shape, npdt))
