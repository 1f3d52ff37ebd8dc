"""KTIR text generators for the benchmark configurations.

Each generator returns a KTIR module in the surface syntax of the reference's
examples (``examples/triton-ktir/*.mlir``) and notebook generators
(``notebooks/demo_gen_mlir.py:109-567``): memory views over pointer
arguments, access tiles indexed by core id / loop variables, ``ktdp.load`` /
``ktdp.store``, and arith/math/linalg/tensor compute on the loaded tiles.
The same text runs on the NumPy oracle and on the GPU backend.

Configurations (all shapes parameterised so tests can shrink them):

1. ``vector_add``       out = x + y, f16, BLOCK elements per block.
2. ``gather_scatter_add`` out[idx[i], :] += f32(table[idx[i], :]) through
   indirect access tiles, in chunks of CH rows per step.
3. ``softmax`` / ``rmsnorm`` row kernels, f32 row reductions;
   ``softmax_extract`` / ``rmsnorm_extract`` / ``layernorm_extract`` the
   same in the f16-math, one-row-per-step form of the reference's examples
   (row statistics read by ``tensor.extract``).
4. ``gemm``              C = A @ B, f16 in, f32 accumulate, f16 out.
5. ``flash_attention``   causal attention, bf16 in/out, online softmax over
   KV tiles with f32 state.
"""

from __future__ import annotations


def _view(name, ptr, sizes, strides, dtype, indent="    "):
    dims = ", ".join(f"d{i}" for i in range(len(sizes)))
    cons = ", ".join(f"d{i} >= 0, -d{i} + {s - 1} >= 0" for i, s in enumerate(sizes))
    mt = "x".join(str(s) for s in sizes) + "x" + dtype
    return (f"{indent}%{name} = ktdp.construct_memory_view %{ptr}, sizes: {list(sizes)}, "
            f"strides: {list(strides)} {{\n"
            f"{indent}  coordinate_set = affine_set<({dims}) : ({cons})>, "
            f"memory_space = #ktdp.memory_space<global>\n"
            f"{indent}}} : memref<{mt}>")


def _tile(name, view, idx, shape, view_shape, dtype, indent="    "):
    dims = ", ".join(f"d{i}" for i in range(len(shape)))
    cons = ", ".join(f"d{i} >= 0, -d{i} + {s - 1} >= 0" for i, s in enumerate(shape))
    vt = "x".join(str(s) for s in view_shape) + "x" + dtype
    at = "x".join(str(s) for s in shape)
    return (f"{indent}%{name} = ktdp.construct_access_tile %{view}[{', '.join(idx)}] {{\n"
            f"{indent}  access_tile_set = affine_set<({dims}) : ({cons})>,\n"
            f"{indent}  access_tile_order = affine_map<({dims}) -> ({dims})>\n"
            f"{indent}}} : memref<{vt}> -> !ktdp.access_tile<{at}xindex>")


def _t(shape, dtype):
    return "tensor<" + "x".join(str(s) for s in shape) + ("x" if shape else "") + dtype + ">"


# ---------------------------------------------------------------------------
# 1. vector_add
# ---------------------------------------------------------------------------

def vector_add(n: int = 4096, block: int = 128, cores: int = 32) -> str:
    """out[i] = x[i] + y[i]; core c owns blocks [c*bpc, (c+1)*bpc)."""
    assert n % (cores * block) == 0
    bpc = n // (cores * block)
    views = "\n".join(_view(v, p, [n], [1], "f16") for v, p in
                      (("x_view", "x_ptr"), ("y_view", "y_ptr"), ("out_view", "output_ptr")))
    ind = "      " if bpc > 1 else "    "
    body = "\n".join([
        _tile("x_tile", "x_view", ["%offset"], [block], [n], "f16", ind),
        _tile("y_tile", "y_view", ["%offset"], [block], [n], "f16", ind),
        f"{ind}%x = ktdp.load %x_tile : !ktdp.access_tile<{block}xindex> -> {_t([block], 'f16')}",
        f"{ind}%y = ktdp.load %y_tile : !ktdp.access_tile<{block}xindex> -> {_t([block], 'f16')}",
        f"{ind}%output = arith.addf %x, %y : {_t([block], 'f16')}",
        _tile("out_tile", "out_view", ["%offset"], [block], [n], "f16", ind),
        f"{ind}ktdp.store %output, %out_tile : {_t([block], 'f16')}, !ktdp.access_tile<{block}xindex>",
    ])
    if bpc == 1:
        loop = f"    %offset = arith.muli %core_id, %BLOCK_SIZE : index\n{body}\n"
    else:
        loop = (f"    %c0 = arith.constant 0 : index\n    %c1 = arith.constant 1 : index\n"
                f"    %bpc = arith.constant {bpc} : index\n"
                f"    %first = arith.muli %core_id, %bpc : index\n"
                f"    scf.for %b = %c0 to %bpc step %c1 : index {{\n"
                f"      %blk = arith.addi %first, %b : index\n"
                f"      %offset = arith.muli %blk, %BLOCK_SIZE : index\n{body}\n"
                f"      scf.yield\n    }}\n")
    return f"""module {{
  func.func @add_kernel(%x_ptr: index, %y_ptr: index, %output_ptr: index, %BLOCK_SIZE: index)
      attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
{views}
{loop}    return
  }}
}}
"""


def vector_copy(n: int = 1 << 26, block: int = 32768, cores: int = 2048, dtype: str = "f32") -> str:
    """out[i] = x[i]: a plain copy of known size (HBM traffic calibration)."""
    assert n % (cores * block) == 0 and n // (cores * block) == 1
    at = f"!ktdp.access_tile<{block}xindex>"
    return f"""module {{
  func.func @copy_kernel(%x_ptr: index, %output_ptr: index)
      attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %BLOCK = arith.constant {block} : index
{_view("x_view", "x_ptr", [n], [1], dtype)}
{_view("out_view", "output_ptr", [n], [1], dtype)}
    %offset = arith.muli %core_id, %BLOCK : index
{_tile("x_tile", "x_view", ["%offset"], [block], [n], dtype)}
    %x = ktdp.load %x_tile : {at} -> {_t([block], dtype)}
{_tile("out_tile", "out_view", ["%offset"], [block], [n], dtype)}
    ktdp.store %x, %out_tile : {_t([block], dtype)}, {at}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# 2. indirect gather + scatter-add
# ---------------------------------------------------------------------------

def gather_scatter_add(rows: int = 1 << 20, dim: int = 128, n_idx: int = 262144,
                       cores: int = 64, chunk: int = 128) -> str:
    """For each index i (core-major, chunk by chunk):
    ``g = table[idx[i], :]`` (f16), ``o = out[idx[i], :]`` (f32),
    ``out[idx[i], :] = o + extf(g)`` — a load/add/store through the same
    indirect access tile, so duplicates inside one chunk keep the last
    writer and duplicates across chunks/cores accumulate in order.
    """
    per_core = n_idx // cores
    assert per_core * cores == n_idx and per_core % chunk == 0
    nch = per_core // chunk
    vss = (f"affine_set<(d0, d1) : (d0 >= 0, -d0 + {chunk - 1} >= 0, "
           f"d1 >= 0, -d1 + {dim - 1} >= 0)>")
    vso = "affine_map<(d0, d1) -> (d0, d1)>"

    def iat(name, view, dtype):
        return (f"      %{name} = ktdp.construct_indirect_access_tile intermediate_variables(%r, %c)\n"
                f"          %{view}[ind(%idx_view[%row0 + %r]), (%c)] {{\n"
                f"        variables_space_set = {vss},\n"
                f"        variables_space_order = {vso}\n"
                f"      }} : memref<{rows}x{dim}x{dtype}>, memref<{n_idx}xi32> "
                f"-> !ktdp.access_tile<{chunk}x{dim}xindex>")

    return f"""module {{
  func.func @gather_scatter_add(%table_ptr: index, %idx_ptr: index, %out_ptr: index)
      attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %nch = arith.constant {nch} : index
    %per_core = arith.constant {per_core} : index
    %chunk = arith.constant {chunk} : index
{_view("table_view", "table_ptr", [rows, dim], [dim, 1], "f16")}
{_view("idx_view", "idx_ptr", [n_idx], [1], "i32")}
{_view("out_view", "out_ptr", [rows, dim], [dim, 1], "f32")}
    %core_base = arith.muli %core_id, %per_core : index
    scf.for %ch = %c0 to %nch step %c1 : index {{
      %ch_off = arith.muli %ch, %chunk : index
      %row0 = arith.addi %core_base, %ch_off : index
{iat("g_tile", "table_view", "f16")}
{iat("o_tile", "out_view", "f32")}
      %g = ktdp.load %g_tile : !ktdp.access_tile<{chunk}x{dim}xindex> -> {_t([chunk, dim], 'f16')}
      %o = ktdp.load %o_tile : !ktdp.access_tile<{chunk}x{dim}xindex> -> {_t([chunk, dim], 'f32')}
      %g32 = arith.extf %g : {_t([chunk, dim], 'f16')} to {_t([chunk, dim], 'f32')}
      %sum = arith.addf %o, %g32 : {_t([chunk, dim], 'f32')}
      ktdp.store %sum, %o_tile : {_t([chunk, dim], 'f32')}, !ktdp.access_tile<{chunk}x{dim}xindex>
      scf.yield
    }}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# 3. row softmax and RMSNorm
# ---------------------------------------------------------------------------

def _row_header(fn, args, rows, cols, cores, rows_per_core):
    return (f"  func.func @{fn}({args})\n      attributes {{grid = [{cores}, 1]}} {{\n"
            f"    %core_id = ktdp.get_compute_tile_id : index\n"
            f"    %c0 = arith.constant 0 : index\n"
            f"    %rpc = arith.constant {rows_per_core} : index\n"
            f"    %row_base = arith.muli %core_id, %rpc : index\n")


def softmax(rows: int = 32768, cols: int = 4096, cores: int = 512, rblk: int = 8, dt: str = "f16") -> str:
    """y = softmax(x) per row: f32 max, exp, f32 sum, divide, round to `dt` (f16 or bf16)."""
    rpc = rows // cores
    assert rpc * cores == rows and rpc % rblk == 0
    T16, T32, V32 = _t([rblk, cols], dt), _t([rblk, cols], "f32"), _t([rblk], "f32")
    return f"""module {{
{_row_header("softmax_kernel", "%x_ptr: index, %y_ptr: index", rows, cols, cores, rpc)}
    %step = arith.constant {rblk} : index
{_view("x_view", "x_ptr", [rows, cols], [cols, 1], dt)}
{_view("y_view", "y_ptr", [rows, cols], [cols, 1], dt)}
    %neg_inf = arith.constant 0xFF800000 : f32
    %zero = arith.constant 0.0 : f32
    scf.for %r = %c0 to %rpc step %step : index {{
      %row = arith.addi %row_base, %r : index
{_tile("x_acc", "x_view", ["%row", "%c0"], [rblk, cols], [rows, cols], dt, "      ")}
      %x = ktdp.load %x_acc : !ktdp.access_tile<{rblk}x{cols}xindex> -> {T16}
      %xf = arith.extf %x : {T16} to {T32}
      %max_init = tensor.splat %neg_inf : {V32}
      %mx = linalg.reduce {{ arith.maximumf }} ins(%xf : {T32}) outs(%max_init : {V32}) dimensions = [1]
      %mxb_init = tensor.empty() : {T32}
      %mxb = linalg.broadcast ins(%mx : {V32}) outs(%mxb_init : {T32}) dimensions = [1]
      %d = arith.subf %xf, %mxb : {T32}
      %e = math.exp %d : {T32}
      %sum_init = tensor.splat %zero : {V32}
      %s = linalg.reduce {{ arith.addf }} ins(%e : {T32}) outs(%sum_init : {V32}) dimensions = [1]
      %sb_init = tensor.empty() : {T32}
      %sb = linalg.broadcast ins(%s : {V32}) outs(%sb_init : {T32}) dimensions = [1]
      %p = arith.divf %e, %sb : {T32}
      %y = arith.truncf %p : {T32} to {T16}
{_tile("y_acc", "y_view", ["%row", "%c0"], [rblk, cols], [rows, cols], dt, "      ")}
      ktdp.store %y, %y_acc : {T16}, !ktdp.access_tile<{rblk}x{cols}xindex>
      scf.yield
    }}
    return
  }}
}}
"""


def rmsnorm(rows: int = 32768, cols: int = 4096, cores: int = 512, rblk: int = 8, dt: str = "f16") -> str:
    """y = x * rsqrt(mean(x^2) + eps) * w, with f32 math and a `dt` (f16 or bf16) result."""
    rpc = rows // cores
    assert rpc * cores == rows and rpc % rblk == 0
    T16, T32, V32 = _t([rblk, cols], dt), _t([rblk, cols], "f32"), _t([rblk], "f32")
    W16, W32 = _t([cols], dt), _t([cols], "f32")
    return f"""module {{
{_row_header("rmsnorm_kernel", "%x_ptr: index, %w_ptr: index, %y_ptr: index, %eps: f32", rows, cols, cores, rpc)}
    %step = arith.constant {rblk} : index
{_view("x_view", "x_ptr", [rows, cols], [cols, 1], dt)}
{_view("w_view", "w_ptr", [cols], [1], dt)}
{_view("y_view", "y_ptr", [rows, cols], [cols, 1], dt)}
    %zero = arith.constant 0.0 : f32
    %ncols = arith.constant {float(cols)} : f32
{_tile("w_acc", "w_view", ["%c0"], [cols], [cols], dt)}
    %w = ktdp.load %w_acc : !ktdp.access_tile<{cols}xindex> -> {W16}
    %wf = arith.extf %w : {W16} to {W32}
    scf.for %r = %c0 to %rpc step %step : index {{
      %row = arith.addi %row_base, %r : index
{_tile("x_acc", "x_view", ["%row", "%c0"], [rblk, cols], [rows, cols], dt, "      ")}
      %x = ktdp.load %x_acc : !ktdp.access_tile<{rblk}x{cols}xindex> -> {T16}
      %xf = arith.extf %x : {T16} to {T32}
      %sq = arith.mulf %xf, %xf : {T32}
      %ss_init = tensor.splat %zero : {V32}
      %ss = linalg.reduce {{ arith.addf }} ins(%sq : {T32}) outs(%ss_init : {V32}) dimensions = [1]
      %n_t = tensor.splat %ncols : {V32}
      %ms = arith.divf %ss, %n_t : {V32}
      %eps_t = tensor.splat %eps : {V32}
      %mse = arith.addf %ms, %eps_t : {V32}
      %rstd = math.rsqrt %mse : {V32}
      %rb_init = tensor.empty() : {T32}
      %rb = linalg.broadcast ins(%rstd : {V32}) outs(%rb_init : {T32}) dimensions = [1]
      %xn = arith.mulf %xf, %rb : {T32}
      %wb_init = tensor.empty() : {T32}
      %wb = linalg.broadcast ins(%wf : {W32}) outs(%wb_init : {T32}) dimensions = [0]
      %yf = arith.mulf %xn, %wb : {T32}
      %y = arith.truncf %yf : {T32} to {T16}
{_tile("y_acc", "y_view", ["%row", "%c0"], [rblk, cols], [rows, cols], dt, "      ")}
      ktdp.store %y, %y_acc : {T16}, !ktdp.access_tile<{rblk}x{cols}xindex>
      scf.yield
    }}
    return
  }}
}}
"""


def _strided_rows(fn, args, rows, cols, cores, body):
    """A kernel whose core c handles rows c, c + cores, ... one (1 x cols)
    row per loop step, as the reference's triton-ktir examples do."""
    return f"""module {{
  func.func @{fn}({args}) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %step = arith.constant {cores} : index
{_view("x_view", "x_ptr", [rows, cols], [cols, 1], "f16")}
{_view("y_view", "y_ptr", [rows, cols], [cols, 1], "f16")}
{body}
  }}
}}
"""


def softmax_extract(rows: int = 4096, cols: int = 1024, cores: int = 32) -> str:
    """Softmax in the form of the reference's triton-ktir softmax_fwd
    example: f16 math, and the row max and row sum read out of a
    tensor<1xf16> by tensor.extract, then spread over the row by
    tensor.splat (a scalar per row held on the device)."""
    T, V = _t([1, cols], "f16"), _t([1], "f16")
    at = f"!ktdp.access_tile<1x{cols}xindex>"
    body = f"""    %neg_inf = arith.constant 0xFC00 : f16
    %zero = arith.constant 0.0 : f16
    scf.for %row = %core_id to %n_rows step %step : index {{
{_tile("x_acc", "x_view", ["%row", "%c0"], [1, cols], [rows, cols], "f16", "      ")}
      %x = ktdp.load %x_acc : {at} -> {T}
      %mx_init = tensor.splat %neg_inf : {V}
      %mx = linalg.reduce {{ arith.maxnumf }} ins(%x : {T}) outs(%mx_init : {V}) dimensions = [1]
      %m = tensor.extract %mx[%c0] : {V}
      %mb = tensor.splat %m : {T}
      %d = arith.subf %x, %mb : {T}
      %e = math.exp %d : {T}
      %s_init = tensor.splat %zero : {V}
      %s = linalg.reduce {{ arith.addf }} ins(%e : {T}) outs(%s_init : {V}) dimensions = [1]
      %sv = tensor.extract %s[%c0] : {V}
      %sb = tensor.splat %sv : {T}
      %p = arith.divf %e, %sb : {T}
{_tile("y_acc", "y_view", ["%row", "%c0"], [1, cols], [rows, cols], "f16", "      ")}
      ktdp.store %p, %y_acc : {T}, {at}
      scf.yield
    }}
    return"""
    return _strided_rows("softmax_fwd", "%x_ptr: index, %y_ptr: index, %n_rows: index", rows, cols, cores, body)


def rmsnorm_extract(rows: int = 4096, cols: int = 1024, cores: int = 32) -> str:
    """RMSNorm in the form of the reference's latency examples: f16 math,
    the row's sum of squares read by tensor.extract, then scalar f16 ops
    (divide by the row length, add eps, rsqrt) before tensor.splat spreads
    the result over the row."""
    T, V = _t([1, cols], "f16"), _t([1], "f16")
    at = f"!ktdp.access_tile<1x{cols}xindex>"
    body = f"""{_view("w_view", "w_ptr", [1, cols], [cols, 1], "f16")}
{_tile("w_acc", "w_view", ["%c0", "%c0"], [1, cols], [1, cols], "f16")}
    %w = ktdp.load %w_acc : {at} -> {T}
    %zero = arith.constant 0.0 : f16
    %nf = arith.constant {float(cols)} : f16
    scf.for %row = %core_id to %n_rows step %step : index {{
{_tile("x_acc", "x_view", ["%row", "%c0"], [1, cols], [rows, cols], "f16", "      ")}
      %x = ktdp.load %x_acc : {at} -> {T}
      %sq = arith.mulf %x, %x : {T}
      %ss_init = tensor.splat %zero : {V}
      %ss = linalg.reduce {{ arith.addf }} ins(%sq : {T}) outs(%ss_init : {V}) dimensions = [1]
      %sv = tensor.extract %ss[%c0] : {V}
      %ms = arith.divf %sv, %nf : f16
      %mse = arith.addf %ms, %eps : f16
      %rs = math.rsqrt %mse : f16
      %rb = tensor.splat %rs : {T}
      %xn = arith.mulf %x, %rb : {T}
      %y = arith.mulf %xn, %w : {T}
{_tile("y_acc", "y_view", ["%row", "%c0"], [1, cols], [rows, cols], "f16", "      ")}
      ktdp.store %y, %y_acc : {T}, {at}
      scf.yield
    }}
    return"""
    return _strided_rows("rmsnorm_fwd", "%x_ptr: index, %w_ptr: index, %y_ptr: index, %n_rows: index, %eps: f16",
                         rows, cols, cores, body)


def layernorm_extract(rows: int = 1151, cols: int = 8192, block: int = 1024, cores: int = 32) -> str:
    """LayerNorm in the form of the reference's triton-ktir layernorm_fwd
    example: f16 math, one row per loop step (rows core, core + cores, ...),
    the row sum and the sum of squared deviations accumulated block by block
    in a loop-carried f16 tile and folded, mean and rstd as one-element
    tensors (mean = sum / N, rstd = 1 / sqrt(var / N + eps)) read by
    tensor.extract and spread by tensor.splat, both also stored, then y =
    (x - mean) * rstd * w + b block by block."""
    T, V = _t([1, block], "f16"), _t([1], "f16")
    at, a1 = f"!ktdp.access_tile<1x{block}xindex>", "!ktdp.access_tile<1xindex>"
    views = "\n".join(_view(n, p, [rows, cols], [cols, 1], "f16") for n, p in
                      (("x_view", "x_ptr"), ("y_view", "y_ptr"), ("w_view", "w_ptr"), ("b_view", "b_ptr")))
    views += "\n" + "\n".join(_view(n, p, [rows], [1], "f16") for n, p in (("mean_view", "mean_ptr"),
                                                                         ("rstd_view", "rstd_ptr")))

    def blk(name, view):
        return _tile(name, view, ["%row", "%col"], [1, block], [rows, cols], "f16", "          ")

    return f"""module {{
  func.func @layernorm_fwd(%x_ptr: index, %y_ptr: index, %w_ptr: index, %b_ptr: index, %mean_ptr: index,
                           %rstd_ptr: index, %n_cols: index, %eps: f16, %blk: index) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %n_rows = arith.constant {rows} : index
    %step = arith.constant {cores} : index
    %one = arith.constant 1.0 : f16
    %zero = arith.constant 0.0 : f16
{views}
    scf.for %row = %core_id to %n_rows step %step : index {{
      %zb = arith.constant dense<0.0> : {T}
      %acc = scf.for %col = %c0 to %n_cols step %blk iter_args(%a = %zb) -> {T} {{
{blk("xa", "x_view")}
        %x = ktdp.load %xa : {at} -> {T}
        %a2 = arith.addf %a, %x : {T}
        scf.yield %a2 : {T}
      }}
      %s0 = tensor.splat %zero : {V}
      %sum = linalg.reduce {{ arith.addf }} ins(%acc : {T}) outs(%s0 : {V}) dimensions = [1]
      %n_i = arith.index_cast %n_cols : index to i32
      %n_h = arith.sitofp %n_i : i32 to f16
      %n_t = tensor.splat %n_h : {V}
      %mean = arith.divf %sum, %n_t : {V}
      %m = tensor.extract %mean[%c0] : {V}
      %mb = tensor.splat %m : {T}
      %vacc = scf.for %col = %c0 to %n_cols step %blk iter_args(%v = %zb) -> {T} {{
{blk("xb", "x_view")}
        %x = ktdp.load %xb : {at} -> {T}
        %d = arith.subf %x, %mb : {T}
        %d2 = arith.mulf %d, %d : {T}
        %v2 = arith.addf %v, %d2 : {T}
        scf.yield %v2 : {T}
      }}
      %q0 = tensor.splat %zero : {V}
      %ssq = linalg.reduce {{ arith.addf }} ins(%vacc : {T}) outs(%q0 : {V}) dimensions = [1]
      %var = arith.divf %ssq, %n_t : {V}
      %eps_t = tensor.splat %eps : {V}
      %ve = arith.addf %var, %eps_t : {V}
      %sd = math.sqrt %ve : {V}
      %one_t = tensor.splat %one : {V}
      %rstd = arith.divf %one_t, %sd : {V}
      %r = tensor.extract %rstd[%c0] : {V}
      %rb = tensor.splat %r : {T}
{_tile("ma", "mean_view", ["%row"], [1], [rows], "f16", "      ")}
{_tile("ra", "rstd_view", ["%row"], [1], [rows], "f16", "      ")}
      ktdp.store %mean, %ma : {V}, {a1}
      ktdp.store %rstd, %ra : {V}, {a1}
      scf.for %col = %c0 to %n_cols step %blk {{
{blk("xc", "x_view")}
{blk("wc", "w_view")}
{blk("bc", "b_view")}
{blk("yc", "y_view")}
        %x = ktdp.load %xc : {at} -> {T}
        %w = ktdp.load %wc : {at} -> {T}
        %b = ktdp.load %bc : {at} -> {T}
        %xm = arith.subf %x, %mb : {T}
        %xh = arith.mulf %xm, %rb : {T}
        %xw = arith.mulf %xh, %w : {T}
        %y = arith.addf %xw, %b : {T}
        ktdp.store %y, %yc : {T}, {at}
        scf.yield
      }}
      scf.yield
    }}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# 4. GEMM
# ---------------------------------------------------------------------------

def gemm(M: int = 8192, N: int = 8192, K: int = 8192, bm: int = 128, bn: int = 128, bk: int = 64,
         gm: int = 8, gn: int = 8, out_dt: str = "f16") -> str:
    """C = A @ B on a gm x gn grid; each core loops over its (M/gm)x(N/gn)
    block in bm x bn tiles, accumulating f32 over K in bk steps; C is f16
    (the f32 sums rounded by arith.truncf) or, with out_dt="f32", the sums."""
    tm, tn = M // gm // bm, N // gn // bn
    assert tm * gm * bm == M and tn * gn * bn == N and K % bk == 0
    A16, B16 = _t([bm, bk], "f16"), _t([bk, bn], "f16")
    A32, B32, C32, C16 = _t([bm, bk], "f32"), _t([bk, bn], "f32"), _t([bm, bn], "f32"), _t([bm, bn], "f16")
    assert out_dt in ("f16", "f32")
    trunc = f"        %c16 = arith.truncf %acc : {C32} to {C16}" if out_dt == "f16" else ""
    cval, CO = ("%c16", C16) if out_dt == "f16" else ("%acc", C32)
    return f"""module {{
  func.func @gemm_kernel(%a_ptr: index, %b_ptr: index, %c_ptr: index)
      attributes {{grid = [{gm}, {gn}]}} {{
    %pid_m, %pid_n = ktdp.get_compute_tile_id : index, index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %K = arith.constant {K} : index
    %BK = arith.constant {bk} : index
    %BM = arith.constant {bm} : index
    %BN = arith.constant {bn} : index
    %TM = arith.constant {tm} : index
    %TN = arith.constant {tn} : index
    %zero = arith.constant 0.0 : f32
{_view("a_view", "a_ptr", [M, K], [K, 1], "f16")}
{_view("b_view", "b_ptr", [K, N], [N, 1], "f16")}
{_view("c_view", "c_ptr", [M, N], [N, 1], out_dt)}
    %m_blk = arith.muli %pid_m, %TM : index
    %n_blk = arith.muli %pid_n, %TN : index
    scf.for %i = %c0 to %TM step %c1 : index {{
      scf.for %j = %c0 to %TN step %c1 : index {{
        %mt = arith.addi %m_blk, %i : index
        %nt = arith.addi %n_blk, %j : index
        %m0 = arith.muli %mt, %BM : index
        %n0 = arith.muli %nt, %BN : index
        %acc0 = tensor.splat %zero : {C32}
        %acc = scf.for %k0 = %c0 to %K step %BK iter_args(%acc_i = %acc0) -> ({C32}) {{
{_tile("a_acc", "a_view", ["%m0", "%k0"], [bm, bk], [M, K], "f16", "          ")}
{_tile("b_acc", "b_view", ["%k0", "%n0"], [bk, bn], [K, N], "f16", "          ")}
          %a = ktdp.load %a_acc : !ktdp.access_tile<{bm}x{bk}xindex> -> {A16}
          %b = ktdp.load %b_acc : !ktdp.access_tile<{bk}x{bn}xindex> -> {B16}
          %a32 = arith.extf %a : {A16} to {A32}
          %b32 = arith.extf %b : {B16} to {B32}
          %acc_n = linalg.matmul ins(%a32, %b32 : {A32}, {B32}) outs(%acc_i : {C32}) -> {C32}
          scf.yield %acc_n : {C32}
        }}
{trunc}
{_tile("c_acc", "c_view", ["%m0", "%n0"], [bm, bn], [M, N], out_dt, "        ")}
        ktdp.store {cval}, %c_acc : {CO}, !ktdp.access_tile<{bm}x{bn}xindex>
        scf.yield
      }}
      scf.yield
    }}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# 5. Flash attention (causal)
# ---------------------------------------------------------------------------

_FA_MASK = """      %sm_init = tensor.empty() : {Sf}
      %sm = linalg.generic {{indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0, d1)>],
                            iterator_types = ["parallel", "parallel"]}}
          ins(%s : {Sf}) outs(%sm_init : {Sf}) {{
        ^bb0(%sv: f32, %out: f32):
          %row = linalg.index 0 : index
          %col = linalg.index 1 : index
          %qpos = arith.addi %q0, %row : index
          %kpos = arith.addi %k0, %col : index
          %keep = arith.cmpi ule, %kpos, %qpos : index
          %r = arith.select %keep, %sv, %neg_inf : f32
          linalg.yield %r : f32
      }} -> {Sf}
"""


def flash_attention(B: int = 4, H: int = 32, S: int = 8192, D: int = 128, blk: int = 128, dt: str = "bf16",
                    causal: bool = True) -> str:
    """O = softmax(Q K^T * scale, causal) V with online softmax over KV tiles.

    Grid [S/blk, H, B]; core (qb, h, b) owns query rows [qb*blk, (qb+1)*blk)
    of head (b, h) and visits KV tiles 0..qb (the causal prefix), or all
    S/blk tiles when `causal` is False.
    """
    nq = S // blk
    shp = [B, H, S, D]
    strides = [H * S * D, S * D, D, 1]
    T4 = _t([1, 1, blk, D], dt)
    Tb, Tf = _t([blk, D], dt), _t([blk, D], "f32")
    Sf = _t([blk, blk], "f32")
    Vf = _t([blk], "f32")
    at = f"!ktdp.access_tile<1x1x{blk}x{D}xindex>"
    n_kv = "arith.addi %qb, %c1 : index" if causal else f"arith.constant {nq} : index"
    sm = "%sm" if causal else "%s"
    mask = _FA_MASK.format(Sf=Sf) if causal else ""

    def tile(name, view, row):
        return _tile(name, view, ["%b", "%h", row, "%c0"], [1, 1, blk, D], shp, dt, "      ")

    return f"""module {{
  func.func @flash_attention(%q_ptr: index, %k_ptr: index, %v_ptr: index, %o_ptr: index, %scale: f32)
      attributes {{grid = [{nq}, {H}, {B}]}} {{
    %qb, %h, %b = ktdp.get_compute_tile_id : index, index, index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %BLK = arith.constant {blk} : index
    %zero = arith.constant 0.0 : f32
    %neg_inf = arith.constant 0xFF800000 : f32
{_view("q_view", "q_ptr", shp, strides, dt)}
{_view("k_view", "k_ptr", shp, strides, dt)}
{_view("v_view", "v_ptr", shp, strides, dt)}
{_view("o_view", "o_ptr", shp, strides, dt)}
    %q0 = arith.muli %qb, %BLK : index
{_tile("q_acc", "q_view", ["%b", "%h", "%q0", "%c0"], [1, 1, blk, D], shp, dt)}
    %q4 = ktdp.load %q_acc : {at} -> {T4}
    %q2 = tensor.collapse_shape %q4 [[0, 1, 2], [3]] : {T4} into {Tb}
    %q = arith.extf %q2 : {Tb} to {Tf}
    %scale_t = tensor.splat %scale : {Sf}
    %m_init = tensor.splat %neg_inf : {Vf}
    %l_init = tensor.splat %zero : {Vf}
    %acc_init = tensor.splat %zero : {Tf}
    %n_kv = {n_kv}
    %m_f, %l_f, %acc_f = scf.for %j = %c0 to %n_kv step %c1
        iter_args(%m = %m_init, %l = %l_init, %acc = %acc_init) -> ({Vf}, {Vf}, {Tf}) {{
      %k0 = arith.muli %j, %BLK : index
{tile("k_acc", "k_view", "%k0")}
{tile("v_acc", "v_view", "%k0")}
      %k4 = ktdp.load %k_acc : {at} -> {T4}
      %v4 = ktdp.load %v_acc : {at} -> {T4}
      %k2 = tensor.collapse_shape %k4 [[0, 1, 2], [3]] : {T4} into {Tb}
      %v2 = tensor.collapse_shape %v4 [[0, 1, 2], [3]] : {T4} into {Tb}
      %kf = arith.extf %k2 : {Tb} to {Tf}
      %vf = arith.extf %v2 : {Tb} to {Tf}
      %kt_init = tensor.empty() : {_t([D, blk], "f32")}
      %kt = linalg.transpose ins(%kf : {Tf}) outs(%kt_init : {_t([D, blk], "f32")}) permutation = [1, 0]
      %s_init = tensor.splat %zero : {Sf}
      %qk = linalg.matmul ins(%q, %kt : {Tf}, {_t([D, blk], "f32")}) outs(%s_init : {Sf}) -> {Sf}
      %s = arith.mulf %scale_t, %qk : {Sf}
{mask}      %rm_init = tensor.splat %neg_inf : {Vf}
      %rm = linalg.reduce {{ arith.maximumf }} ins({sm} : {Sf}) outs(%rm_init : {Vf}) dimensions = [1]
      %m_new = arith.maximumf %m, %rm : {Vf}
      %p_init = tensor.empty() : {Sf}
      %p = linalg.generic {{indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>,
                                            affine_map<(d0, d1) -> (d0, d1)>],
                           iterator_types = ["parallel", "parallel"]}}
          ins({sm}, %m_new : {Sf}, {Vf}) outs(%p_init : {Sf}) {{
        ^bb0(%sv: f32, %mv: f32, %out: f32):
          %dd = arith.subf %sv, %mv : f32
          %ee = math.exp %dd : f32
          linalg.yield %ee : f32
      }} -> {Sf}
      %ls_init = tensor.splat %zero : {Vf}
      %ls = linalg.reduce {{ arith.addf }} ins(%p : {Sf}) outs(%ls_init : {Vf}) dimensions = [1]
      %md = arith.subf %m, %m_new : {Vf}
      %alpha = math.exp %md : {Vf}
      %accs_init = tensor.empty() : {Tf}
      %accs = linalg.generic {{indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>,
                                               affine_map<(d0, d1) -> (d0, d1)>],
                              iterator_types = ["parallel", "parallel"]}}
          ins(%acc, %alpha : {Tf}, {Vf}) outs(%accs_init : {Tf}) {{
        ^bb0(%av: f32, %al: f32, %out: f32):
          %sc = arith.mulf %av, %al : f32
          linalg.yield %sc : f32
      }} -> {Tf}
      %acc_n = linalg.matmul ins(%p, %vf : {Sf}, {Tf}) outs(%accs : {Tf}) -> {Tf}
      %la = arith.mulf %l, %alpha : {Vf}
      %l_n = arith.addf %la, %ls : {Vf}
      scf.yield %m_new, %l_n, %acc_n : {Vf}, {Vf}, {Tf}
    }}
    %o_init = tensor.empty() : {Tf}
    %of = linalg.generic {{indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>,
                                          affine_map<(d0, d1) -> (d0, d1)>],
                         iterator_types = ["parallel", "parallel"]}}
        ins(%acc_f, %l_f : {Tf}, {Vf}) outs(%o_init : {Tf}) {{
      ^bb0(%av: f32, %lv: f32, %out: f32):
        %q_ = arith.divf %av, %lv : f32
        linalg.yield %q_ : f32
    }} -> {Tf}
    %ob = arith.truncf %of : {Tf} to {Tb}
    %o4 = tensor.expand_shape %ob [[0, 1, 2], [3]] output_shape [1, 1, {blk}, {D}] : {Tb} into {T4}
{_tile("o_acc", "o_view", ["%b", "%h", "%q0", "%c0"], [1, 1, blk, D], shp, dt)}
    ktdp.store %o4, %o_acc : {T4}, {at}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# 6. paged attention (unified 2-D attention over a paged KV cache)
# ---------------------------------------------------------------------------

def _gen2(ins, maps, out_t, args, body, res, indent="      "):
    """A two-dimensional parallel linalg.generic with a scalar body."""
    m = ", ".join(f"affine_map<(d0, d1) -> ({x})>" for x in maps)
    i = ", ".join(n for n, _ in ins)
    it = ", ".join(t for _, t in ins)
    lines = [f"linalg.generic {{indexing_maps = [{m}],",
             '    iterator_types = ["parallel", "parallel"]}',
             f"    ins({i} : {it}) outs({res} : {out_t}) {{",
             f"  ^bb0({args}):"] + [f"    {b}" for b in body] + [f"}} -> {out_t}"]
    return ("\n" + indent).join(lines)


def _gen1(ins, out_t, args, body, res, indent="      "):
    """A one-dimensional parallel linalg.generic with identity maps."""
    m = ", ".join(["affine_map<(d0) -> (d0)>"] * (len(ins) + 1))
    i = ", ".join(n for n, _ in ins)
    it = ", ".join(t for _, t in ins)
    lines = [f'linalg.generic {{indexing_maps = [{m}], iterator_types = ["parallel"]}}',
             f"    ins({i} : {it}) outs({res} : {out_t}) {{",
             f"  ^bb0({args}):"] + [f"    {b}" for b in body] + [f"}} -> {out_t}"]
    return ("\n" + indent).join(lines)


def paged_attention(tokens: int = 8, q_heads: int = 32, kv_heads: int = 8, head: int = 128,
                    page: int = 16, blocks: int = 64, max_pages: int = 16, block_q: int = 2,
                    total_tokens: int = 0, dt: str = "f16", causal: bool = True) -> str:
    """Causal grouped-query attention over a paged KV cache, in the form of
    the reference's unified 2-D attention example
    (examples/triton-ktir/paged_attention.mlir, parameters in its header and
    tests/conftest.py:222-236).

    query/output [total_tokens (default tokens), q_heads, head] f16; key/value caches
    [blocks, page, kv_heads, head] f16; block_tables [1, max_pages] i32.
    Grid [tokens / block_q, kv_heads]: core (p0, p1) takes query tokens
    [start + p0*block_q, +block_q) of the q_heads/kv_heads query heads that
    share KV head p1 (BM = block_q * group rows), then for j < num_tiles
    reads page block_tables[0, offset + j] of K and V through indirect access
    tiles, masks key position j*page + c above context_len + token position,
    and keeps the online-softmax state (row max M, row sum L starting at 1,
    f32 accumulator).  Output = acc / L, truncated to f16.  `dt` sets the
    element type of query, caches and output (f16 or bf16); `causal` False
    drops the mask generic.
    """
    g = q_heads // kv_heads
    bm = block_q * g
    D = head
    qs, cs = [max(total_tokens, tokens), q_heads, D], [blocks, page, kv_heads, D]
    qst, cst = [q_heads * D, D, 1], [page * kv_heads * D, kv_heads * D, D, 1]
    Q3 = _t([block_q, g, D], dt)
    Qh, Qf = _t([bm, D], dt), _t([bm, D], "f32")
    K4 = _t([1, page, 1, D], dt)
    Kh, Kf = _t([page, D], dt), _t([page, D], "f32")
    KTh, KTf = _t([D, page], dt), _t([D, page], "f32")
    Sf, Vf = _t([bm, page], "f32"), _t([bm], "f32")
    at_q = f"!ktdp.access_tile<{block_q}x{g}x{D}xindex>"
    at_kv = f"!ktdp.access_tile<1x{page}x1x{D}xindex>"
    vss = (f"affine_set<(d0, d1, d2, d3) : (d0 >= 0, -d0 >= 0, d1 >= 0, -d1 + {page - 1} >= 0, "
           f"d2 >= 0, -d2 >= 0, d3 >= 0, -d3 + {D - 1} >= 0)>")

    def kv_tile(name, view):
        return (f"      %{name} = ktdp.construct_indirect_access_tile intermediate_variables(%e0, %e1, %e2, %e3)\n"
                f"          %{view}[ind(%bt_view[%c0, %bt_col + %e0]), (%e1), (%p1 + %e2), (%e3)] {{\n"
                f"        variables_space_set = {vss},\n"
                f"        variables_space_order = affine_map<(d0, d1, d2, d3) -> (d0, d1, d2, d3)>\n"
                f"      }} : memref<{'x'.join(map(str, cs))}x{dt}>, memref<1x{max_pages}xi32> -> {at_kv}")

    mask = _gen2([("%s", Sf)], ["d0, d1", "d0, d1"], Sf, "%sv: f32, %o: f32", [
        "%r = linalg.index 0 : index",
        "%cc = linalg.index 1 : index",
        "%tok = arith.divui %r, %cG : index",
        "%qpos = arith.addi %p0_q, %tok : index",
        "%qabs = arith.addi %context_len, %qpos : index",
        "%kpos = arith.addi %k0, %cc : index",
        "%keep = arith.cmpi ule, %kpos, %qabs : index",
        "%mv = arith.select %keep, %sv, %neg_inf : f32",
        "linalg.yield %mv : f32"], "%sm_init")
    m_new = _gen1([("%M", Vf), ("%rm", Vf)], Vf, "%a: f32, %b: f32, %o: f32",
                  ["%mx = arith.maximumf %a, %b : f32", "linalg.yield %mx : f32"], "%mn_init")
    sm = "%sm" if causal else "%s"
    p = _gen2([(sm, Sf), ("%m_new", Vf)], ["d0, d1", "d0", "d0, d1"], Sf, "%sv: f32, %mv: f32, %o: f32",
              ["%dd = arith.subf %sv, %mv : f32", "%ee = math.exp %dd : f32", "linalg.yield %ee : f32"], "%p_init")
    alpha = _gen1([("%M", Vf), ("%m_new", Vf)], Vf, "%a: f32, %b: f32, %o: f32",
                  ["%dd = arith.subf %a, %b : f32", "%ee = math.exp %dd : f32", "linalg.yield %ee : f32"],
                  "%al_init")
    accs = _gen2([("%acc", Qf), ("%alpha", Vf)], ["d0, d1", "d0", "d0, d1"], Qf, "%av: f32, %al: f32, %o: f32",
                 ["%sc = arith.mulf %av, %al : f32", "linalg.yield %sc : f32"], "%accs_init")
    l_new = _gen1([("%L", Vf), ("%alpha", Vf), ("%ls", Vf)], Vf, "%l: f32, %al: f32, %lj: f32, %o: f32",
                  ["%la = arith.mulf %l, %al : f32", "%ln = arith.addf %la, %lj : f32", "linalg.yield %ln : f32"],
                  "%ln_init")
    masked = f"      %sm_init = tensor.empty() : {Sf}\n      %sm = {mask}\n" if causal else ""
    fin = _gen2([("%acc_f", Qf), ("%L_f", Vf)], ["d0, d1", "d0", "d0, d1"], Qf, "%av: f32, %lv: f32, %o: f32",
                ["%qq = arith.divf %av, %lv : f32", "linalg.yield %qq : f32"], "%fin_init", "    ")
    return f"""module {{
  func.func @kernel_unified_attention_spyre_2d(%output_ptr: index, %query_ptr: index, %key_cache_ptr: index,
      %value_cache_ptr: index, %block_tables_ptr: index, %cur_batch_start_index: index,
      %block_table_offset: index, %num_tiles: index, %context_len: index, %scale: f32)
      attributes {{grid = [{tokens // block_q}, {kv_heads}]}} {{
    %p0, %p1 = ktdp.get_compute_tile_id : index, index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %cBQ = arith.constant {block_q} : index
    %cG = arith.constant {g} : index
    %cP = arith.constant {page} : index
    %p0_q = arith.muli %p0, %cBQ : index
    %q_row = arith.addi %cur_batch_start_index, %p0_q : index
    %head0 = arith.muli %p1, %cG : index
{_view("q_view", "query_ptr", qs, qst, dt)}
{_view("k_view", "key_cache_ptr", cs, cst, dt)}
{_view("v_view", "value_cache_ptr", cs, cst, dt)}
{_view("bt_view", "block_tables_ptr", [1, max_pages], [max_pages, 1], "i32")}
{_view("o_view", "output_ptr", qs, qst, dt)}
{_tile("q_acc", "q_view", ["%q_row", "%head0", "%c0"], [block_q, g, D], qs, dt)}
    %q3 = ktdp.load %q_acc : {at_q} -> {Q3}
    %qh = tensor.collapse_shape %q3 [[0, 1], [2]] : {Q3} into {Qh}
    %q = arith.extf %qh : {Qh} to {Qf}
    %neg_bits = arith.constant 0xFF800000 : i32
    %neg_inf = arith.bitcast %neg_bits : i32 to f32
    %zero = arith.constant 0.0 : f32
    %one = arith.constant 1.0 : f32
    %M0 = tensor.splat %neg_inf : {Vf}
    %L0 = tensor.splat %one : {Vf}
    %acc0 = tensor.splat %zero : {Qf}
    %M_f, %L_f, %acc_f = scf.for %j = %c0 to %num_tiles step %c1
        iter_args(%M = %M0, %L = %L0, %acc = %acc0) -> ({Vf}, {Vf}, {Qf}) {{
      %bt_col = arith.addi %block_table_offset, %j : index
{kv_tile("k_acc", "k_view")}
{kv_tile("v_acc", "v_view")}
      %k4 = ktdp.load %k_acc : {at_kv} -> {K4}
      %v4 = ktdp.load %v_acc : {at_kv} -> {K4}
      %kh = tensor.collapse_shape %k4 [[0, 1], [2, 3]] : {K4} into {Kh}
      %kt_init = tensor.empty() : {KTh}
      %kth = linalg.transpose ins(%kh : {Kh}) outs(%kt_init : {KTh}) permutation = [1, 0]
      %vh = tensor.collapse_shape %v4 [[0, 1], [2, 3]] : {K4} into {Kh}
      %kt = arith.extf %kth : {KTh} to {KTf}
      %v = arith.extf %vh : {Kh} to {Kf}
      %s_init = tensor.splat %zero : {Sf}
      %qk = linalg.matmul ins(%q, %kt : {Qf}, {KTf}) outs(%s_init : {Sf}) -> {Sf}
      %scale_t = tensor.splat %scale : {Sf}
      %s = arith.mulf %scale_t, %qk : {Sf}
      %k0 = arith.muli %j, %cP : index
{masked}      %rm_init = tensor.splat %neg_inf : {Vf}
      %rm = linalg.reduce ins({sm} : {Sf}) outs(%rm_init : {Vf}) dimensions = [1]
        (%a: f32, %b: f32) {{
          %mx = arith.maximumf %a, %b : f32
          linalg.yield %mx : f32
        }}
      %mn_init = tensor.empty() : {Vf}
      %m_new = {m_new}
      %p_init = tensor.empty() : {Sf}
      %p = {p}
      %ls_init = tensor.splat %zero : {Vf}
      %ls = linalg.reduce ins(%p : {Sf}) outs(%ls_init : {Vf}) dimensions = [1]
        (%a: f32, %b: f32) {{
          %sum = arith.addf %a, %b : f32
          linalg.yield %sum : f32
        }}
      %al_init = tensor.empty() : {Vf}
      %alpha = {alpha}
      %accs_init = tensor.empty() : {Qf}
      %accs = {accs}
      %acc_n = linalg.matmul ins(%p, %v : {Sf}, {Kf}) outs(%accs : {Qf}) -> {Qf}
      %ln_init = tensor.empty() : {Vf}
      %L_n = {l_new}
      scf.yield %m_new, %L_n, %acc_n : {Vf}, {Vf}, {Qf}
    }}
    %fin_init = tensor.empty() : {Qf}
    %of = {fin}
    %oh = arith.truncf %of : {Qf} to {Qh}
    %o3 = tensor.expand_shape %oh [[0, 1], [2]] output_shape [{block_q}, {g}, {D}] : {Qh} into {Q3}
{_tile("o_acc", "o_view", ["%q_row", "%head0", "%c0"], [block_q, g, D], qs, dt)}
    ktdp.store %o3, %o_acc : {Q3}, {at_q}
    return
  }}
}}
"""


# ---------------------------------------------------------------------------
# 7. single-tile attention with f16 arithmetic, and rotary embedding
# ---------------------------------------------------------------------------

def sdpa_f16(n: int = 32, d: int = 64, rows: int = 32) -> str:
    """out = softmax(Q K^T * 0.125) V with every step in f16, in the form of
    the reference's examples/triton-ktir/sdpa_2d.mlir (f16 matmuls into f16
    outs, linalg.fill inits, linalg.broadcast of the row max and row sum).

    Q, K, V, out are [n, d] f16; grid [n / rows]: core p takes query rows
    [p * rows, (p + 1) * rows) against all n keys."""
    Qt, Kt, KTt, St, Rt = (_t([rows, d], "f16"), _t([n, d], "f16"), _t([d, n], "f16"),
                           _t([rows, n], "f16"), _t([rows], "f16"))
    vs = [n, d]

    def load(name, view, row, shape):
        at = "x".join(map(str, shape))
        return (_tile(f"{name}_acc", view, [row, "%c0"], shape, vs, "f16") + "\n"
                f"    %{name} = ktdp.load %{name}_acc : !ktdp.access_tile<{at}xindex> -> {_t(shape, 'f16')}")

    return f"""module {{
  func.func @sdpa_kernel_2d(%q_ptr: index, %k_ptr: index, %v_ptr: index, %output_ptr: index)
      attributes {{grid = [{n // rows}]}} {{
    %pid = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %cR = arith.constant {rows} : index
    %zero = arith.constant 0.0 : f16
    %scale = arith.constant 1.25e-01 : f16
    %neg_inf = arith.constant 0xFC00 : f16
    %row0 = arith.muli %pid, %cR : index
{_view("q_view", "q_ptr", vs, [d, 1], "f16")}
{_view("k_view", "k_ptr", vs, [d, 1], "f16")}
{_view("v_view", "v_ptr", vs, [d, 1], "f16")}
{_view("o_view", "output_ptr", vs, [d, 1], "f16")}
{load("q", "q_view", "%row0", [rows, d])}
{load("k", "k_view", "%c0", [n, d])}
    %kt_init = tensor.empty() : {KTt}
    %kt = linalg.transpose ins(%k : {Kt}) outs(%kt_init : {KTt}) permutation = [1, 0]
    %qk_init = tensor.empty() : {St}
    %qk = linalg.matmul ins(%q, %kt : {Qt}, {KTt}) outs(%qk_init : {St}) -> {St}
    %scale_t = tensor.splat %scale : {St}
    %s = arith.mulf %qk, %scale_t : {St}
    %m_init = tensor.empty() : {Rt}
    %m_fill = linalg.fill ins(%neg_inf : f16) outs(%m_init : {Rt}) -> {Rt}
    %m = linalg.reduce {{ arith.maximumf }} ins(%s : {St}) outs(%m_fill : {Rt}) dimensions = [1]
    %mb_init = tensor.empty() : {St}
    %mb = linalg.broadcast ins(%m : {Rt}) outs(%mb_init : {St}) dimensions = [1]
    %sh = arith.subf %s, %mb : {St}
    %p = math.exp %sh : {St}
    %l_init = tensor.empty() : {Rt}
    %l_fill = linalg.fill ins(%zero : f16) outs(%l_init : {Rt}) -> {Rt}
    %l = linalg.reduce {{ arith.addf }} ins(%p : {St}) outs(%l_fill : {Rt}) dimensions = [1]
    %lb_init = tensor.empty() : {St}
    %lb = linalg.broadcast ins(%l : {Rt}) outs(%lb_init : {St}) dimensions = [1]
    %pn = arith.divf %p, %lb : {St}
{load("v", "v_view", "%c0", [n, d])}
    %acc_init = tensor.empty() : {Qt}
    %acc_fill = linalg.fill ins(%zero : f16) outs(%acc_init : {Qt}) -> {Qt}
    %acc = linalg.matmul ins(%pn, %v : {St}, {Kt}) outs(%acc_fill : {Qt}) -> {Qt}
{_tile("o_acc", "o_view", ["%row0", "%c0"], [rows, d], vs, "f16")}
    ktdp.store %acc, %o_acc : {Qt}, !ktdp.access_tile<{rows}x{d}xindex>
    return
  }}
}}
"""


def rope(heads: int = 40, seq: int = 4096, head: int = 128, grid_s: int = 4, grid_h: int = 2,
         tile: int = 256) -> str:
    """Rotary position embedding in half layout, f16, in the form of the
    reference's examples/latency/rope_fwd_4x2.mlir:
    y[:, :D/2] = x1 * cos - x2 * sin, y[:, D/2:] = x1 * sin + x2 * cos,
    with x1 / x2 the two halves of each [seq, head] row block of one head.

    x / out are [heads * seq, head] f16, cos / sin [seq, head / 2] f16.
    Grid [grid_s, grid_h]: core (ps, ph) takes positions
    [ps * seq / grid_s, +seq / grid_s) in tiles of `tile` rows, and for each
    tile the heads [ph * heads / grid_h, +heads / grid_h)."""
    half = head // 2
    per_s, per_h = seq // grid_s, heads // grid_h
    T = _t([tile, half], "f16")
    at = f"!ktdp.access_tile<{tile}x{half}xindex>"
    xs, cs = [heads * seq, head], [seq, half]

    def tl(name, view, row, col, vshape, indent):
        return _tile(name, view, [row, col], [tile, half], vshape, "f16", indent)

    return f"""module {{
  func.func @rope_fwd_kernel(%x_ptr: index, %cos_ptr: index, %sin_ptr: index, %out_ptr: index)
      attributes {{grid = [{grid_s}, {grid_h}]}} {{
    %ps, %ph = ktdp.get_compute_tile_id : index, index
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %cH = arith.constant {half} : index
    %cT = arith.constant {tile} : index
    %cS = arith.constant {seq} : index
    %n_tiles = arith.constant {per_s // tile} : index
    %n_heads = arith.constant {per_h} : index
    %cPS = arith.constant {per_s} : index
    %s0 = arith.muli %ps, %cPS : index
    %h0 = arith.muli %ph, %n_heads : index
{_view("x_view", "x_ptr", xs, [head, 1], "f16")}
{_view("cos_view", "cos_ptr", cs, [half, 1], "f16")}
{_view("sin_view", "sin_ptr", cs, [half, 1], "f16")}
{_view("o_view", "out_ptr", xs, [head, 1], "f16")}
    scf.for %t = %c0 to %n_tiles step %c1 {{
      %toff = arith.muli %t, %cT : index
      %pos = arith.addi %s0, %toff : index
{tl("cos_acc", "cos_view", "%pos", "%c0", cs, "      ")}
      %cos = ktdp.load %cos_acc : {at} -> {T}
{tl("sin_acc", "sin_view", "%pos", "%c0", cs, "      ")}
      %sin = ktdp.load %sin_acc : {at} -> {T}
      scf.for %h = %c0 to %n_heads step %c1 {{
        %hh = arith.addi %h0, %h : index
        %hb = arith.muli %hh, %cS : index
        %row = arith.addi %hb, %pos : index
{tl("x1_acc", "x_view", "%row", "%c0", xs, "        ")}
        %x1 = ktdp.load %x1_acc : {at} -> {T}
{tl("x2_acc", "x_view", "%row", "%cH", xs, "        ")}
        %x2 = ktdp.load %x2_acc : {at} -> {T}
        %a = arith.mulf %x1, %cos : {T}
        %b = arith.mulf %x2, %sin : {T}
        %y1 = arith.subf %a, %b : {T}
{tl("y1_acc", "o_view", "%row", "%c0", xs, "        ")}
        ktdp.store %y1, %y1_acc : {T}, {at}
        %c = arith.mulf %x1, %sin : {T}
        %e = arith.mulf %x2, %cos : {T}
        %y2 = arith.addf %c, %e : {T}
{tl("y2_acc", "o_view", "%row", "%cH", xs, "        ")}
        ktdp.store %y2, %y2_acc : {T}, {at}
        scf.yield
      }}
      scf.yield
    }}
    return
  }}
}}
"""
