"""Small KTIR kernels with known answers.

The expected values are the reference test suite's golden vectors for the
hot path; the kernels are written here from scratch around them (pointer
arguments instead of the reference tests' hand-seeded HBM sticks):

- indirect gather Y[m,k] = X[IDX1[m,k], IDX2[m,k]] -> [[12, 9, 6, 3]] x 4
  (reference tests/test_indirect_access.py:122-155)
- indirect scatter bijection and all-to-one collision (last writer wins,
  Y[0,0] = 15, untouched cells keep their value) (:371-441)
- negative index -> IndexError (:444-470)
- sub-tile load [[4,5],[8,9]], strided load [[0,1],[4,5]], strided store,
  upper-triangle gather/scatter, transposed access order
  (tests/test_tile.py:175-328)
- reductions: sum(1..4) = 10, with outs init 100 -> 110
  (tests/test_examples.py:410-437, tests/test_dialects_exec.py:855-1047)
- HBM reads past an allocation's end give zeros, writes past it are dropped
  (tests/test_ktir_cpu.py:51-115, memory.py:253-305)
"""

import numpy as np

from ktir_cpu_amd.configs import _t, _tile, _view

BOX4 = "affine_set<(d0, d1) : (d0 >= 0, -d0 + 3 >= 0, d1 >= 0, -d1 + 3 >= 0)>"
ID2 = "affine_map<(d0, d1) -> (d0, d1)>"


def _fn(name, args, body, grid="[1, 1]"):
    return (f"module {{\n  func.func @{name}({args}) attributes {{grid = {grid}}} {{\n"
            f"{body}\n    return\n  }}\n}}\n")


def _iat(name, view, i1, i2, vdt):
    return (f"    %{name} = ktdp.construct_indirect_access_tile intermediate_variables(%m, %k)\n"
            f"        %{view}[ind(%{i1}[%m, %k]), ind(%{i2}[%m, %k])] {{\n"
            f"      variables_space_set = {BOX4},\n      variables_space_order = {ID2}\n"
            f"    }} : memref<4x4x{vdt}>, memref<4x4xi32>, memref<4x4xi32> -> !ktdp.access_tile<4x4xindex>")


def _views4():
    return "\n".join([
        _view("X", "x_ptr", [4, 4], [4, 1], "f16"),
        _view("I1", "i1_ptr", [4, 4], [4, 1], "i32"),
        _view("I2", "i2_ptr", [4, 4], [4, 1], "i32"),
        _view("Y", "y_ptr", [4, 4], [4, 1], "f16"),
        "    %c0 = arith.constant 0 : index",
    ])


ARGS4 = "%x_ptr: index, %i1_ptr: index, %i2_ptr: index, %y_ptr: index"


def indirect_gather():
    body = "\n".join([
        _views4(),
        _iat("xt", "X", "I1", "I2", "f16"),
        _tile("yt", "Y", ["%c0", "%c0"], [4, 4], [4, 4], "f16"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<4x4xindex> -> tensor<4x4xf16>",
        "    ktdp.store %v, %yt : tensor<4x4xf16>, !ktdp.access_tile<4x4xindex>",
    ])
    x = np.arange(16, dtype=np.float16).reshape(4, 4)
    i1 = np.tile(np.array([3, 2, 1, 0], np.int32), 4).reshape(4, 4)
    i2 = np.tile(np.array([0, 1, 2, 3], np.int32), 4).reshape(4, 4)
    kw = dict(x_ptr=x, i1_ptr=i1, i2_ptr=i2, y_ptr=np.zeros((4, 4), np.float16))
    expected = np.array([[12, 9, 6, 3]] * 4, dtype=np.float16)
    return _fn("gather4", ARGS4, body), "gather4", kw, "y_ptr", expected


def indirect_scatter(collide=False):
    body = "\n".join([
        _views4(),
        _tile("xt", "X", ["%c0", "%c0"], [4, 4], [4, 4], "f16"),
        _iat("yt", "Y", "I1", "I2", "f16"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<4x4xindex> -> tensor<4x4xf16>",
        "    ktdp.store %v, %yt : tensor<4x4xf16>, !ktdp.access_tile<4x4xindex>",
    ])
    x = np.arange(16, dtype=np.float16).reshape(4, 4)
    if collide:
        i1 = np.zeros((4, 4), np.int32)
        i2 = np.zeros((4, 4), np.int32)
        y0 = np.full((4, 4), -1, np.float16)
        expected = y0.copy()
        expected[0, 0] = 15
    else:
        i1 = np.repeat(np.array([3, 2, 1, 0], np.int32), 4).reshape(4, 4)
        i2 = np.tile(np.array([3, 2, 1, 0], np.int32), 4).reshape(4, 4)
        y0 = np.zeros((4, 4), np.float16)
        expected = np.array([[(3 - r) * 4 + (3 - c) for c in range(4)] for r in range(4)], dtype=np.float16)
    kw = dict(x_ptr=x, i1_ptr=i1, i2_ptr=i2, y_ptr=y0)
    return _fn("scatter4", ARGS4, body), "scatter4", kw, "y_ptr", expected


def negative_index(scatter=False):
    src, fn, kw, key, _ = indirect_scatter() if scatter else indirect_gather()
    kw["i1_ptr"] = kw["i1_ptr"].copy()
    kw["i1_ptr"][2, 1] = -1
    return src, fn, kw


def subtile_load():
    """Y (2x2) = X[1:3, 0:2] of a 4x4 arange."""
    body = "\n".join([
        _view("X", "x_ptr", [4, 4], [4, 1], "f16"),
        _view("Y", "y_ptr", [2, 2], [2, 1], "f16"),
        "    %c0 = arith.constant 0 : index",
        "    %c1 = arith.constant 1 : index",
        _tile("xt", "X", ["%c1", "%c0"], [2, 2], [4, 4], "f16"),
        _tile("yt", "Y", ["%c0", "%c0"], [2, 2], [2, 2], "f16"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<2x2xindex> -> tensor<2x2xf16>",
        "    ktdp.store %v, %yt : tensor<2x2xf16>, !ktdp.access_tile<2x2xindex>",
    ])
    kw = dict(x_ptr=np.arange(16, dtype=np.float16).reshape(4, 4), y_ptr=np.zeros((2, 2), np.float16))
    return (_fn("subtile", "%x_ptr: index, %y_ptr: index", body), "subtile", kw, "y_ptr",
            np.array([[4, 5], [8, 9]], np.float16))


def strided_store():
    """Write a 2x2 patch into the top-left of a 4x4 zero tensor."""
    body = "\n".join([
        _view("P", "p_ptr", [2, 2], [2, 1], "f16"),
        _view("Y", "y_ptr", [4, 4], [4, 1], "f16"),
        "    %c0 = arith.constant 0 : index",
        _tile("pt", "P", ["%c0", "%c0"], [2, 2], [2, 2], "f16"),
        _tile("yt", "Y", ["%c0", "%c0"], [2, 2], [4, 4], "f16"),
        "    %v = ktdp.load %pt : !ktdp.access_tile<2x2xindex> -> tensor<2x2xf16>",
        "    ktdp.store %v, %yt : tensor<2x2xf16>, !ktdp.access_tile<2x2xindex>",
    ])
    kw = dict(p_ptr=np.array([[1, 2], [3, 4]], np.float16), y_ptr=np.zeros((4, 4), np.float16))
    exp = np.zeros((4, 4), np.float16)
    exp[:2, :2] = [[1, 2], [3, 4]]
    return _fn("sstore", "%p_ptr: index, %y_ptr: index", body), "sstore", kw, "y_ptr", exp


def upper_triangle_double():
    """Y[r, c] = 2 * X[r, c] on the upper triangle (c >= r), through a
    non-rectangular access_tile_set (coordinate list, 10 points)."""
    tri = "affine_set<(d0, d1) : (d0 >= 0, -d0 + 3 >= 0, d1 >= 0, -d1 + 3 >= 0, d1 - d0 >= 0)>"

    def t(name, view):
        return (f"    %{name} = ktdp.construct_access_tile %{view}[%c0, %c0] {{\n"
                f"      access_tile_set = {tri},\n      access_tile_order = {ID2}\n"
                f"    }} : memref<4x4xf16> -> !ktdp.access_tile<4x4xindex>")

    body = "\n".join([
        _view("X", "x_ptr", [4, 4], [4, 1], "f16"),
        _view("Y", "y_ptr", [4, 4], [4, 1], "f16"),
        "    %c0 = arith.constant 0 : index",
        t("xt", "X"), t("yt", "Y"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<4x4xindex> -> tensor<10xf16>",
        "    %two = arith.constant 2.0 : f16",
        "    %tt = tensor.splat %two : tensor<10xf16>",
        "    %w = arith.mulf %v, %tt : tensor<10xf16>",
        "    ktdp.store %w, %yt : tensor<10xf16>, !ktdp.access_tile<4x4xindex>",
    ])
    x = np.arange(16, dtype=np.float16).reshape(4, 4)
    exp = x.copy()
    for r in range(4):
        for c in range(r, 4):
            exp[r, c] = x[r, c] * 2
    kw = dict(x_ptr=x, y_ptr=x.copy())
    return _fn("tri", "%x_ptr: index, %y_ptr: index", body), "tri", kw, "y_ptr", exp


def transposed_order():
    """access_tile_order (d1, d0): the loaded tile is X transposed."""
    body = "\n".join([
        _view("X", "x_ptr", [3, 3], [3, 1], "f16"),
        _view("Y", "y_ptr", [3, 3], [3, 1], "f16"),
        "    %c0 = arith.constant 0 : index",
        "    %xt = ktdp.construct_access_tile %X[%c0, %c0] {\n"
        "      access_tile_set = affine_set<(d0, d1) : (d0 >= 0, -d0 + 2 >= 0, d1 >= 0, -d1 + 2 >= 0)>,\n"
        "      access_tile_order = affine_map<(d0, d1) -> (d1, d0)>\n"
        "    } : memref<3x3xf16> -> !ktdp.access_tile<3x3xindex>",
        _tile("yt", "Y", ["%c0", "%c0"], [3, 3], [3, 3], "f16"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<3x3xindex> -> tensor<3x3xf16>",
        "    ktdp.store %v, %yt : tensor<3x3xf16>, !ktdp.access_tile<3x3xindex>",
    ])
    x = np.arange(9, dtype=np.float16).reshape(3, 3)
    kw = dict(x_ptr=x, y_ptr=np.zeros((3, 3), np.float16))
    return _fn("tord", "%x_ptr: index, %y_ptr: index", body), "tord", kw, "y_ptr", x.T.copy()


def reduce_sum(init=0.0):
    """out[0] = init + sum(x) over a 1x4 tile: 10, and 110 with init 100."""
    body = "\n".join([
        _view("X", "x_ptr", [1, 4], [4, 1], "f32"),
        _view("O", "o_ptr", [1], [1], "f32"),
        "    %c0 = arith.constant 0 : index",
        _tile("xt", "X", ["%c0", "%c0"], [1, 4], [1, 4], "f32"),
        _tile("ot", "O", ["%c0"], [1], [1], "f32"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<1x4xindex> -> tensor<1x4xf32>",
        f"    %init = arith.constant {float(init)} : f32",
        "    %acc = tensor.splat %init : tensor<1xf32>",
        "    %s = linalg.reduce { arith.addf } ins(%v : tensor<1x4xf32>) outs(%acc : tensor<1xf32>) dimensions = [1]",
        "    ktdp.store %s, %ot : tensor<1xf32>, !ktdp.access_tile<1xindex>",
    ])
    kw = dict(x_ptr=np.array([[1, 2, 3, 4]], np.float32), o_ptr=np.zeros(1, np.float32))
    return (_fn("rsum", "%x_ptr: index, %o_ptr: index", body), "rsum", kw, "o_ptr",
            np.array([10.0 + init], np.float32))


def overread_zero_pad():
    """Load 8 elements starting 2 before the end of a 6-element tensor: the
    two in range are read, the rest read as zero."""
    body = "\n".join([
        _view("X", "x_ptr", [8], [1], "f16"),
        _view("Y", "y_ptr", [8], [1], "f16"),
        "    %c0 = arith.constant 0 : index",
        "    %c4 = arith.constant 4 : index",
        _tile("xt", "X", ["%c4"], [8], [8], "f16"),
        _tile("yt", "Y", ["%c0"], [8], [8], "f16"),
        "    %v = ktdp.load %xt : !ktdp.access_tile<8xindex> -> tensor<8xf16>",
        "    ktdp.store %v, %yt : tensor<8xf16>, !ktdp.access_tile<8xindex>",
    ])
    x = np.arange(1, 7, dtype=np.float16)
    kw = dict(x_ptr=x, y_ptr=np.full(8, 7, np.float16))
    exp = np.array([5, 6, 0, 0, 0, 0, 0, 0], np.float16)
    return _fn("pad", "%x_ptr: index, %y_ptr: index", body), "pad", kw, "y_ptr", exp


def overwrite_truncate():
    """Store 8 elements starting 2 before the end of a 6-element tensor: only
    the two in range are written; the next tensor is untouched."""
    body = "\n".join([
        _view("S", "s_ptr", [8], [1], "f16"),
        _view("Y", "y_ptr", [8], [1], "f16"),
        "    %c0 = arith.constant 0 : index",
        "    %c4 = arith.constant 4 : index",
        _tile("st", "S", ["%c0"], [8], [8], "f16"),
        _tile("yt", "Y", ["%c4"], [8], [8], "f16"),
        "    %v = ktdp.load %st : !ktdp.access_tile<8xindex> -> tensor<8xf16>",
        "    ktdp.store %v, %yt : tensor<8xf16>, !ktdp.access_tile<8xindex>",
    ])
    s = np.arange(10, 18, dtype=np.float16)
    kw = dict(s_ptr=s, y_ptr=np.zeros(6, np.float16), z_ptr=np.full(8, 3, np.float16))
    exp = np.array([0, 0, 0, 0, 10, 11], np.float16)
    return (_fn("trunc", "%s_ptr: index, %y_ptr: index, %z_ptr: index", body), "trunc", kw, "y_ptr", exp)


def lx_matmul_loop():
    """K loop of a 512x256 f16 accumulator over 512x64 @ 64x256 products,
    with a tensor.empty outs and an arith.addf accumulate: the reference's
    LX accounting (last-use freeing on) peaks at 622592 bytes per core,
    accumulator 256 KiB + A 64 KiB + B 32 KiB + outs 256 KiB
    (reference tests/test_lx_scoping.py:1095-1185)."""
    M, N, K, BK = 512, 256, 256, 64
    T = lambda sh: _t(sh, "f16")
    body = "\n".join([
        "    %pm, %pn = ktdp.get_compute_tile_id : index, index",
        _view("A", "a_ptr", [M, K], [K, 1], "f16"),
        _view("B", "b_ptr", [K, N], [N, 1], "f16"),
        _view("C", "c_ptr", [M, N], [N, 1], "f16"),
        "    %c0 = arith.constant 0 : index",
        f"    %kk = arith.constant {K} : index",
        f"    %bk = arith.constant {BK} : index",
        f"    %z = arith.constant dense<0.0> : {T([M, N])}",
        f"    %c = scf.for %k = %c0 to %kk step %bk iter_args(%acc = %z) -> ({T([M, N])}) {{",
        _tile("at", "A", ["%pm", "%k"], [M, BK], [M, K], "f16", "      "),
        _tile("bt", "B", ["%k", "%pn"], [BK, N], [K, N], "f16", "      "),
        f"      %a = ktdp.load %at : !ktdp.access_tile<{M}x{BK}xindex> -> {T([M, BK])}",
        f"      %b = ktdp.load %bt : !ktdp.access_tile<{BK}x{N}xindex> -> {T([BK, N])}",
        f"      %e = tensor.empty() : {T([M, N])}",
        f"      %p = linalg.matmul ins(%a, %b : {T([M, BK])}, {T([BK, N])}) outs(%e : {T([M, N])}) -> {T([M, N])}",
        f"      %n = arith.addf %acc, %p : {T([M, N])}",
        f"      scf.yield %n : {T([M, N])}",
        "    }",
        _tile("ct", "C", ["%pm", "%pn"], [M, N], [M, N], "f16"),
        f"    ktdp.store %c, %ct : {T([M, N])}, !ktdp.access_tile<{M}x{N}xindex>",
    ])
    rng = np.random.default_rng(3)
    kw = dict(a_ptr=rng.random((M, K)).astype(np.float16), b_ptr=rng.random((K, N)).astype(np.float16),
              c_ptr=np.zeros((M, N), np.float16))
    return _fn("lx_mm", "%a_ptr: index, %b_ptr: index, %c_ptr: index", body), "lx_mm", kw, 622592


ALL = {
    "indirect_gather": indirect_gather,
    "indirect_scatter": indirect_scatter,
    "indirect_scatter_collision": lambda: indirect_scatter(True),
    "subtile_load": subtile_load,
    "strided_store": strided_store,
    "upper_triangle": upper_triangle_double,
    "transposed_order": transposed_order,
    "reduce_sum": reduce_sum,
    "reduce_sum_init": lambda: reduce_sum(100.0),
    "overread_zero_pad": overread_zero_pad,
    "overwrite_truncate": overwrite_truncate,
}
