"""Pins for the layer the oracle shares with the product: the affine
evaluator (maps, sets, their lowering to boxes) and the KTIR parser.

Both sides of every GPU-vs-oracle test read the kernel through
``ktir_cpu_amd.parser`` and evaluate its index maps through
``ktir_cpu_amd.affine``, so a bug there would be invisible to those tests.
Here that layer is checked against things it does not compute itself:
MLIR's integer semantics written from their definitions (floor and ceiling
of exact rationals, a non-negative remainder), brute-force enumeration of
set members, and the structure of small kernels written out by hand
(reference ``affine.py:294-507``, ``parser_ast.py:440-461``, ``parser.py:85-147``).
"""
import itertools
import math
from fractions import Fraction

import pytest

from ktir_cpu_amd import configs
from ktir_cpu_amd.affine import Box, AffineSet, box_from_set, parse_affine_map, parse_affine_set, parse_affine_set_raw
from ktir_cpu_amd.ir import ShapedType, iter_ops
from ktir_cpu_amd.parser import KTIRParser


def floordiv(a, b):
    return math.floor(Fraction(a, b))


def ceildiv(a, b):
    return math.ceil(Fraction(a, b))


def mod(a, b):
    # MLIR: the remainder of floor division, in [0, b) for b > 0
    r = a - b * floordiv(a, b)
    assert 0 <= r < b
    return r


PTS = range(-7, 8)


@pytest.mark.parametrize("text,ref", [
    # precedence: * and floordiv / ceildiv / mod bind tighter than + and -
    ("affine_map<(d0, d1) -> (d0 + d1 * 3, d0 * 2 - d1)>",
     lambda i, j, s: (i + 3 * j, 2 * i - j)),
    ("affine_map<(d0, d1) -> (d0 floordiv 4, d1 ceildiv 3, d0 mod 5)>",
     lambda i, j, s: (floordiv(i, 4), ceildiv(j, 3), mod(i, 5))),
    ("affine_map<(d0, d1) -> ((d0 + d1) mod 3, d0 + d1 mod 3, -d0 + 5)>",
     lambda i, j, s: (mod(i + j, 3), i + mod(j, 3), 5 - i)),
    ("affine_map<(d0, d1)[s0] -> (d0 * 4 + s0, (d1 - s0) floordiv 2, s0 * 2 - d1 ceildiv 4)>",
     lambda i, j, s: (4 * i + s, floordiv(j - s, 2), 2 * s - ceildiv(j, 4))),
    ("affine_map<(d0, d1) -> (d1, d0)>", lambda i, j, s: (j, i)),
])
def test_affine_map_integer_semantics(text, ref):
    """Every map on a grid that includes negative operands, where truncating
    division or a C-style remainder would differ from MLIR's."""
    m = parse_affine_map(text)
    for i, j in itertools.product(PTS, PTS):
        for s in ((-3, 2) if m.n_syms else (0,)):
            syms = (s,) if m.n_syms else ()
            assert m.eval((i, j), syms) == ref(i, j, s), (text, i, j, s)


def test_affine_map_permutation_detection():
    assert parse_affine_map("affine_map<(d0, d1, d2) -> (d2, d0, d1)>").permutation() == (2, 0, 1)
    assert parse_affine_map("affine_map<(d0, d1) -> (d0, d1)>").is_identity()
    # not permutations: a scaled dim, a repeated dim, an offset, a dropped dim
    for t in ("affine_map<(d0, d1) -> (d1 * 2, d0)>", "affine_map<(d0, d1) -> (d0, d0)>",
              "affine_map<(d0, d1) -> (d1 + 1, d0)>", "affine_map<(d0, d1) -> (d1)>"):
        assert parse_affine_map(t).permutation() is None, t


SETS = [
    ("affine_set<(d0, d1) : (d0 >= 0, -d0 + 5 >= 0, d1 - d0 >= 0, -d1 + 6 >= 0)>", 0,
     lambda i, j, s: 0 <= i <= 5 and i <= j <= 6),
    ("affine_set<(d0, d1) : ((d0 - d1) mod 3 == 0, d0 >= 0, d1 >= 0, -d0 + 8 >= 0, -d1 + 8 >= 0)>", 0,
     lambda i, j, s: (i - j) % 3 == 0 and 0 <= i <= 8 and 0 <= j <= 8),
    ("affine_set<(d0, d1)[s0] : (d0 - s0 >= 0, -d0 + s0 + 3 >= 0, d1 floordiv 3 <= 1, d1 >= 0)>", 1,
     lambda i, j, s: s <= i <= s + 3 and floordiv(j, 3) <= 1 and j >= 0),
    ("affine_set<(d0, d1) : (d0 == 2, d1 * 2 - 3 >= 0, -d1 + 4 >= 0)>", 0,
     lambda i, j, s: i == 2 and 2 * j >= 3 and j <= 4),
]


@pytest.mark.parametrize("text,n_syms,ref", SETS)
def test_affine_set_membership_against_brute_force(text, n_syms, ref):
    """contains, the vectorised mask and enumerate agree with the constraints
    evaluated point by point."""
    aset = parse_affine_set_raw(text)
    for s in ((1, 4) if n_syms else (0,)):
        syms = (s,) if n_syms else ()
        want = [(i, j) for i in range(10) for j in range(10) if ref(i, j, s)]
        assert aset.enumerate((10, 10), syms) == want
        for i, j in itertools.product(range(-3, 12), range(-3, 12)):
            assert aset.contains((i, j), syms) == ref(i, j, s), (text, i, j, s)


@pytest.mark.parametrize("text,syms,lo,hi", [
    ("affine_set<(d0, d1) : (d0 >= 0, -d0 + 5 >= 0, d1 - 2 >= 0, -d1 + 6 >= 0)>", (), (0, 2), (6, 7)),
    # repeated bounds combine to the tightest; an equality pins one point
    ("affine_set<(d0, d1) : (d0 - 1 >= 0, d0 - 3 >= 0, -d0 + 9 >= 0, -d0 + 7 >= 0, d1 == 4)>", (), (3, 4), (8, 5)),
    # bounds written with <= and a symbol
    ("affine_set<(d0)[s0] : (d0 >= s0, d0 <= s0 + 15)>", (32,), (32,), (48,)),
])
def test_box_lowering_matches_enumerated_members(text, syms, lo, hi):
    """An axis-aligned set lowers to a Box whose points are exactly the set's
    members (enumerated over a bounding grid), with the expected bounds."""
    b = parse_affine_set(text)
    assert isinstance(b, Box)
    b = b.specialize(syms) if not b.is_concrete else b
    assert (b.lo, b.hi) == (lo, hi)
    raw = parse_affine_set_raw(text)
    shape = tuple(h + 2 for h in hi)
    assert b.enumerate(shape) == raw.enumerate(shape, syms)


def test_non_axis_aligned_sets_stay_sets():
    for t in ("affine_set<(d0, d1) : (d1 - d0 >= 0, d0 >= 0, -d1 + 6 >= 0)>",
              "affine_set<(d0) : (d0 mod 2 == 0, d0 >= 0, -d0 + 6 >= 0)>",
              "affine_set<(d0) : (d0 * 2 >= 0, -d0 + 6 >= 0)>",
              "affine_set<(d0) : (d0 >= 0)>"):                  # unbounded above
        assert not isinstance(parse_affine_set(t), Box), t
    # an empty axis-aligned set is not lowered to an empty box
    assert box_from_set(parse_affine_set_raw("affine_set<(d0) : (d0 - 5 >= 0, -d0 + 2 >= 0)>")) is None


def test_parser_structure_of_a_loop_kernel():
    """The vector_add kernel with two blocks per core, read back: arguments,
    grid, views, the scf.for region and every op's operands and types."""
    m = KTIRParser().parse_module(configs.vector_add(n=8192, block=128, cores=32))
    f = m.get_function("add_kernel")
    assert f.arg_names == ["x_ptr", "y_ptr", "output_ptr", "BLOCK_SIZE"]
    assert f.grid == (32, 1, 1) and f.num_cores == 32
    assert f.tensor_sizes == {p: {"shape": (8192,), "dtype": "f16"} for p in ("x_ptr", "y_ptr", "output_ptr")}
    top = [op.op_type for op in f.operations]
    assert top == ["ktdp.get_compute_tile_id"] + ["ktdp.construct_memory_view"] * 3 + \
        ["arith.constant"] * 3 + ["arith.muli", "scf.for", "return"]
    consts = [op.attributes["value"] for op in f.operations if op.op_type == "arith.constant"]
    assert consts == [0, 1, 2]
    loop = next(op for op in f.operations if op.op_type == "scf.for")
    assert loop.operands == ["%c0", "%bpc", "%c1"] and loop.attributes["iter_var"] == "%b"
    body = loop.regions[0].ops
    assert [op.op_type for op in body] == [
        "arith.addi", "arith.muli", "ktdp.construct_access_tile", "ktdp.construct_access_tile",
        "ktdp.load", "ktdp.load", "arith.addf", "ktdp.construct_access_tile", "ktdp.store", "scf.yield"]
    add = next(op for op in body if op.op_type == "arith.addf")
    assert add.operands == ["%x", "%y"] and add.results == ["%output"]
    assert add.result_types == [ShapedType("tensor", (128,), "f16")]
    tile = next(op for op in body if op.op_type == "ktdp.construct_access_tile")
    assert tile.operands == ["%x_view", "%offset"] and tile.attributes["shape"] == (128,)
    assert (tile.attributes["coordinate_set"].lo, tile.attributes["coordinate_set"].hi) == ((0,), (128,))
    store = next(op for op in body if op.op_type == "ktdp.store")
    assert store.operands == ["%output", "%out_tile"]
    # every SSA value used is defined earlier or is an argument / loop variable
    defined = {f"%{a}" for a in f.arg_names} | {"%b"}
    for op in iter_ops(f.operations):
        for x in op.operands:
            assert x in defined, (op.op_type, x)
        defined.update(op.results)


def test_parser_reads_2d_views_and_multi_dim_tiles():
    """The RMSNorm kernel: 2-D memory views with row strides, and tiles whose
    sets and orders are 2-D."""
    m = KTIRParser().parse_module(configs.rmsnorm(rows=64, cols=256, cores=8, rblk=8, dt="f16"))
    (f,) = m.functions.values()
    views = [op for op in iter_ops(f.operations) if op.op_type == "ktdp.construct_memory_view"]
    assert views and all(op.attributes["shape"][-1] == 256 for op in views if len(op.attributes["shape"]) == 2)
    two_d = [op for op in views if len(op.attributes["shape"]) == 2]
    assert two_d and all(op.attributes["strides"] == [256, 1] for op in two_d)
    tiles = [op for op in iter_ops(f.operations) if op.op_type == "ktdp.construct_access_tile"]
    for op in tiles:
        cs = op.attributes["coordinate_set"]
        shape = op.attributes["shape"]
        if isinstance(cs, Box):
            assert cs.extent == tuple(shape), (cs, shape)
