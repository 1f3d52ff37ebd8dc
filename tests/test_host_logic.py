"""Host-side logic of the executor that needs no GPU: the cross-lane hazard
check, view reshapes, lane offsets, and the oracle's pairwise-halving fold."""
import numpy as np
import pytest

from ktir_cpu_amd.executor import Access, Alloc, Instances, verify
from ktir_cpu_amd.program import LaneOff
from ktir_cpu_amd.walker import _reshape_strides


def _acc(alloc, store, inst, base, shape=(2, 2), strides=(8, 1), **kw):
    return Access(alloc, store, np.asarray(inst, np.int64), np.asarray(base, np.int64), shape, strides, **kw)


def test_verify_disjoint_tiles_pass():
    a = Alloc("y", "f16", 0x10000, 128, (8, 8))
    ins = Instances(4)
    # 4 cores each storing its own 2x2 tile of an 8x8 tensor (grid-aligned)
    acc = [_acc(a, True, [0, 1, 2, 3], [0, 2, 16, 18])]
    assert verify(acc, ins) is None


def test_verify_overlapping_stores_fail():
    a = Alloc("y", "f16", 0x10000, 128, (8, 8))
    ins = Instances(2)
    acc = [_acc(a, True, [0, 1], [0, 0])]
    assert verify(acc, ins) is not None


def test_verify_read_after_write_across_cores_fails():
    a = Alloc("y", "f16", 0x10000, 128, (8, 8))
    ins = Instances(2)
    acc = [_acc(a, True, [0, 1], [0, 2]), _acc(a, False, [0, 1], [2, 0])]
    assert verify(acc, ins) is not None


def test_verify_same_lane_in_place_update_passes():
    a = Alloc("y", "f16", 0x10000, 128, (8, 8))
    ins = Instances(2)
    acc = [_acc(a, False, [0, 1], [0, 2]), _acc(a, True, [0, 1], [0, 2])]
    assert verify(acc, ins) is None


def test_verify_loop_iterations_are_instances():
    a = Alloc("y", "f16", 0x10000, 128, (8, 8))
    ins = Instances(1)
    it = ins.new(np.array([0, 0]))           # two iterations of core 0
    # both iterations store the same tile: a loop-carried dependence through HBM
    acc = [_acc(a, True, it, [0, 0])]
    assert verify(acc, ins) is not None
    # a core-level access and its own iterations are ordered (ancestor chain)
    acc = [_acc(a, True, [0], [0]), _acc(a, False, it[:1], [0])]
    assert verify(acc, ins) is None


def test_verify_data_dependent_store_needs_one_lane():
    a = Alloc("y", "f16", 0x10000, 128, (8, 8))
    ins = Instances(2)
    assert verify([_acc(a, True, [0, 1], [0, 0], whole=True)], ins) is not None
    assert verify([_acc(a, True, [0], [0], whole=True)], ins) is None
    # an internally ordered fused launch is accepted
    assert verify([_acc(a, True, [0, 1], [0, 0], whole=True, group=7)], ins) is None


def _brute_conflict(bases, stores, inst, shape, strides):
    cells = []
    for b in bases:
        idx = np.indices(shape).reshape(len(shape), -1)
        cells.append(set((b + np.tensordot(np.asarray(strides), idx, 1)).tolist()))
    for i in range(len(bases)):
        for j in range(i + 1, len(bases)):
            if inst[i] != inst[j] and (stores[i] or stores[j]) and cells[i] & cells[j]:
                return True
    return False


@pytest.mark.parametrize("seed", range(40))
def test_verify_unaligned_equal_tiles_exact(seed):
    """Equal tiles at arbitrary (not shape-aligned) starts: verify flags a
    conflict exactly when two lanes' element sets meet and one of them
    stores, checked by brute force on the element sets."""
    rng = np.random.default_rng(seed)
    shape = (2, 3) if seed % 2 else (2, 3, 4)
    vshape = (12, 9) if seed % 2 else (6, 5, 8)
    strides = tuple(int(np.prod(vshape[d + 1:])) for d in range(len(vshape)))
    n = int(rng.integers(2, 6))
    starts = [tuple(int(rng.integers(0, v - s + 1)) for v, s in zip(vshape, shape)) for _ in range(n)]
    bases = [int(np.dot(st, strides)) for st in starts]
    stores = [bool(rng.integers(0, 2)) or k == 0 for k in range(n)]
    a = Alloc("y", "f16", 0x10000, 2 * int(np.prod(vshape)), vshape)
    ins = Instances(n)
    acc = [_acc(a, st, [k], [b], shape=shape, strides=strides) for k, (b, st) in enumerate(zip(bases, stores))]
    want = _brute_conflict(bases, stores, list(range(n)), shape, strides)
    assert (verify(acc, ins) is not None) == want


def test_verify_unaligned_row_pairs_pass():
    """Tiles of 2 rows x 4 heads starting at row 9 (an odd batch start), the
    shape of the paged attention output store: disjoint, so accepted."""
    a = Alloc("o", "f16", 0x10000, 2 * 20 * 32 * 128, (20, 32, 128))
    ins = Instances(32)
    bases = [(9 + 2 * p0) * 4096 + 4 * p1 * 128 for p0 in range(4) for p1 in range(8)]
    acc = [_acc(a, True, list(range(32)), bases, shape=(2, 4, 128), strides=(4096, 128, 1))]
    assert verify(acc, ins) is None


@pytest.mark.parametrize("strides,old,new,expect", [
    ((8192 * 128, 128, 1), (1, 128, 128), (128, 128), (128, 1)),
    ((4096, 1), (8, 4096), (8 * 4096,), (1,)),
    ((4096, 1), (8, 16), (128,), None),                 # rows not contiguous
    ((1,), (128,), (1, 128), (0, 1)),
    ((64, 1), (4, 64), (2, 2, 64), (128, 64, 1)),
])
def test_reshape_strides(strides, old, new, expect):
    assert _reshape_strides(strides, old, new) == expect


@pytest.mark.parametrize("strides,old,new,expect", [
    ((1, 0), (8, 128), (2, 4, 128), (4, 1, 0)),        # a row-broadcast leaf split by rows
    ((0, 1), (8, 128), (2, 4, 128), (0, 0, 1)),        # a column-broadcast leaf
    ((0, 1), (4, 8), (32,), None),                     # broadcast rows do not merge
    ((24, 4, 1), (2, 6, 4), (2, 3, 8), (24, 8, 1)),    # split 6 and merge with the contiguous 4
])
def test_reshape_strides_split_groups(strides, old, new, expect):
    assert _reshape_strides(strides, old, new) == expect


def test_reshape_strides_against_brute_force():
    """Every reshape the function expresses lands on the same element
    offsets as NumPy's row-major reshape of the view's offset array, over
    random shapes and strides (contiguous, padded, broadcast and permuted)."""
    rng = np.random.default_rng(5)
    factor = {4: [(4,), (2, 2), (1, 4, 1)], 6: [(6,), (2, 3), (3, 2)], 8: [(8,), (2, 4), (4, 2), (2, 2, 2)],
              12: [(12,), (3, 4), (2, 6), (2, 2, 3)]}
    found = 0
    for _ in range(3000):
        dims = [int(rng.choice(list(factor))) for _ in range(int(rng.integers(1, 4)))]
        old = tuple(x for d in dims for x in factor[d][int(rng.integers(len(factor[d])))])
        new = tuple(x for d in dims for x in factor[d][int(rng.integers(len(factor[d])))])
        kind = int(rng.integers(4))
        st, acc = [], 1
        for n in reversed(old):
            st.append(acc)
            acc *= n + (1 if kind == 1 else 0)
        st = list(reversed(st))
        if kind == 2:
            st[int(rng.integers(len(st)))] = 0
        if kind == 3:
            st = list(rng.permutation(st))
        offs = np.zeros(old, np.int64)
        for ax, (n, t) in enumerate(zip(old, st)):
            sh = [1] * len(old)
            sh[ax] = n
            offs = offs + (np.arange(n) * t).reshape(sh)
        got = _reshape_strides(tuple(st), old, new)
        if got is None:
            continue
        found += 1
        mine = np.zeros(new, np.int64)
        for ax, (n, t) in enumerate(zip(new, got)):
            sh = [1] * len(new)
            sh[ax] = n
            mine = mine + (np.arange(n) * t).reshape(sh)
        np.testing.assert_array_equal(mine, offs.reshape(new))
    assert found > 1000


def test_lane_offsets_affine_detection():
    lo = LaneOff.from_array(np.array([4, 12, 20, 28]))
    assert lo.arr is None and (lo.base, lo.stride) == (4, 8)
    lo = LaneOff.from_array(np.array([0, 128, 0, 128]))
    assert lo.arr is not None
    np.testing.assert_array_equal(lo.take(np.array([1, 3])).values(2), [128, 128])


def _tree_fold_reference(x):
    """Brute-force restatement of pairwise halving with odd-tail carry on a list."""
    acc = list(x)
    while len(acc) > 1:
        half = len(acc) // 2
        nxt = [acc[i] + acc[i + half] for i in range(half)]
        if len(acc) % 2:
            nxt.append(acc[-1])
        acc = nxt
    return acc[0]


@pytest.mark.parametrize("n", [1, 2, 3, 5, 7, 8, 13, 64, 100])
def test_oracle_tree_fold_order(n):
    """The oracle's linalg.reduce follows the pairwise-halving order exactly
    (f16 data, where the order changes the rounding)."""
    from oracle.interp import OracleInterpreter
    from ktir_cpu_amd.configs import _tile, _view
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 100).astype(np.float16)
    src = ("module {\n  func.func @f(%x_ptr: index, %o_ptr: index) attributes {grid = [1, 1]} {\n"
           + _view("X", "x_ptr", [1, n], [n, 1], "f16") + "\n" + _view("O", "o_ptr", [1], [1], "f16") + "\n"
           "    %c0 = arith.constant 0 : index\n"
           + _tile("xt", "X", ["%c0", "%c0"], [1, n], [1, n], "f16") + "\n"
           + _tile("ot", "O", ["%c0"], [1], [1], "f16") + "\n"
           f"    %v = ktdp.load %xt : !ktdp.access_tile<1x{n}xindex> -> tensor<1x{n}xf16>\n"
           "    %z = arith.constant 0.0 : f16\n    %acc = tensor.splat %z : tensor<1xf16>\n"
           f"    %s = linalg.reduce {{ arith.addf }} ins(%v : tensor<1x{n}xf16>) outs(%acc : tensor<1xf16>) dimensions = [1]\n"
           "    ktdp.store %s, %ot : tensor<1xf16>, !ktdp.access_tile<1xindex>\n    return\n  }\n}\n")
    o = OracleInterpreter()
    o.load(src)
    out = o.execute_function("f", x_ptr=x, o_ptr=np.zeros(1, np.float16))
    expect = np.float16(_tree_fold_reference([np.float16(v) for v in x]) + np.float16(0))
    assert out["o_ptr"][0] == expect


def _gemm_leaves(tm, tn, K=256, T=128):
    """A and B leaves of a tm x tn grid of T x T matmul tiles over row-major
    A [tm*T, K] and B [K, tn*T], lanes in a shuffled order."""
    from ktir_cpu_amd.program import LeafSpec
    rng = np.random.default_rng(1)
    mi, ni = np.divmod(rng.permutation(tm * tn), tn)
    N = tn * T
    la = LeafSpec(0, "f16", LaneOff.from_array(mi * T * K), (K, 1), 0, tm * T * K)
    lb = LeafSpec(0, "f16", LaneOff.from_array(ni * T), (N, 1), 0, K * N)
    return la, lb, mi, ni


def test_mm_quads_groups_2x2():
    """Every group is {tl, tr, bl, br}: the right lane T columns right of the
    left one with the same A, the bottom lane T rows below with the same B."""
    from ktir_cpu_amd.walker import _mm_quads
    tm, tn = 6, 4
    la, lb, mi, ni = _gemm_leaves(tm, tn)
    q = _mm_quads(la, lb, tm * tn, 128, 128).reshape(-1, 4)
    assert sorted(q.ravel().tolist()) == list(range(tm * tn))
    for tl, tr, bl, br in q:
        assert (mi[tr], ni[tr]) == (mi[tl], ni[tl] + 1)
        assert (mi[bl], ni[bl]) == (mi[tl] + 1, ni[tl])
        assert (mi[br], ni[br]) == (mi[tl] + 1, ni[tl] + 1)
    la, lb, _, _ = _gemm_leaves(3, 4)           # odd tile rows: no grouping
    assert _mm_quads(la, lb, 12, 128, 128) is None


def test_mm_quads_xcd_blocks():
    """64 x 64 tiles = 32 x 32 groups: the kernel gives XCD x groups
    [128 x, 128 x + 128); round r of that XCD runs 32 of them, which must
    cover 4 group rows x 8 group columns."""
    from ktir_cpu_amd.walker import _mm_quads
    tm = tn = 64
    la, lb, mi, ni = _gemm_leaves(tm, tn)
    q = _mm_quads(la, lb, tm * tn, 128, 128).reshape(-1, 4)
    assert sorted(q.ravel().tolist()) == list(range(tm * tn))
    for x in range(8):
        for r in range(4):
            tl = q[128 * x + 32 * r:128 * x + 32 * r + 32, 0]
            assert len(set((mi[tl] // 2).tolist())) == 4 and len(set((ni[tl] // 2).tolist())) == 8


@pytest.mark.parametrize("seed", range(40))
def test_strides_injective_is_sufficient_against_brute_force(seed):
    """Whenever the store path's test says a box is injective, no two
    positions reach one element (brute force over small boxes); and the
    layouts that overlap (a row tile wider than the row stride, a zero
    stride) are reported as not injective."""
    from ktir_cpu_amd.walker import _strides_injective
    rng = np.random.default_rng(seed)
    nd = int(rng.integers(1, 4))
    shape = tuple(int(x) for x in rng.integers(1, 6, nd))
    strides = tuple(int(x) for x in rng.integers(-3, 40, nd))
    offs = [sum(i * s for i, s in zip(p, strides)) for p in np.ndindex(*shape)]
    if _strides_injective(shape, strides):
        assert len(set(offs)) == len(offs), (shape, strides)
    assert _strides_injective((64, 32), (32, 1)) and not _strides_injective((64, 32), (16, 1))
    assert not _strides_injective((4, 3), (0, 1)) and _strides_injective((1, 3), (0, 1))


def test_collapse_dims_keeps_every_element_offset():
    """A 5-d expression with a unit dim and mergeable dims compiles over <= 4
    dims: each leaf and the destination address the same elements, in the
    same flattened order, and linalg.index dims keep their values."""
    from ktir_cpu_amd.program import Expr, LeafSpec
    from ktir_cpu_amd.walker import _collapse_dims, _cstrides
    shape = (1, 4, 2, 4, 4)
    a = LeafSpec(0, "f32", LaneOff(0, 32), (0, 4, 16, 1, 0), 0, 1 << 20)
    g = LeafSpec(0, "f32", LaneOff(0, 128), _cstrides(shape), 0, 1 << 20)
    g.offsets = object()                       # an offset-list (gather) leaf
    dest = LeafSpec(0, "f32", LaneOff(0, 128), _cstrides(shape), 0, 1 << 20)
    e = Expr("bin", "f32", shape, [Expr("ld", "f32", shape, attr=a), Expr("ld", "f32", shape, attr=g)], 0)
    e = Expr("bin", "f32", shape, [e, Expr("idx", "i32", shape, attr=4)], 0)
    out = _collapse_dims(e, dest, 4)
    assert out is not None
    e2, d2 = out
    assert len(e2.shape) <= 4 and int(np.prod(e2.shape)) == int(np.prod(shape))
    pts_old = list(np.ndindex(*shape))
    pts_new = list(np.ndindex(*e2.shape))
    leaves = [n for n in [e2.args[0].args[0], e2.args[0].args[1]]]
    for old, new in zip((a, g, dest), (leaves[0].attr, leaves[1].attr, d2)):
        o = [sum(i * s for i, s in zip(p, old.strides)) for p in pts_old]
        n = [sum(i * s for i, s in zip(p, new.strides)) for p in pts_new]
        assert o == n
    idx = e2.args[1]
    assert idx.kind == "idx" and [p[idx.attr] for p in pts_new] == [p[4] for p in pts_old]
    # a linalg.index over a merged pair blocks that merge
    e3 = Expr("bin", "f32", (2, 3, 4, 5, 6), [Expr("idx", "i32", (2, 3, 4, 5, 6), attr=d) for d in (0, 1)], 0)
    d3 = LeafSpec(0, "f32", LaneOff(0, 720), _cstrides((2, 3, 4, 5, 6)), 0, 1 << 20)
    e4, _ = _collapse_dims(e3, d3, 4)
    assert e4.shape == (2, 3, 20, 6)          # merges only until the rank fits
