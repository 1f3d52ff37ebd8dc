"""Distributed memory views and per-core LX (ct_local) routing.

Pinned by the reference's own table (tests/test_distributed_view.py:207-470):
a 4 x 4 tensor arange(16) split into two partitions (HBM or LX, row-major or
column-packed), an access tile loaded from the distributed view and stored
to HBM must equal the tensor's slice.  The oracle is checked against those
slices on the CPU; the GPU path against the slices and the oracle.  A 2-core
kernel adds ct_id routing: core 1 reads core 0's LX.
"""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _cases

FULL = np.arange(16, dtype=np.float16).reshape(4, 4)


def _blocks(p0, p1):
    out = []
    for rows, cols, sp, st, addr in (p0, p1):
        blk = FULL[rows[0]:rows[1] + 1, cols[0]:cols[1] + 1]
        out.append((sp, addr, _cases.strided_block(blk, st)))
    return out


def _expected(ashape, idx):
    return FULL[idx[0]:idx[0] + ashape[0], idx[1]:idx[1] + ashape[1]]


def oracle_dist_copy(p0, p1, ashape, idx):
    o = OracleInterpreter()
    o.load(_cases.dist_copy(p0, p1, ashape, idx))

    def seed(o):
        for sp, addr, buf in _blocks(p0, p1):
            mem = o.hbm.memory if sp == "HBM" else o.lxs[0].memory
            mem.write(addr * 2, buf)
        o.hbm.memory.write(_cases.DIST_OUT * 2, np.zeros(ashape[0] * ashape[1], np.float16))
        o.lxs[0].next_ptr = 1 << 20      # keep loaded tiles clear of the seeded LX data
    o.prepare_hook = seed
    o.execute_function("dist_copy")
    return o.hbm.memory.read(_cases.DIST_OUT * 2, ashape[0] * ashape[1], "f16").reshape(ashape)


@pytest.mark.parametrize("case", _cases.DIST_CASES, ids=[c[0] for c in _cases.DIST_CASES])
def test_oracle_distributed_copy(case):
    _, p0, p1, ashape, idx = case
    np.testing.assert_array_equal(oracle_dist_copy(p0, p1, ashape, idx), _expected(ashape, idx))


def _full192():
    return np.arange(192 * 64, dtype=np.float16).reshape(192, 64)


def oracle_dist_rows():
    o = OracleInterpreter()
    o.load(_cases.dist_copy_2core())
    full = _full192()

    def seed(o):
        o.hbm.memory.write(0, full[:96].reshape(-1))
        o.lxs[0].memory.write(12288 * 2, _cases.strided_block(full[96:128], (1, 32)))
        o.lxs[1].memory.write(16384 * 2, full[128:].reshape(-1))
        o.hbm.memory.write(24576 * 2, np.zeros(192 * 64, np.float16))
        o.lxs[0].next_ptr = o.lxs[1].next_ptr = 1 << 20
    o.prepare_hook = seed
    o.execute_function("dist_rows")
    return o.hbm.memory.read(24576 * 2, 192 * 64, "f16").reshape(192, 64)


def test_oracle_distributed_ct_id_routing():
    np.testing.assert_array_equal(oracle_dist_rows(), _full192())


def test_oracle_distributed_view_rejects_wrong_extent():
    src = _cases.dist_copy(((0, 1), (0, 3), "HBM", (4, 1), 0), ((2, 3), (0, 3), "HBM", (4, 1), 4096),
                           (4, 4), (0, 0), gshape=(5, 4))
    o = OracleInterpreter()
    o.load(src)
    with pytest.raises(ValueError):
        o.execute_function("dist_copy")


BG = -(np.arange(16, dtype=np.float16) + 1).reshape(4, 4)


def store_input(ashape):
    return (100 + np.arange(ashape[0] * ashape[1])).astype(np.float16).reshape(ashape)


def expected_store_images(p0, p1, ashape, idx):
    """Each partition's memory image after the store: the background tensor
    with the access tile's region replaced by the input, laid out with the
    partition's strides (holes stay zero)."""
    g = BG.copy()
    g[idx[0]:idx[0] + ashape[0], idx[1]:idx[1] + ashape[1]] = store_input(ashape)
    return [_cases.strided_block(g[r[0]:r[1] + 1, c[0]:c[1] + 1], st) for r, c, _, st, _ in (p0, p1)]


def store_seeds(p0, p1):
    return [(sp, addr, _cases.strided_block(BG[r[0]:r[1] + 1, c[0]:c[1] + 1], st)) for r, c, sp, st, addr in (p0, p1)]


def oracle_dist_store(p0, p1, ashape, idx):
    o = OracleInterpreter()
    o.load(_cases.dist_store(p0, p1, ashape, idx))
    seeds = store_seeds(p0, p1)

    def seed(o):
        for sp, addr, buf in seeds:
            (o.hbm.memory if sp == "HBM" else o.lxs[0].memory).write(addr * 2, buf)
        o.hbm.memory.write(_cases.DIST_IN * 2, store_input(ashape).reshape(-1))
        o.lxs[0].next_ptr = 1 << 20
    o.prepare_hook = seed
    o.execute_function("dist_store")
    return [(o.hbm.memory if sp == "HBM" else o.lxs[0].memory).read(addr * 2, buf.size, "f16")
            for sp, addr, buf in seeds]


@pytest.mark.parametrize("case", _cases.DIST_CASES, ids=[c[0] for c in _cases.DIST_CASES])
def test_oracle_distributed_store(case):
    _, p0, p1, ashape, idx = case
    for got, want in zip(oracle_dist_store(p0, p1, ashape, idx), expected_store_images(p0, p1, ashape, idx)):
        np.testing.assert_array_equal(got, want)


def oracle_lx_exchange(n=256):
    s0 = np.arange(n, dtype=np.float16)
    s1 = -np.arange(n, dtype=np.float16) - 1
    o = OracleInterpreter()
    o.load(_cases.lx_exchange(n))

    def seed(o):
        o.lxs[0].memory.write(0, s0)
        o.lxs[1].memory.write(0, s1)
        o.hbm.memory.write(4096 * 2, np.zeros(2 * n, np.float16))
        o.lxs[0].next_ptr = o.lxs[1].next_ptr = 1 << 20
    o.prepare_hook = seed
    o.execute_function("lx_exchange")
    return o.hbm.memory.read(4096 * 2, 2 * n, "f16"), o.lxs[1].memory.read(0, n, "f16"), s0, s1


def test_oracle_lx_exchange_in_core_order():
    """Core 1 runs after core 0, so it loads the values core 0 stored into
    its LX: both HBM halves and core 1's LX end up holding core 0's data."""
    out, lx1, s0, _ = oracle_lx_exchange()
    np.testing.assert_array_equal(out, np.concatenate([s0, s0]))
    np.testing.assert_array_equal(lx1, s0)
