"""Distributed memory views and per-core LX (ct_local) on the GPU.

The same kernels and seeds as the oracle tests beside them: partitions in
HBM (seeded at literal sticks through ``memory.hbm``) or in core 0's LX
(seeded through ``memory.get_lx(0)``), loads and stores through access
tiles of the distributed view, and a two-core kernel whose result depends on
core order through LX (reference ``ops/memory_ops.py:986-1259``,
``tests/test_distributed_view.py:207-470``).
"""
import numpy as np
import pytest

from tests import _cases
from tests.test_distributed_views import (FULL, _blocks, _expected, _full192, expected_store_images,
                                          oracle_dist_copy, oracle_dist_rows, oracle_dist_store,
                                          oracle_lx_exchange, store_input, store_seeds)

pytestmark = pytest.mark.gpu


def _seeded(src, seed_fn):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    interp = KTIRInterpreter()
    interp.load(src)
    orig = interp._prepare_execution

    def prepare_and_seed(grid):
        orig(grid)
        seed_fn(interp.memory)

    interp._prepare_execution = prepare_and_seed
    return interp


def _put(mem, sp, addr, buf):
    """Element address `addr` (f16) in HBM or core 0's LX."""
    if sp == "HBM":
        stick, intra = divmod(addr * 2, 128)
        mem.hbm.write(stick, buf, intra_byte=intra)
    else:
        mem.get_lx(0).write(addr * 2, buf)


def _get(mem, sp, addr, n):
    if sp == "HBM":
        stick, intra = divmod(addr * 2, 128)
        return mem.hbm.read(stick, n, "f16", intra_byte=intra)
    return mem.get_lx(0).read(addr * 2, n, "f16")


@pytest.mark.parametrize("case", _cases.DIST_CASES, ids=[c[0] for c in _cases.DIST_CASES])
def test_distributed_load(case):
    name, p0, p1, ashape, idx = case
    print(f"[dist] load {name}", flush=True)
    n = ashape[0] * ashape[1]

    def seed(mem):
        for sp, addr, buf in _blocks(p0, p1):
            _put(mem, sp, addr, buf)
        _put(mem, "HBM", _cases.DIST_OUT, np.zeros(n, np.float16))

    interp = _seeded(_cases.dist_copy(p0, p1, ashape, idx), seed)
    interp.execute_function("dist_copy")
    got = _get(interp.memory, "HBM", _cases.DIST_OUT, n).reshape(ashape)
    np.testing.assert_array_equal(got, _expected(ashape, idx))
    np.testing.assert_array_equal(got, oracle_dist_copy(p0, p1, ashape, idx))


@pytest.mark.parametrize("case", _cases.DIST_CASES, ids=[c[0] for c in _cases.DIST_CASES])
def test_distributed_store(case):
    name, p0, p1, ashape, idx = case
    print(f"[dist] store {name}", flush=True)
    seeds = store_seeds(p0, p1)

    def seed(mem):
        for sp, addr, buf in seeds:
            _put(mem, sp, addr, buf)
        _put(mem, "HBM", _cases.DIST_IN, store_input(ashape).reshape(-1))

    interp = _seeded(_cases.dist_store(p0, p1, ashape, idx), seed)
    interp.execute_function("dist_store")
    got = [_get(interp.memory, sp, addr, buf.size) for sp, addr, buf in seeds]
    for g, want, orc in zip(got, expected_store_images(p0, p1, ashape, idx), oracle_dist_store(p0, p1, ashape, idx)):
        np.testing.assert_array_equal(g, want)
        np.testing.assert_array_equal(g, orc)


def test_distributed_ct_id_routing_two_cores():
    """Core 1's rows come from core 0's LX (ct_id = 0) and its own (ct_id = 1)."""
    print("[dist] ct_id routing", flush=True)
    full = _full192()

    def seed(mem):
        mem.hbm.write(0, full[:96].reshape(-1))
        mem.get_lx(0).write(12288 * 2, _cases.strided_block(full[96:128], (1, 32)))
        mem.get_lx(1).write(16384 * 2, full[128:].reshape(-1))
        mem.hbm.write(24576 * 2 // 128, np.zeros(192 * 64, np.float16))

    interp = _seeded(_cases.dist_copy_2core(), seed)
    interp.execute_function("dist_rows")
    got = interp.memory.hbm.read(24576 * 2 // 128, 192 * 64, "f16").reshape(192, 64)
    np.testing.assert_array_equal(got, full)
    np.testing.assert_array_equal(got, oracle_dist_rows())


def test_lx_exchange_keeps_core_order():
    """Core 0 stores into core 1's LX before core 1 loads it (reference core
    order): the hazard check must see the shared LX bytes and run the cores
    in order.  Both LX scratchpads read back after the run."""
    print("[dist] lx exchange", flush=True)
    n = 256
    want_out, want_lx1, s0, s1 = oracle_lx_exchange(n)

    def seed(mem):
        mem.get_lx(0).write(0, s0)
        mem.get_lx(1).write(0, s1)
        mem.hbm.write(4096 * 2 // 128, np.zeros(2 * n, np.float16))

    interp = _seeded(_cases.lx_exchange(n), seed)
    interp.execute_function("lx_exchange")
    out = interp.memory.hbm.read(4096 * 2 // 128, 2 * n, "f16")
    np.testing.assert_array_equal(out, want_out)
    np.testing.assert_array_equal(out, np.concatenate([s0, s0]))
    np.testing.assert_array_equal(interp.memory.get_lx(1).read(0, n, "f16"), want_lx1)
    np.testing.assert_array_equal(interp.memory.get_lx(0).read(0, n, "f16"), s0)
    assert interp.last_plan.mode == "sequential"


def test_lx_access_past_capacity_is_refused():
    """An LX view reaching past the scratchpad's capacity raises instead of
    touching another core's bytes."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src = _cases.lx_exchange(256).replace("%c0 = arith.constant 0 : index",
                                          "%c0 = arith.constant 0 : index\n    %far = arith.constant 1048500 : index")
    src = src.replace("%own = ktdp.construct_memory_view %c0", "%own = ktdp.construct_memory_view %far")
    interp = KTIRInterpreter()
    interp.load(src)
    with pytest.raises(NotImplementedError):
        interp.execute_function("lx_exchange")
