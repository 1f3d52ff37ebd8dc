"""ktir_launch_row_rmw_noalloc (the ordered row RMW with the library's own
scratch array) against ktir_launch_row_rmw (caller scratch): bit-identical
results on two calls in a row, the second on a smaller input, through the
C ABI."""
import ctypes as C

import numpy as np
import pytest

from tests import _cases

pytestmark = pytest.mark.gpu


def _prepared(rows, dim, n_idx, cores, chunk, hot, seed):
    """The gather + scatter-add kernel placed on the device and run once by
    the existing entry point; returns (keep-alive, prepared, descriptor, result)."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw = _cases.gather_scatter_add(rows=rows, dim=dim, n_idx=n_idx, cores=cores, chunk=chunk)
    rng = np.random.default_rng(seed)
    kw["idx_ptr"] = rng.integers(0, hot, n_idx).astype(np.int32)
    kw["out_ptr"] = rng.standard_normal((rows, dim)).astype(np.float32)
    g = KTIRInterpreter()
    g.load(src)
    prep = g.prepare(fn, **kw)
    ref = prep.outputs()["out_ptr"]
    assert [k for k, _, _ in prep.plan.launches] == ["rmw"]
    return g, prep, prep.plan.launches[0][1], ref


def _noalloc(prep, desc):
    from ktir_cpu_amd import runtime as rt
    prep.reset_inputs()
    rt.check(rt.lib().ktir_launch_row_rmw_noalloc(C.byref(desc)), "ktir_launch_row_rmw_noalloc")
    return prep.outputs()["out_ptr"]


def test_noalloc_matches_caller_scratch_twice():
    # 1: 8192 destination rows of 128 columns (row-order apply kernel), long chains
    keep1, prep1, d1, ref1 = _prepared(8192, 128, 4096, 8, 64, 3000, 1)
    print("call 1: rows 8192, dim 128, entries 4096", flush=True)
    np.testing.assert_array_equal(_noalloc(prep1, d1), ref1)
    # 2: a smaller input (fewer rows and entries, 32 columns: generic apply kernel)
    keep2, prep2, d2, ref2 = _prepared(1024, 32, 512, 4, 32, 40, 2)
    print("call 2: rows 1024, dim 32, entries 512", flush=True)
    np.testing.assert_array_equal(_noalloc(prep2, d2), ref2)
    # and the first input again: the heads left by call 2 are all empty
    np.testing.assert_array_equal(_noalloc(prep1, d1), ref1)


def test_noalloc_rejects_sizes_past_its_array():
    """Sizes beyond the scratch array are refused before anything launches."""
    from ktir_cpu_amd import runtime as rt
    keep, prep, d, ref = _prepared(1024, 32, 512, 4, 32, 40, 3)
    big = type(d).from_buffer_copy(d)
    big.n_rows = (2 << 20) + 1
    with pytest.raises(NotImplementedError):
        rt.check(rt.lib().ktir_launch_row_rmw_noalloc(C.byref(big)), "ktir_launch_row_rmw_noalloc")
    big = type(d).from_buffer_copy(d)
    big.n_inst = ((1 << 20) // big.K) + 1
    with pytest.raises(NotImplementedError):
        rt.check(rt.lib().ktir_launch_row_rmw_noalloc(C.byref(big)), "ktir_launch_row_rmw_noalloc")
