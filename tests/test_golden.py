"""Golden vectors of the reference test suite, on the oracle (CPU) and on the
HIP backend (GPU).  The oracle tests pin the oracle itself; the GPU tests are
parity tests to the same bit-exact bar."""
import numpy as np
import pytest

from oracle.interp import OracleInterpreter
from tests import _golden_kernels as gk


def _copy(kw):
    return {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()}


@pytest.mark.parametrize("name", sorted(gk.ALL))
def test_oracle_golden(name):
    src, fn, kw, key, expected = gk.ALL[name]()
    o = OracleInterpreter()
    o.load(src)
    out = o.execute_function(fn, **_copy(kw))
    np.testing.assert_array_equal(out[key], expected)


@pytest.mark.parametrize("scatter", [False, True], ids=["indirect_load", "indirect_store"])
def test_oracle_negative_index_raises(scatter):
    src, fn, kw = gk.negative_index(scatter)
    o = OracleInterpreter()
    o.load(src)
    with pytest.raises(IndexError):
        o.execute_function(fn, **kw)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(gk.ALL))
def test_gpu_golden(name):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw, key, expected = gk.ALL[name]()
    g = KTIRInterpreter()
    g.load(src)
    out = g.execute_function(fn, **_copy(kw))
    print(name, g.last_plan.mode, g.last_plan.counts(), flush=True)
    np.testing.assert_array_equal(out[key], expected)
    for k, v in kw.items():          # inputs come back unchanged, other outputs too
        if isinstance(v, np.ndarray) and k != key:
            np.testing.assert_array_equal(out[k], v)


@pytest.mark.gpu
@pytest.mark.parametrize("scatter", [False, True], ids=["indirect_load", "indirect_store"])
def test_gpu_negative_index_raises(scatter):
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw = gk.negative_index(scatter)
    g = KTIRInterpreter()
    g.load(src)
    with pytest.raises(IndexError):
        g.execute_function(fn, **kw)


@pytest.mark.parametrize("slack", [0, -1])
def test_oracle_lx_peak(slack):
    """The reference's LX peak for its K-loop matmul kernel is 622592 bytes:
    a capacity of exactly that runs, one byte less overflows."""
    from fractions import Fraction
    src, fn, kw, peak = gk.lx_matmul_loop()
    o = OracleInterpreter(lx_size_mb=Fraction(peak + slack, 1 << 20))
    o.load(src)
    if slack < 0:
        with pytest.raises(MemoryError, match="LX scratchpad overflow"):
            o.execute_function(fn, **_copy(kw))
    else:
        o.execute_function(fn, **_copy(kw))


@pytest.mark.gpu
@pytest.mark.parametrize("slack", [0, -1])
def test_gpu_lx_peak(slack):
    """The same boundary through the HIP backend's LX accounting, with
    results equal to the oracle's where it runs."""
    from fractions import Fraction
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    src, fn, kw, peak = gk.lx_matmul_loop()
    g = KTIRInterpreter(lx_size_mb=Fraction(peak + slack, 1 << 20))
    g.load(src)
    if slack < 0:
        with pytest.raises(MemoryError, match="LX scratchpad overflow"):
            g.execute_function(fn, **_copy(kw))
        return
    out = g.execute_function(fn, **_copy(kw))
    o = OracleInterpreter(lx_size_mb=Fraction(peak, 1 << 20))
    o.load(src)
    ref = o.execute_function(fn, **_copy(kw))
    np.testing.assert_allclose(out["c_ptr"].astype(np.float32), ref["c_ptr"].astype(np.float32), rtol=1e-2, atol=1e-3)
