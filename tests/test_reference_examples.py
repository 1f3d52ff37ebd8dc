"""The KTIR text front end on the reference's own example kernels (read from
the reference checkout when it is present; nothing of it is copied here):
every file parses, each function's grid, argument names and memory-view
sizes match what its text declares, as the reference's
tests/test_examples.py:104-135 checks for its interpreter."""
import glob
import os
import re

import numpy as np
import pytest

from ktir_cpu_amd.interpreter import KTIRInterpreter

EXAMPLES = "/root/reference/examples"
FILES = sorted(glob.glob(os.path.join(EXAMPLES, "**", "*.mlir"), recursive=True)
               + glob.glob(os.path.join(EXAMPLES, "**", "*.ktir"), recursive=True))

pytestmark = pytest.mark.skipif(not FILES, reason="reference example kernels not present")


def _declared(text):
    """(name, [arg names], grid) of every func.func in the text, by regex."""
    text = re.sub(r"//[^\n]*", "", text)
    out = []
    for m in re.finditer(r"func\.func\s+@(\w+)\s*\(([^)]*)\)\s*(?:->[^{]*)?(attributes\s*\{[^}]*\})?", text):
        args = re.findall(r"%(\w+)\s*:", m.group(2))
        g = re.search(r"grid\s*=\s*\[([^\]]*)\]", m.group(3) or "")
        grid = [int(x) for x in g.group(1).split(",")] if g else [1]
        grid = tuple(grid + [1] * (3 - len(grid)))
        out.append((m.group(1), args, grid))
    return out


@pytest.mark.parametrize("path", FILES, ids=[os.path.relpath(f, EXAMPLES) for f in FILES])
def test_example_parses_with_declared_structure(path):
    text = open(path).read()
    interp = KTIRInterpreter()
    interp.load(path)
    assert interp.module is not None and interp.module.functions
    for name, args, grid in _declared(text):
        fn = interp.module.get_function(name)
        assert fn.grid == grid
        assert interp.arg_names(name) == args
        for info in interp.tensor_input_output_sizes(name).values():
            assert len(info["shape"]) > 0 and isinstance(info["dtype"], str)


def _oracle_seeded(path, seeds):
    from oracle.interp import OracleInterpreter
    o = OracleInterpreter()
    o.load(path)

    def hook(o):
        for elem, arr in seeds:
            o.hbm.memory.write(elem * 2, arr.reshape(-1))
    o.prepare_hook = hook
    return o


@pytest.mark.parametrize("name,n,iters,groups", [("ktir/ring_reduce.mlir", 4, 1, 1),
                                                 ("ktir/ring_reduce_inner_loop.mlir", 4, 3, 1),
                                                 ("latency/ring_reduce_multi_group.mlir", 16, 1, 4)])
def test_oracle_runs_reference_ring_examples(name, n, iters, groups):
    """The reference's expected values for its ring-reduce examples
    (tests/test_examples.py:639-776): the first core of every group writes
    iters x its group's row sum (rtol 1e-2, as there)."""
    path = os.path.join(EXAMPLES, name)
    rows = np.random.default_rng(7).uniform(0.5, 1.5, size=(n, 128)).astype(np.float16)
    out_elem = 128 * n
    kw = {"in_ptr": 0, "out_ptr": out_elem}
    if iters > 1:
        kw["n_iters"] = iters
    o = _oracle_seeded(path, [(0, rows), (out_elem, np.zeros(128 * groups, np.float16))])
    fn = next(iter(o.module.functions))
    o.execute_function(fn, **kw)
    got = o.hbm.memory.read(out_elem * 2, 128 * groups, "f16").reshape(groups, 128).astype(np.float32)
    want = rows.astype(np.float32).reshape(groups, n // groups, 128).sum(1) * iters
    np.testing.assert_allclose(got, want, rtol=1e-2)


def test_oracle_runs_reference_rmsnorm_2x2():
    """examples/latency/rmsnorm_4core_2x2.mlir: distributed views plus the
    column partners' ring reduce give RMSNorm (f16 accumulation, so the
    tolerance of the reference's RMSNorm checks, rtol 1e-2 / atol 1e-2)."""
    from oracle.interp import OracleInterpreter
    rng = np.random.default_rng(1)
    X = rng.standard_normal((256, 4096)).astype(np.float16)
    W = rng.uniform(0.5, 1.5, (256, 4096)).astype(np.float16)
    o = OracleInterpreter()
    o.load(os.path.join(EXAMPLES, "latency/rmsnorm_4core_2x2.mlir"))
    out = o.execute_function("rmsnorm_2x2", X=X, Y=np.zeros_like(X), W=W, N=4096, eps=np.float16(1e-5),
                             BLOCK_SIZE=1024)
    x = X.astype(np.float64)
    want = x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-5) * W.astype(np.float64)
    np.testing.assert_allclose(out["Y"].astype(np.float64), want, rtol=1e-2, atol=1e-2)
