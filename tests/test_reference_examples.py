"""The KTIR text front end on the reference's own example kernels (read from
the reference checkout when it is present; nothing of it is copied here):
every file parses, each function's grid, argument names and memory-view
sizes match what its text declares, as the reference's
tests/test_examples.py:104-135 checks for its interpreter."""
import glob
import os
import re

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
