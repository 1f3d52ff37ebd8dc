"""The C-ABI library: it builds for gfx950 and exports every entry point the
public header declares; ctypes mirrors of the descriptors match the C layout.
No GPU needed (nothing is called)."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ktir_hip.h")
LIB = os.path.join(ROOT, "ktir_cpu_amd", "libktir_hip.so")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(ktir_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = _declared()
    for n in ("ktir_init", "ktir_malloc", "ktir_launch_program", "ktir_launch_matmul", "ktir_launch_row_rmw",
              "ktir_iat_offsets", "ktir_scatter_winners", "ktir_last_error"):
        assert n in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="libktir_hip.so not built")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s(ktir_\w+)", out))
    missing = [n for n in _declared() if n not in exported]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="libktir_hip.so not built")
def test_library_loads_without_gpu():
    # dlopen only: no HIP call is made
    lib = C.CDLL(LIB)
    for n in _declared():
        assert hasattr(lib, n)


def test_struct_sizes_match_c():
    """Compile a tiny host program that prints sizeof() of every descriptor."""
    from ktir_cpu_amd import runtime as rt
    src = '#include <stdio.h>\n#include "ktir_hip.h"\nint main(){printf("%zu %zu %zu %zu %zu %zu %zu\\n",' \
          'sizeof(ktir_leaf_t), sizeof(ktir_instr_t), sizeof(ktir_prog_t), sizeof(ktir_iat_t), ' \
          'sizeof(ktir_mm_t), sizeof(ktir_rmw_t), sizeof(ktir_attn_t));return 0;}'
    tmp = os.path.join(ROOT, "_build_sizes")
    os.makedirs(tmp, exist_ok=True)
    with open(os.path.join(tmp, "s.c"), "w") as f:
        f.write(src)
    exe = os.path.join(tmp, "s")
    r = subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), os.path.join(tmp, "s.c"), "-o", exe],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    sizes = [int(x) for x in subprocess.run([exe], capture_output=True, text=True).stdout.split()]
    assert sizes == [C.sizeof(rt.Leaf), C.sizeof(rt.Instr), C.sizeof(rt.Prog), C.sizeof(rt.IAT),
                     C.sizeof(rt.MM), C.sizeof(rt.RMW), C.sizeof(rt.ATTN)]
    assert C.sizeof(rt.Prog) < 4096   # travels in the kernel arguments
