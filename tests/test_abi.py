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


def test_struct_sizes_match_c(tmp_path):
    """Compile a tiny host program that prints sizeof() of every descriptor."""
    from ktir_cpu_amd import runtime as rt
    src = '#include <stdio.h>\n#include "ktir_hip.h"\nint main(){printf("%zu %zu %zu %zu %zu %zu %zu %zu\\n",' \
          'sizeof(ktir_leaf_t), sizeof(ktir_instr_t), sizeof(ktir_prog_t), sizeof(ktir_iat_t), ' \
          'sizeof(ktir_mm_t), sizeof(ktir_rmw_t), sizeof(ktir_attn_t), sizeof(ktir_pattn_t));return 0;}'
    tmp = str(tmp_path)
    with open(os.path.join(tmp, "s.c"), "w") as f:
        f.write(src)
    exe = os.path.join(tmp, "s")
    r = subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), os.path.join(tmp, "s.c"), "-o", exe],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    sizes = [int(x) for x in subprocess.run([exe], capture_output=True, text=True).stdout.split()]
    assert sizes == [C.sizeof(rt.Leaf), C.sizeof(rt.Instr), C.sizeof(rt.Prog), C.sizeof(rt.IAT),
                     C.sizeof(rt.MM), C.sizeof(rt.RMW), C.sizeof(rt.ATTN), C.sizeof(rt.PATTN)]
    assert C.sizeof(rt.Prog) < 4096   # travels in the kernel arguments


def _rmw_desc(**kw):
    from ktir_cpu_amd import runtime as rt
    d = rt.RMW()
    d.n_inst, d.K, d.D, d.n_rows = 4, 128, 128, 1024
    d.dst_dtype, d.src_dtype, d.dt = rt.DTYPE_CODE["f32"], rt.DTYPE_CODE["f16"], rt.DTYPE_CODE["f32"]
    d.dst_row, d.dst_col, d.src_row, d.src_col = 128, 1, 128, 1
    d.dst_ptr, d.src_ptr = 1 << 20, 1 << 24
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.skipif(not os.path.exists(LIB), reason="libktir_hip.so not built")
def test_rmw_variant_choice():
    """The apply-kernel choice of the ordered row RMW (a host-only query: no
    HIP call).  The row-order kernel needs f32 rows of a multiple of 128
    columns, unit column strides and 16-byte alignment; anything else, and the
    D = 32 form, takes the generic kernel."""
    from ktir_cpu_amd import runtime as rt
    lib = C.CDLL(LIB)
    lib.ktir_rmw_variant.argtypes = [C.POINTER(rt.RMW)]
    v = lambda **kw: lib.ktir_rmw_variant(C.byref(_rmw_desc(**kw)))
    ROWS, GEN = rt.K["KTIR_RMW_ROWS"], rt.K["KTIR_RMW_GENERIC"]
    assert v() == ROWS
    assert v(src_dtype=rt.DTYPE_CODE["f32"]) == ROWS
    assert v(D=256, dst_row=256, src_row=256) == ROWS
    assert v(D=32, dst_row=32, src_row=32) == GEN
    assert v(D=96) == GEN
    assert v(dst_col=2) == GEN
    assert v(dst_dtype=rt.DTYPE_CODE["f16"], dt=rt.DTYPE_CODE["f16"]) == GEN
    assert v(src_dtype=rt.DTYPE_CODE["bf16"]) == GEN
    assert v(dst_base=2) == GEN
    assert v(src_ptr=(1 << 24) + 8) == GEN
    assert v(dst_row=0) == GEN
    assert v(K=0) == rt.K["KTIR_E_ARG"]
    assert v(K=2048) == rt.K["KTIR_E_ARG"]
