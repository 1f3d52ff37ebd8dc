"""Build the gfx950 HIP library ``libktir_hip.so`` in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled for gfx950 and linked into one shared
library that exports the C ABI declared in ``include/ktir_hip.h``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libktir_hip.so")
OBJ = os.path.join(HERE, "_build")
ARCH = os.environ.get("KTIR_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep hipcc from emitting packed FP32 instructions.
# -ffp-contract=off: a*b+c stays two roundings, as in NumPy.
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wno-unused-result"]
# per-source additions: the paged attention MFMA kernel keeps its
# accumulators in VGPRs (MFMA C/D operands in the VGPR form), since it
# rescales them with VALU multiplies between products
FILE_FLAGS = {"ktir_pattn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found: the KTIR GPU backend needs ROCm's hipcc to build")


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link libktir_hip.so; returns its path."""
    hipcc = _hipcc()
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))

    def compile_one(src):
        obj = os.path.join(OBJ, src[:-4] + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-4000:]}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
