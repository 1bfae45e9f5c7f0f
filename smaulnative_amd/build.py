"""Builds libsmaul_rocm.so in-tree with hipcc for gfx950.

    python -m smaulnative_amd.build

Flags:
- ``--offload-arch=gfx950``: MI355X (CDNA4) only.
- ``-ffp-contract=off``: no implicit fused multiply-add; the kernels use
  explicit ``fmaf`` where they want one, so the combine's mul-then-add matches
  the reference's rounding (model.py:582).
- ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 VALU
  instructions in generated code.
- ``-mllvm -amdgpu-mfma-vgpr-form``: MFMA results in ordinary VGPRs.  The
  GEMM scales every MFMA partial with a VALU fma; with the results in AGPRs
  each of those would need two extra v_accvgpr moves.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "smaul_rocm.hip")
OUT = os.path.join(HERE, "libsmaul_rocm.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I" + os.path.join(REPO, "include"), "-I" + os.path.join(HERE, "csrc"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = [hipcc()] + HIPCC_FLAGS + [SRC, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    if verbose and res.stderr:
        sys.stderr.write("\n".join(l for l in res.stderr.splitlines() if "packed-fp32" not in l))
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
