"""Builds libsmaul_rocm.so in-tree with hipcc for gfx950 (one object per source, then one link).

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
CSRC = os.path.join(HERE, "csrc")
SOURCES = [os.path.join(CSRC, n) for n in ("smaul_rocm.hip", "attn.hip", "quant.hip", "backward.hip", "peaks.hip")]
OUT = os.path.join(HERE, "libsmaul_rocm.so")
OBJDIR = os.path.join(HERE, "_build")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I" + os.path.join(REPO, "include"), "-I" + CSRC,
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
    res = subprocess.run([hipcc()] + HIPCC_FLAGS + ["-c", src, "-o", obj], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src} ({res.returncode}):\n{res.stderr[-4000:]}")
    return obj, res.stderr


def build(verbose: bool = False) -> str:
    """Compile every source (in parallel) and link libsmaul_rocm.so; always rebuilds."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OBJDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        results = list(ex.map(_compile, SOURCES))
    if verbose:
        for _, err in results:
            if err:
                sys.stderr.write("\n".join(l for l in err.splitlines() if "packed-fp32" not in l))
    tmp = OUT + ".tmp"
    res = subprocess.run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC"] + [o for o, _ in results]
                         + ["-o", tmp], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
