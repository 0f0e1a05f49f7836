"""Builds the gfx950 attention library `libllmtie_hip.so` in-tree with hipcc.

The library is the product: HIP kernels plus the C ABI declared in
include/llmtie_hip.h. It links only the HIP runtime (no torch), so any host
language can bind it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libllmtie_hip.so"
SOURCES = ["api.hip", "decode.hip", "prefill.hip", "kvcache.hip"]
ARCH = "gfx950"
# Packed-FP32 instructions stay off (they have given silent wrong results on
# this pool); -O3 would otherwise form them from ordinary float code.
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return cand


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into the in-tree shared library."""
    srcs = [str(CSRC / s) for s in SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, "-I", str(ROOT / "include"), *srcs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
