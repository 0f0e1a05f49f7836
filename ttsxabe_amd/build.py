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
# The bench's measurement probes (peak MFMA rate, HBM read rate): a separate
# library so the attention ABI stays the reference's operators only.
PEAKS_LIB = PKG / "libllmtie_peaks.so"
PEAKS_SRC = "peaks.hip"
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


# Per-source extra flags. The prefill kernels' softmax takes maxima of raw
# MFMA outputs; with NaNs honoured every fmaxf operand first gets a
# canonicalising v_max of its own. Infinities (the -inf of masked keys)
# stay honoured. The decode kernels' MFMAs write VGPRs: in the AGPR form the
# batched Q8_0 kernel kept its context in AGPRs for the MFMAs and in VGPRs
# across the loop, 64 register moves a block (C5 68.6 -> 66.3 us).
EXTRA = {"prefill.hip": ["-fno-honor-nans"], "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
COMPILE = [f for f in FLAGS if f != "-shared"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source (one object each, in parallel) and link the
    in-tree shared library."""
    from concurrent.futures import ThreadPoolExecutor
    out = PKG / "_build"
    out.mkdir(exist_ok=True)
    objs = [out / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[hipcc(), *COMPILE, *EXTRA.get(s, []), "-I", str(ROOT / "include"), "-c", str(CSRC / s), "-o", str(o)]
            for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(len(cmds)) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc(), *FLAGS, *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    ptmp = PEAKS_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *FLAGS, str(CSRC / PEAKS_SRC), "-o", str(ptmp)], verbose)
    os.replace(ptmp, PEAKS_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
