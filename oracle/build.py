"""Builds the CPU oracle `oracle/liboracle.so` with gcc (test infrastructure).

No fast-math and no FMA contraction, so each f32 operation is one IEEE
operation as in the reference's Rust. OpenMP only parallelises over heads or
sequences; the per-row arithmetic is the same at any thread count.

The reference itself is Rust (no cargo/rustc in this image), so there is no
`oracle/_ref` build: the restatement in oracle.c is the oracle.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


def build(verbose: bool = False) -> Path:
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
           "-fno-fast-math", str(HERE / "oracle.c"), "-o", str(LIB) + ".tmp", "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{r.stderr}")
    Path(str(LIB) + ".tmp").replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
