"""Build recipe for the CPU oracle (test infrastructure only).

gcc -O2 -ffp-contract=off -fopenmp on q4_oracle.c and cq4_oracle.c ->
oracle/_build/libq4oracle.so. The reference's own int4 CPU functions
(vulkan-runtime/tests/test_q4gemm.cpp:58-119) sit in a translation unit that
needs the Vulkan SDK, Vulkan-Hpp and VMA, none of which this image has, so
q4_oracle.c restates them. The reference's CQ4 CPU library does build here
(clang++ on its two source files): build_ref.py puts it in oracle/_ref/, where it
checks cq4_oracle.c.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
BUILD_DIR = ORACLE_DIR / "_build"
LIB = BUILD_DIR / "libq4oracle.so"


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared",
           "-Wall", "-Wextra", str(ORACLE_DIR / "q4_oracle.c"), str(ORACLE_DIR / "cq4_oracle.c"), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
