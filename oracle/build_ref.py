"""Builds the reference's own CQ4 CPU library into oracle/_ref/ (test infrastructure only).

vulkan-runtime/src/cactus/cactus_x86.cpp and cactus_x86_bridge.cpp compile on
their own (standard headers only) but need clang, for the ARM-style `__fp16`
storage type (cactus_x86.h:17-24): ROCm's clang++ compiles them in place, from
/root/reference, into oracle/_ref/libcactus_ref.so. Nothing of the reference is
copied; the library is git-ignored and travels to the GPU box like the product's
own built libraries. Tests use it, when it is there, to check cq4_oracle.c
against cactus_bridge_quant_matmul (cactus_x86_bridge.h).
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

REFERENCE = Path("/root/reference/vulkan-runtime/src")
ORACLE_DIR = Path(__file__).resolve().parent
REF_DIR = ORACLE_DIR / "_ref"
LIB = REF_DIR / "libcactus_ref.so"


def clang() -> str | None:
    for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++")):
        if c and Path(c).exists():
            return c
    return None


def build(verbose: bool = False) -> Path | None:
    """Returns the library path, or None when the reference sources or clang are absent."""
    srcs = [REFERENCE / "cactus" / "cactus_x86.cpp", REFERENCE / "cactus" / "cactus_x86_bridge.cpp"]
    cxx = clang()
    if cxx is None or not all(s.is_file() for s in srcs):
        return None
    REF_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cxx, "-std=c++17", "-O2", "-fPIC", "-shared", f"-I{REFERENCE}", *map(str, srcs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
