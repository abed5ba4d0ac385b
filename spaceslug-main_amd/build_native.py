"""Build recipe for libspaceslug_runtime.so (HIP kernels for gfx950 + the C-ABI).

Compiles every source under csrc/ with hipcc for gfx950 and links one shared
library into _lib/. Run as a script (``python build_native.py``) or call
``build()``. No cmake: one hipcc line per translation unit, printed when
``verbose`` is set.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
OBJ_DIR = LIB_DIR / "obj"
LIB_NAME = "libspaceslug_runtime.so"
# Launch-floor and HBM-read probes for the benchmark, in a library of their own.
PROBES_SOURCE = "bench_probes.hip"
PROBES_LIB_NAME = "libspaceslug_probes.so"
ARCH = "gfx950"

SOURCES = ["q4_gemv.hip", "q4_gemm.hip", "q4_small.hip", "q4_quantize.hip", "cq4.hip", "sgemm.hip", "runtime_abi.cpp"]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops (v_pk_fma_f32 and friends) stay disabled in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments arrive in SGPRs at wave launch (gfx950 kernarg preload) instead of
    # through a scalar load at kernel start: ~0.1 us less per GEMV launch of 8 us, whose
    # first global load needs the x pointer.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # MFMA results in architected VGPRs rather than accumulation registers: the int4
    # GEMM's float64 fold then reads them directly instead of through v_accvgpr_read
    # (M=2048, K=4096, N=14336: 2.37 -> 2.31 ms; LoRA 512x4096x4096: 200 -> 195 us).
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")
    return path


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def probes_library_path() -> Path:
    return LIB_DIR / PROBES_LIB_NAME


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32-ops feature; drop that one warning.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources for gfx950 and link the shared library. Returns its path."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    objs = []
    procs = []
    for src in SOURCES:
        obj = OBJ_DIR / (src + ".o")
        cmd = [cc, *COMMON_FLAGS]
        if src.endswith(".cpp"):
            cmd += ["-x", "hip"]
        cmd += ["-c", str(CSRC / src), "-o", str(obj)]
        procs.append(cmd)
        objs.append(obj)
    # Translation units are independent: compile them in parallel.
    max_jobs = jobs or min(len(procs), int(os.environ.get("MAX_JOBS", "8")))
    running: list[tuple[list[str], subprocess.Popen]] = []
    noise = "'-packed-fp32-ops' is not a recognized feature"
    errors = []
    for cmd in procs:
        if verbose:
            print(" ".join(cmd), flush=True)
        running.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        if len(running) >= max_jobs:
            c, p = running.pop(0)
            _, err = p.communicate()
            err = "\n".join(line for line in err.splitlines() if noise not in line)
            if p.returncode != 0:
                errors.append(f"command failed ({p.returncode}): {' '.join(c)}\n{err}")
    for c, p in running:
        _, err = p.communicate()
        err = "\n".join(line for line in err.splitlines() if noise not in line)
        if p.returncode != 0:
            errors.append(f"command failed ({p.returncode}): {' '.join(c)}\n{err}")
    if errors:
        raise RuntimeError("\n".join(errors))
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    probes = probes_library_path()
    ptmp = probes.with_suffix(".so.tmp")
    _run([cc, *COMMON_FLAGS, "-shared", str(CSRC / PROBES_SOURCE), "-o", str(ptmp)], verbose)
    os.replace(ptmp, probes)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
