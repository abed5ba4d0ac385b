"""The CPU oracle and the host side of the C-ABI under AddressSanitizer and UndefinedBehaviorSanitizer.

Two programs are built from the repository's sources in a temporary directory and run on this
machine's CPU (no GPU is needed or used):
  - tests/sanitize/oracle_driver.c with oracle/q4_oracle.c and oracle/cq4_oracle.c (gcc,
    -fsanitize=address,undefined): every oracle function, its argument rejections included;
  - tests/sanitize/abi_driver.cpp with every source of libspaceslug_runtime.so (hipcc; only the
    host code is instrumented, the gfx950 code objects are built as usual): argument validation of
    every entry point, the no-device path of every compute entry point (also from eight threads at
    once, racing on the first device query), the retained-chain rejections and the CPU entry points.
Leak detection is on. Any sanitizer report aborts the program, so a zero exit status with the
driver's "all checks passed" line is a clean run. A first test plants an out-of-bounds read in a
throwaway program and checks that the same flags catch it, so a silently ineffective sanitizer
build cannot pass.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "spaceslug-main_amd" / "csrc"
SANITIZE = REPO / "tests" / "sanitize"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CLANGXX = "/opt/rocm/llvm/bin/clang++"
RUNTIME_SOURCES = ["q4_gemv.hip", "q4_gemm.hip", "q4_small.hip", "q4_quantize.hip", "cq4.hip", "sgemm.hip",
                   "runtime_abi.cpp"]
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
GCC_SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
# hipcc: instrument the host code only (the device code is built as it is for the product).
HIPCC_SAN = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=all",
             "-Xarch_host", "-fno-omit-frame-pointer"]


def _run(cmd, **kw):
    proc = subprocess.run(cmd, capture_output=True, text=True, **kw)
    return proc.returncode, proc.stdout + proc.stderr


def test_sanitizers_catch_a_planted_overflow(tmp_path):
    src = tmp_path / "planted.c"
    src.write_text("#include <stdlib.h>\nint main(void) { volatile int* p = malloc(4 * sizeof(int));\n"
                   "  int v = p[4]; free((void*)p); return v & 0; }\n")
    exe = tmp_path / "planted"
    rc, out = _run(["gcc", "-O0", "-g", *GCC_SAN, str(src), "-o", str(exe)])
    assert rc == 0, out
    rc, out = _run([str(exe)], env=SAN_ENV)
    assert rc != 0 and "heap-buffer-overflow" in out


def test_oracle_under_asan_ubsan(tmp_path):
    exe = tmp_path / "oracle_driver"
    rc, out = _run(["gcc", "-O1", "-g", *GCC_SAN, "-fopenmp", f"-I{REPO / 'oracle'}",
                    str(SANITIZE / "oracle_driver.c"), str(REPO / "oracle" / "q4_oracle.c"),
                    str(REPO / "oracle" / "cq4_oracle.c"), "-o", str(exe), "-lm"])
    assert rc == 0, out
    rc, out = _run([str(exe)], env=SAN_ENV, timeout=300)
    assert rc == 0, out
    assert "all checks passed" in out


@pytest.mark.skipif(not Path(HIPCC).exists() or not Path(CLANGXX).exists(), reason="ROCm toolchain not installed")
@pytest.mark.skipif(Path("/dev/kfd").exists(),
                    reason="the driver passes stand-in device addresses, valid only where no GPU can be reached")
def test_abi_host_code_under_asan_ubsan(tmp_path):
    common = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
              "-packed-fp32-ops", *HIPCC_SAN, f"-I{REPO / 'include'}", f"-I{CSRC}"]
    jobs = []
    objs = []
    for name in RUNTIME_SOURCES + ["abi_driver.cpp"]:
        src = (SANITIZE if name == "abi_driver.cpp" else CSRC) / name
        obj = tmp_path / (name + ".o")
        lang = ["-x", "hip"] if name.endswith(".cpp") else []
        jobs.append(subprocess.Popen([HIPCC, *common, *lang, "-c", str(src), "-o", str(obj)],
                                     stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
        objs.append(obj)
    for job in jobs:
        out, err = job.communicate(timeout=600)
        assert job.returncode == 0, err
    exe = tmp_path / "abi_driver"
    # Linked by ROCm's clang++, whose sanitizer runtimes match the instrumentation hipcc emitted.
    rc, out = _run([CLANGXX, "-fsanitize=address,undefined", *map(str, objs), "-o", str(exe), "-L/opt/rocm/lib",
                    "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"])
    assert rc == 0, out
    rc, out = _run([str(exe)], env=SAN_ENV, timeout=300)
    assert rc == 0, out
    assert "all checks passed" in out
