"""The C-ABI from a compiled C++ caller (spaceslug-main_amd/examples/runtime_abi_client.cpp), built with g++
against include/runtime_abi.h and the runtime library the way a C++ host would link it."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
SRC = REPO / "spaceslug-main_amd" / "examples" / "runtime_abi_client.cpp"


def build_client(runtime_lib_path: Path, out: Path) -> Path:
    lib_dir = runtime_lib_path.parent
    subprocess.run(["g++", "-std=c++17", "-O2", f"-I{REPO / 'include'}", str(SRC), f"-L{lib_dir}",
                    "-lspaceslug_runtime", f"-Wl,-rpath,{lib_dir}", "-o", str(out)], check=True)
    return out


def test_client_builds_and_runs_without_gpu(runtime_lib_path, tmp_path):
    exe = build_client(runtime_lib_path, tmp_path / "client")
    r = subprocess.run([str(exe), "--allow-no-device"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "vector_add: PASS" in r.stdout


@pytest.mark.gpu
def test_client_int4_call_on_gpu(runtime_lib_path, gpu, tmp_path):
    exe = build_client(runtime_lib_path, tmp_path / "client")
    print("[gpu-case] C++ client", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "q4gemm: PASS" in r.stdout


REFERENCE_NATIVE_CALLER = Path("/root/reference/native/runtime_abi_test.cpp")


def test_native_header_path_builds_a_caller(runtime_lib_path, tmp_path):
    """native/runtime_abi.h, at the path the reference's native callers include it from, declares the same
    ABI: the example client builds against it alone and runs its CPU part."""
    lib_dir = runtime_lib_path.parent
    exe = tmp_path / "client_native"
    subprocess.run(["g++", "-std=c++17", "-O2", f"-I{REPO / 'native'}", str(SRC), f"-L{lib_dir}",
                    "-lspaceslug_runtime", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe), "--allow-no-device"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "vector_add: PASS" in r.stdout


@pytest.mark.skipif(not REFERENCE_NATIVE_CALLER.is_file(), reason="reference sources not mounted here")
def test_reference_native_caller_builds_unchanged(runtime_lib_path, tmp_path):
    """The reference's own native caller (native/runtime_abi_test.cpp, compiled where it lies, not copied)
    builds against native/runtime_abi.h, links against libspaceslug_runtime.so and passes."""
    lib_dir = runtime_lib_path.parent
    exe = tmp_path / "reference_native_caller"
    subprocess.run(["g++", "-std=c++17", "-O2", f"-I{REPO / 'native'}", str(REFERENCE_NATIVE_CALLER),
                    f"-L{lib_dir}", "-lspaceslug_runtime", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout


CHAIN_SRC = REPO / "spaceslug-main_amd" / "examples" / "tiny_projection_chain.cpp"
ROCM = Path("/opt/rocm")


def build_chain_driver(runtime_lib_path: Path, out: Path) -> Path:
    lib_dir = runtime_lib_path.parent
    subprocess.run(["g++", "-std=c++17", "-O2", "-D__HIP_PLATFORM_AMD__", f"-I{REPO / 'include'}",
                    f"-I{ROCM / 'include'}", str(CHAIN_SRC), f"-L{lib_dir}", "-lspaceslug_runtime",
                    f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{ROCM / 'lib'}",
                    "-o", str(out)], check=True)
    return out


def test_chain_driver_builds_and_skips_without_gpu(runtime_lib_path, tmp_path):
    exe = build_chain_driver(runtime_lib_path, tmp_path / "chain")
    r = subprocess.run([str(exe), "--allow-no-device"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_chain_driver_on_gpu(runtime_lib_path, gpu, tmp_path):
    exe = build_chain_driver(runtime_lib_path, tmp_path / "chain")
    print("[gpu-case] C++ tiny projection chain", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 4
