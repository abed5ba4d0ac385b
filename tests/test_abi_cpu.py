"""C-ABI and host-shim tests that need no GPU.

The library must load, export every entry point include/runtime_abi.h declares,
reject contract violations with status 1 before touching a device (the
reference's fail-closed codes: sgemm_api.cpp:38, lora_delta_api.cpp:44), and
report a missing device as status 2 rather than computing on the CPU.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "runtime_abi.h"

f32p = ctypes.POINTER(ctypes.c_float)
u8p = ctypes.POINTER(ctypes.c_uint8)


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(spaceslug_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib(runtime_lib_path):
    L = ctypes.CDLL(str(runtime_lib_path))
    L.spaceslug_last_error.restype = ctypes.c_char_p
    L.spaceslug_q4gemm_capability.restype = ctypes.c_char_p
    L.spaceslug_q4_weight_create.restype = ctypes.c_void_p
    return L


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for required in ("spaceslug_vector_add", "spaceslug_sgemm", "spaceslug_q4gemm", "spaceslug_q4gemm_lora",
                     "spaceslug_q4gemm_device", "spaceslug_q4gemm_lora_device", "spaceslug_q4_weight_create",
                     "spaceslug_q4_weight_destroy", "spaceslug_q4gemm_run", "spaceslug_q4gemm_capability",
                     "spaceslug_last_error", "spaceslug_q4_quantize", "spaceslug_q4_quantize_device",
                     "spaceslug_q4_chain_create", "spaceslug_q4_chain_run", "spaceslug_q4_chain_destroy",
                     "spaceslug_cq4_matmul", "spaceslug_cq4_matmul_device"):
        assert required in names


def test_library_exports_every_declared_symbol(lib, runtime_lib_path):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert missing == []
    # exported with C linkage (unmangled) in the dynamic symbol table
    out = subprocess.run(["nm", "-D", "--defined-only", str(runtime_lib_path)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\s[TW]\s(spaceslug_\w+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported


def test_library_contains_gfx950_code_object(runtime_lib_path):
    data = runtime_lib_path.read_bytes()
    assert b"gfx950" in data


def test_capability_string(lib):
    cap = lib.spaceslug_q4gemm_capability().decode()
    assert "gfx950" in cap and "group=32" in cap


def test_vector_add_contract(lib):
    # native/runtime_abi_test.cpp:5-8
    a = (ctypes.c_float * 3)(0.25, 1.5, -2.0)
    b = (ctypes.c_float * 3)(0.75, 2.5, 3.0)
    out = (ctypes.c_float * 3)()
    assert lib.spaceslug_vector_add(a, b, out, ctypes.c_size_t(3)) == 0
    assert list(out) == [1.0, 4.0, 1.0]
    assert lib.spaceslug_vector_add(None, b, out, ctypes.c_size_t(3)) == 1


def _arrays(m, n, k):
    x = np.zeros(m * k, np.float32)
    w = np.zeros(n * k // 2, np.uint8)
    s = np.ones(n * k // 32, np.float32)
    y = np.zeros(m * n, np.float32)
    return x, w, s, y


def _p(a, t=f32p):
    return a.ctypes.data_as(t)


def test_q4gemm_rejects_invalid_arguments(lib):
    x, w, s, y = _arrays(2, 8, 64)
    call = lib.spaceslug_q4gemm
    assert call(None, _p(w, u8p), _p(s), _p(y), 2, 8, 64) == 1
    assert call(_p(x), None, _p(s), _p(y), 2, 8, 64) == 1
    assert call(_p(x), _p(w, u8p), None, _p(y), 2, 8, 64) == 1
    assert call(_p(x), _p(w, u8p), _p(s), None, 2, 8, 64) == 1
    for m, n, k in ((0, 8, 64), (2, 0, 64), (2, 8, 0), (2, 8, 48), (2, 8, 16), (2, 8, 2**31 + 32),
                    (2, 2**31 - 2**16 + 1, 64), (2**31 - 2**16 + 1, 8, 64)):
        assert call(_p(x), _p(w, u8p), _p(s), _p(y), m, n, k) == 1
    assert b"k%32" in lib.spaceslug_last_error()


def test_q4gemm_lora_rejects_invalid_rank(lib):
    x, w, s, y = _arrays(2, 8, 64)
    la = np.zeros(64 * 65, np.float32)
    lb = np.zeros(65 * 8, np.float32)
    for rank in (0, 65):
        assert lib.spaceslug_q4gemm_lora(_p(x), _p(w, u8p), _p(s), _p(la), _p(lb), _p(y), 2, 8, 64, rank,
                                         ctypes.c_float(1.0)) == 1
    assert lib.spaceslug_q4gemm_lora(_p(x), _p(w, u8p), _p(s), None, _p(lb), _p(y), 2, 8, 64, 4,
                                     ctypes.c_float(1.0)) == 1


def test_device_entry_rejects_misaligned_pointers(lib):
    vp = ctypes.c_void_p
    args = [vp(0x100000), vp(0x200000), vp(0x300000), vp(0x400000)]
    bad_x = [vp(0x100004)] + args[1:]
    assert lib.spaceslug_q4gemm_device(*bad_x, 1, 8, 64, None) == 1
    bad_w = [args[0], vp(0x200008)] + args[2:]
    assert lib.spaceslug_q4gemm_device(*bad_w, 1, 8, 64, None) == 1
    bad_s = args[:2] + [vp(0x300002), args[3]]
    assert lib.spaceslug_q4gemm_device(*bad_s, 1, 8, 64, None) == 1
    assert lib.spaceslug_q4gemm_device(None, *args[1:], 1, 8, 64, None) == 1
    assert lib.spaceslug_q4gemm_device(*args, 1, 8, 40, None) == 1
    assert b"k%32" in lib.spaceslug_last_error()
    assert lib.spaceslug_q4gemm_device(*bad_s, 1, 8, 64, None) == 1
    assert b"misaligned" in lib.spaceslug_last_error()


def test_sgemm_rejects_reference_shape_violations(lib):
    a = np.zeros(64 * 64, np.float32)
    err = ctypes.c_float()
    for m, n, k in ((32, 64, 32), (64, 48, 32), (64, 64, 16), (0, 64, 32)):
        assert lib.spaceslug_sgemm(_p(a), _p(a), _p(a), m, n, k, ctypes.byref(err)) == 1
    assert lib.spaceslug_sgemm(_p(a), _p(a), _p(a), 64, 64, 32, None) == 1


def test_weight_handle_rejects_invalid_arguments(lib):
    w = np.zeros(64, np.uint8)
    s = np.ones(4, np.float32)
    assert lib.spaceslug_q4_weight_create(None, _p(s), 2, 64) is None
    assert lib.spaceslug_q4_weight_create(_p(w, u8p), _p(s), 2, 40) is None
    lib.spaceslug_q4_weight_destroy(None)  # accepts NULL
    x = np.zeros(64, np.float32)
    assert lib.spaceslug_q4gemm_run(None, _p(x), _p(x), 1) == 1


def test_chain_rejects_invalid_steps_before_device(lib):
    from spaceslug_amd.backend import Q4Step

    lib.spaceslug_q4_chain_create.restype = ctypes.c_void_p
    lib.spaceslug_q4_chain_create.argtypes = [ctypes.POINTER(Q4Step), ctypes.c_uint32]
    lib.spaceslug_q4_chain_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.spaceslug_q4_chain_destroy.argtypes = [ctypes.c_void_p]
    good = dict(d_x=0x100000, d_w_packed=0x200000, d_w_scales=0x300000, d_y=0x400000, m=1, n=8, k=64,
                d_lora_a=None, d_lora_b=None, rank=0, lora_scale=0.0)

    def steps(*variants):
        arr = (Q4Step * len(variants))()
        for i, v in enumerate(variants):
            arr[i] = Q4Step(**{**good, **v})
        return arr

    assert lib.spaceslug_q4_chain_create(None, 1) is None
    assert lib.spaceslug_q4_chain_create(steps({}), 0) is None
    assert b"at least one step" in lib.spaceslug_last_error()
    assert lib.spaceslug_q4_chain_create(steps({}, {"k": 48}), 2) is None
    assert b"step 1" in lib.spaceslug_last_error() and b"k%32" in lib.spaceslug_last_error()
    assert lib.spaceslug_q4_chain_create(steps({"d_x": 0x100004}), 1) is None
    assert b"misaligned" in lib.spaceslug_last_error()
    assert lib.spaceslug_q4_chain_create(steps({"d_lora_a": 0x500000}), 1) is None
    assert b"both factors" in lib.spaceslug_last_error()
    assert lib.spaceslug_q4_chain_create(steps({"d_lora_a": 0x500000, "d_lora_b": 0x600000, "rank": 65}), 1) is None
    assert b"rank" in lib.spaceslug_last_error()
    assert lib.spaceslug_q4_chain_run(None, None) == 1
    lib.spaceslug_q4_chain_destroy(None)  # accepts NULL


def _gpu_visible() -> bool:
    import torch

    return torch.cuda.is_available()


def test_no_cpu_fallback_without_device(lib):
    """Valid arguments with no HIP device must fail with 2, never compute on the CPU."""
    if _gpu_visible():
        pytest.skip("a GPU is visible: the device path is covered by the gpu-marked tests")
    x, w, s, y = _arrays(1, 8, 64)
    y[:] = 123.0
    assert lib.spaceslug_q4gemm(_p(x), _p(w, u8p), _p(s), _p(y), 1, 8, 64) == 2
    assert b"no HIP device" in lib.spaceslug_last_error()
    assert np.all(y == 123.0)
    err = ctypes.c_float()
    a = np.zeros(64 * 64, np.float32)
    assert lib.spaceslug_sgemm(_p(a), _p(a), _p(a), 64, 64, 32, ctypes.byref(err)) == 2
    packed = np.zeros(64 * 32, np.uint8)
    assert lib.spaceslug_q4_quantize(_p(a), _p(packed, u8p), _p(a), 64, 64) == 2
    from spaceslug_amd.backend import Q4Step

    lib.spaceslug_q4_chain_create.restype = ctypes.c_void_p
    lib.spaceslug_q4_chain_create.argtypes = [ctypes.POINTER(Q4Step), ctypes.c_uint32]
    one = (Q4Step * 1)(Q4Step(0x100000, 0x200000, 0x300000, 0x400000, 1, 8, 64, None, None, 0, 0.0))
    assert lib.spaceslug_q4_chain_create(one, 1) is None
    assert b"no HIP device" in lib.spaceslug_last_error()
    from oracle import cq4

    W = cq4.random_matrix(np.random.default_rng(0), bits=4, K=64, N=8, group_size=64)
    s = W.struct()
    a16 = np.zeros((1, 64), np.uint16)
    c16 = np.full((1, 8), 0x3C00, np.uint16)
    lib.spaceslug_cq4_matmul.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
    assert lib.spaceslug_cq4_matmul(ctypes.addressof(s), a16.ctypes.data, 1, c16.ctypes.data) == 2
    assert np.all(c16 == 0x3C00)


# -- host shim (spaceslug_amd.BackendSession) --------------------------------------------------------

def _stub_library(tmp_path: Path, name: str, body: str) -> Path:
    src = tmp_path / f"{name}.c"
    src.write_text(body)
    so = tmp_path / f"lib{name}.so"
    subprocess.run(["gcc", "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
    return so


def test_session_requires_mandatory_symbols(tmp_path):
    from spaceslug_amd import BackendError, BackendSession

    so = _stub_library(tmp_path, "onlyadd", "#include <stddef.h>\n"
                       "int spaceslug_vector_add(const float*a,const float*b,float*o,size_t n){return 0;}\n")
    with pytest.raises(BackendError, match="spaceslug_sgemm"):
        BackendSession(library=so)._native()
    with pytest.raises(BackendError, match="missing"):
        BackendSession(library=tmp_path / "absent.so")._native()


def test_session_probes_optional_symbols(tmp_path):
    from spaceslug_amd import BackendError, BackendSession

    so = _stub_library(tmp_path, "reflike", "#include <stddef.h>\n#include <stdint.h>\n"
                       "int spaceslug_vector_add(const float*a,const float*b,float*o,size_t n){"
                       "for(size_t i=0;i<n;++i)o[i]=a[i]+b[i];return 0;}\n"
                       "int spaceslug_sgemm(const float*a,const float*b,float*c,uint32_t m,uint32_t n,uint32_t k,"
                       "float*e){return 2;}\n")
    sess = BackendSession(library=so)
    res = sess.execute_vector_add([1.0, 2.0], [3.0, 4.0])
    assert res.status == "ok" and res.output["first"] == 4.0
    with pytest.raises(BackendError, match="does not export spaceslug_q4gemm"):
        sess.q4gemm_values(np.zeros(64), np.zeros(32, np.uint8), np.ones(2), 1, 1, 64)
    with pytest.raises(BackendError, match="returned 2"):
        sess.sgemm_values(np.zeros(64 * 64), np.zeros(64 * 64), 64, 64, 64)


def test_session_validates_shapes_before_calling(session):
    from spaceslug_amd import BackendError

    with pytest.raises(BackendError):
        session.q4gemm_values(np.zeros(10), np.zeros(16, np.uint8), np.ones(1), 1, 1, 32)
    with pytest.raises(BackendError):
        session.q4gemm_values(np.zeros(40), np.zeros(20, np.uint8), np.ones(1), 1, 1, 40)
    with pytest.raises(BackendError):
        session.sgemm_values(np.zeros(10), np.zeros(10), 32, 64, 32)


def test_session_reports_device_absence(session):
    from spaceslug_amd import BackendError

    if _gpu_visible():
        pytest.skip("a GPU is visible")
    with pytest.raises(BackendError, match="returned 2: no HIP device"):
        session.q4gemm_values(np.zeros(64), np.zeros(32, np.uint8), np.ones(2), 1, 1, 64)


def test_parity_report_matches_reference_metric():
    from spaceslug_amd import compare_float_arrays

    rep = compare_float_arrays([0.502, 10.005, -3.0], [0.5, 10.0, -3.0], tolerance=1e-3)
    assert rep["status"] == "fail" and rep["first_bad_index"] == 0
    assert abs(rep["max_relative_error"] - 2e-3) < 1e-9
    with pytest.raises(ValueError):
        compare_float_arrays([1.0], [1.0, 2.0])
