"""spaceslug_q4gemm_device_noalloc: the device entry point that allocates nothing.

Called through the C-ABI (ctypes) and checked against spaceslug_q4gemm_device, which runs
the same kernels on the library's grow-only workspace: two calls in a row, the second on a
smaller input that reuses the fixed scratch the first left full, must give the same bits
as the workspace entry point and meet the 1e-5 bar against the oracle. A shape whose
scratch exceeds the fixed size is rejected with status 1 before anything is enqueued.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from cases import make_case

pytestmark = pytest.mark.gpu

TOL = 1e-5


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def threads():
    import os

    return min(16, os.cpu_count() or 1)


def _lib(runtime_lib_path):
    L = ctypes.CDLL(str(runtime_lib_path))
    for name in ("spaceslug_q4gemm_device_noalloc", "spaceslug_q4gemm_device"):
        fn = getattr(L, name)
        fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_uint32] * 3 + [ctypes.c_void_p]
        fn.restype = ctypes.c_int
    L.spaceslug_last_error.restype = ctypes.c_char_p
    return L


def _run(fn, torch, x, w, s, m, n, k):
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream()
    rc = fn(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(s.data_ptr()),
            ctypes.c_void_p(y.data_ptr()), m, n, k, ctypes.c_void_p(st.cuda_stream))
    st.synchronize()
    return rc, y


def test_noalloc_matches_workspace_entry(runtime_lib_path, oracle, gpu):
    import torch

    L = _lib(runtime_lib_path)
    # first a K-split wide call (x limbs and split partials in the scratch: 28 MiB), then a smaller
    # one whose split partials land on what the first call left there, then a mid-size call (64 x 64
    # whole-K tiles: x limbs by rows in the scratch) and a small-batch one (no scratch)
    for m, n, k in ((512, 4096, 4096), (40, 300, 1056), (100, 301, 512), (16, 512, 512)):
        note(f"noalloc {m}x{n}x{k}")
        c = make_case(m, n, k, seed_a=0x12345678 + m, seed_b=0x9ABCDEF0 + n)
        x = torch.from_numpy(c.x).to("cuda:0")
        w = torch.from_numpy(c.packed).to("cuda:0")
        s = torch.from_numpy(c.scales).to("cuda:0")
        rc, y = _run(L.spaceslug_q4gemm_device_noalloc, torch, x, w, s, m, n, k)
        assert rc == 0, L.spaceslug_last_error()
        rc, y_ws = _run(L.spaceslug_q4gemm_device, torch, x, w, s, m, n, k)
        assert rc == 0, L.spaceslug_last_error()
        assert torch.equal(y, y_ws), "fixed-scratch result differs from the workspace entry point"
        rep = oracle.compare(y.cpu().numpy(), oracle.q4gemm_packed(c.x, c.packed, c.scales, threads=threads()), TOL)
        note(f"noalloc {m}x{n}x{k} max_rel={rep['max_relative_error']:.3e}")
        assert rep["status"] == "pass", rep


def test_noalloc_rejects_scratch_beyond_its_size(runtime_lib_path, gpu):
    import torch

    L = _lib(runtime_lib_path)
    # 4096 rows x 8192 values of x need 192 MiB of bf16 limbs: more than the fixed 64 MiB
    m, n, k = 4096, 64, 8192
    note(f"noalloc rejects {m}x{n}x{k}")
    x = torch.zeros(64, dtype=torch.float32, device="cuda:0")
    y = torch.zeros(64, dtype=torch.float32, device="cuda:0")
    rc = L.spaceslug_q4gemm_device_noalloc(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                           ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), m, n, k,
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 1
    assert b"scratch" in L.spaceslug_last_error()
    assert torch.count_nonzero(y).item() == 0
