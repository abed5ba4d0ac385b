"""ctypes/numpy front end of the CPU oracle (libq4oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. See q4_oracle.h for the
reference file:line each function restates and for how each one is pinned.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "libq4oracle.so"

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            from oracle import build_oracle

            build_oracle.build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        L = _lib
        L.oracle_lcg_next.argtypes = [ctypes.c_uint32]
        L.oracle_lcg_next.restype = ctypes.c_uint32
        L.oracle_generate_floats.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        L.oracle_generate_floats.restype = None
        L.oracle_generate_int4.argtypes = [_i8p, ctypes.c_size_t, ctypes.c_uint32]
        L.oracle_generate_int4.restype = None
        L.oracle_generate_normal.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        L.oracle_generate_normal.restype = None
        L.oracle_pack_q4.argtypes = [_i8p, ctypes.c_uint32, ctypes.c_uint32, _u8p]
        L.oracle_pack_q4.restype = ctypes.c_int
        L.oracle_unpack_q4.argtypes = [_u8p, ctypes.c_uint32, ctypes.c_uint32, _i8p]
        L.oracle_unpack_q4.restype = ctypes.c_int
        L.oracle_q4gemm_ref.argtypes = [_f32p, _i8p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _f64p]
        L.oracle_q4gemm_ref.restype = ctypes.c_int
        L.oracle_q4gemm_packed_rows.argtypes = [_f32p, _u8p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, _f64p]
        L.oracle_q4gemm_packed_rows.restype = ctypes.c_int
        L.oracle_q4gemm_lora_rows.argtypes = [_f32p, _u8p, _f32p, _f32p, _f32p, ctypes.c_uint32, ctypes.c_double,
                                              ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                              ctypes.c_uint32, ctypes.c_int, _f64p]
        L.oracle_q4gemm_lora_rows.restype = ctypes.c_int
        L.oracle_compare.argtypes = [_f32p, _f64p, ctypes.c_size_t, ctypes.c_double, _f64p, _f64p,
                                     ctypes.POINTER(ctypes.c_int64), _f64p]
        L.oracle_compare.restype = ctypes.c_size_t
        L.oracle_q4_quantize.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, _u8p, _f32p]
        L.oracle_q4_quantize.restype = ctypes.c_int
    return _lib


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def lcg_next(state: int) -> int:
    return int(lib().oracle_lcg_next(state & 0xFFFFFFFF))


def generate_floats(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_generate_floats(_ptr(out, _f32p), n, seed & 0xFFFFFFFF, lo, hi)
    return out


def generate_int4(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int8)
    lib().oracle_generate_int4(_ptr(out, _i8p), n, seed & 0xFFFFFFFF)
    return out


def generate_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_generate_normal(_ptr(out, _f32p), n, seed & 0xFFFFFFFF, mean, std)
    return out


def pack_q4(b: np.ndarray) -> np.ndarray:
    """b: int8 [K, N] in [-8, 7] -> uint8 [N, K/2] in the reference layout."""
    b = np.ascontiguousarray(b, dtype=np.int8)
    K, N = b.shape
    out = np.empty((N, K // 2), dtype=np.uint8)
    if lib().oracle_pack_q4(_ptr(b, _i8p), K, N, _ptr(out, _u8p)) != 0:
        raise ValueError("pack_q4: K must be even")
    return out


def unpack_q4(packed: np.ndarray, K: int, N: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    if packed.size != N * (K // 2):
        raise ValueError("unpack_q4: size mismatch")
    out = np.empty((K, N), dtype=np.int8)
    if lib().oracle_unpack_q4(_ptr(packed, _u8p), K, N, _ptr(out, _i8p)) != 0:
        raise ValueError("unpack_q4: K must be even")
    return out


def q4gemm_ref(a: np.ndarray, b: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """cpu_reference of test_q4gemm.cpp:102-119 (unpacked int8 B [K, N])."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), dtype=np.float64)
    if lib().oracle_q4gemm_ref(_ptr(a, _f32p), _ptr(b, _i8p), _ptr(scales, _f32p), M, N, K, _ptr(c, _f64p)) != 0:
        raise ValueError("q4gemm_ref: K must be a multiple of 32")
    return c


def default_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def q4gemm_packed(a: np.ndarray, packed: np.ndarray, scales: np.ndarray, rows: tuple[int, int] | None = None,
                  threads: int | None = None) -> np.ndarray:
    """Double reference from the packed bytes, rows [r0, r1) (bit-identical to q4gemm_ref)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    M, K = a.shape
    N = packed.shape[0] if packed.ndim == 2 else packed.size // (K // 2)
    r0, r1 = rows if rows is not None else (0, M)
    c = np.empty((r1 - r0, N), dtype=np.float64)
    rc = lib().oracle_q4gemm_packed_rows(_ptr(a, _f32p), _ptr(packed, _u8p), _ptr(scales, _f32p), M, N, K, r0, r1,
                                         threads or 1, _ptr(c, _f64p))
    if rc != 0:
        raise ValueError("q4gemm_packed: bad arguments")
    return c


def q4gemm_lora(a: np.ndarray, packed: np.ndarray, scales: np.ndarray, la: np.ndarray, lb: np.ndarray,
                scale: float, rows: tuple[int, int] | None = None, threads: int | None = None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    la = np.ascontiguousarray(la, dtype=np.float32)
    lb = np.ascontiguousarray(lb, dtype=np.float32)
    M, K = a.shape
    R = la.shape[1]
    N = lb.shape[1]
    r0, r1 = rows if rows is not None else (0, M)
    c = np.empty((r1 - r0, N), dtype=np.float64)
    rc = lib().oracle_q4gemm_lora_rows(_ptr(a, _f32p), _ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(la, _f32p),
                                       _ptr(lb, _f32p), R, float(scale), M, N, K, r0, r1, threads or 1,
                                       _ptr(c, _f64p))
    if rc != 0:
        raise ValueError("q4gemm_lora: bad arguments")
    return c


def q4_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp32 w [K, N] -> (packed uint8 [N, K/2], scales float32 [N, K/32]), the rule of spaceslug_q4_quantize."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    K, N = w.shape
    packed = np.empty((N, K // 2), dtype=np.uint8)
    scales = np.empty((N, K // 32), dtype=np.float32)
    if lib().oracle_q4_quantize(_ptr(w, _f32p), K, N, _ptr(packed, _u8p), _ptr(scales, _f32p)) != 0:
        raise ValueError("q4_quantize: K must be a multiple of 32")
    return packed, scales


def compare(actual: np.ndarray, expected: np.ndarray, tol: float) -> dict:
    """Comparator of test_q4gemm.cpp:376-390 / parity.py:6-16 (+ normwise error)."""
    act = np.ascontiguousarray(actual, dtype=np.float32).ravel()
    exp = np.ascontiguousarray(expected, dtype=np.float64).ravel()
    if act.size != exp.size:
        raise ValueError("compare: arrays must have equal length")
    mr, ma, nw = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    fb = ctypes.c_int64()
    bad = lib().oracle_compare(_ptr(act, _f32p), _ptr(exp, _f64p), act.size, tol, ctypes.byref(mr),
                               ctypes.byref(ma), ctypes.byref(fb), ctypes.byref(nw))
    return {"status": "pass" if bad == 0 else "fail", "tolerance": tol, "max_relative_error": mr.value,
            "max_abs_error": ma.value, "first_bad_index": None if fb.value < 0 else int(fb.value),
            "bad_count": int(bad), "normwise_error": nw.value, "count": int(act.size)}
