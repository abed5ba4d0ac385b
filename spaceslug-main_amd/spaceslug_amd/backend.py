"""ctypes binding of libspaceslug_runtime.so, mirroring the reference host's conventions.

Reference: python/spaceslug/backend.py
  - ExecutionResult / BackendError            :28-41
  - BackendSession._native()                  :56-67  (CDLL, mandatory symbols
    spaceslug_vector_add and spaceslug_sgemm bound unconditionally, every other
    symbol probed with hasattr)
  - execute_sgemm_native                      :571-583
  - _native_sgemm_values (projection caller)  :1692-1705
  - execute_tiny_lora_forward's projected()   :794-799 (base + LoRA delta)
A nonzero status from the library raises BackendError carrying the status and
spaceslug_last_error(). The int4 path exists only on the GPU: there is no CPU
fallback, so a missing library or a missing HIP device is an error.

Parity is reported, as in execute_projected_qkv (:585-600), against a
``cpu_reference`` supplied by the caller; without one the metrics say
"parity": "not-run".
"""
from __future__ import annotations

import ctypes
import os
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Sequence

import numpy as np

from .parity import compare_float_arrays

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
DEFAULT_LIBRARY = PACKAGE_ROOT / "_lib" / "libspaceslug_runtime.so"

# Status codes of include/runtime_abi.h.
OK = 0
ERR_INVALID = 1
ERR_DEVICE = 2
ERR_UNSUPPORTED = -4

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32 = ctypes.c_uint32


def library_path() -> Path:
    """SPACESLUG_RUNTIME_LIB overrides the in-tree build location."""
    env = os.environ.get("SPACESLUG_RUNTIME_LIB")
    return Path(env) if env else DEFAULT_LIBRARY


@dataclass(frozen=True)
class ExecutionResult:
    status: str
    operation: str
    backend: str
    runtime_revision: str
    device: str | None
    fallback_used: bool
    metrics: dict[str, Any] = field(default_factory=dict)
    output: dict[str, Any] = field(default_factory=dict)


class BackendError(RuntimeError):
    """A structured backend invocation failure."""


def _f32(values: Any, count: int, name: str) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(values, dtype=np.float32).ravel())
    if arr.size != count:
        raise BackendError(f"{name} has {arr.size} elements, expected {count}")
    return arr


def _u8(values: Any, count: int, name: str) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(values, dtype=np.uint8).ravel())
    if arr.size != count:
        raise BackendError(f"{name} has {arr.size} bytes, expected {count}")
    return arr


class Q4Weight:
    """Device-resident int4 weights (spaceslug_q4_weight_create / _destroy)."""

    def __init__(self, session: "BackendSession", handle: int, n: int, k: int) -> None:
        self._session = session
        self._handle = handle
        self.n = n
        self.k = k

    @property
    def handle(self) -> int:
        if not self._handle:
            raise BackendError("Q4Weight is closed")
        return self._handle

    def run(self, x: Any, m: int) -> np.ndarray:
        """y[m][n] = x[m][k] * dequant(W), synchronous (spaceslug_q4gemm_run)."""
        xx = _f32(x, m * self.k, "x")
        yy = np.empty(m * self.n, dtype=np.float32)
        lib = self._session._native()
        code = lib.spaceslug_q4gemm_run(ctypes.c_void_p(self.handle), xx.ctypes.data_as(_f32p),
                                        yy.ctypes.data_as(_f32p), m)
        self._session._check(code, "spaceslug_q4gemm_run")
        return yy.reshape(m, self.n)

    def close(self) -> None:
        if self._handle:
            self._session._native().spaceslug_q4_weight_destroy(ctypes.c_void_p(self._handle))
            self._handle = 0

    def __enter__(self) -> "Q4Weight":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def __del__(self) -> None:  # best effort; explicit close() is preferred
        try:
            self.close()
        except Exception:
            pass


class CQ4MatrixStruct(ctypes.Structure):
    """spaceslug_cq4_matrix (include/runtime_abi.h), the field order of the reference's
    CactusQuantMatrixBridge (vulkan-runtime/src/cactus/cactus_x86_bridge.h)."""

    _fields_ = [("bits", ctypes.c_uint32), ("K", ctypes.c_uint32), ("N", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32), ("num_groups", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("codebook", ctypes.c_void_p), ("input_scale", ctypes.c_void_p),
                ("input_scale_recip", ctypes.c_void_p), ("norms", ctypes.c_void_p),
                ("packed_indices", ctypes.c_void_p), ("left_signs", ctypes.c_void_p),
                ("right_signs", ctypes.c_void_p), ("permutation", ctypes.c_void_p), ("rotation", ctypes.c_void_p),
                ("expanded", ctypes.c_void_p), ("norm_f32", ctypes.c_void_p)]


CQ4_FLAG_ORTHOGONAL = 1 << 2
CQ4_FLAG_INTERLEAVED_4ROW = 1 << 3


class Q4Step(ctypes.Structure):
    """spaceslug_q4_step (include/runtime_abi.h): one device-pointer projection of a chain."""

    _fields_ = [("d_x", ctypes.c_void_p), ("d_w_packed", ctypes.c_void_p), ("d_w_scales", ctypes.c_void_p),
                ("d_y", ctypes.c_void_p), ("m", ctypes.c_uint32), ("n", ctypes.c_uint32), ("k", ctypes.c_uint32),
                ("d_lora_a", ctypes.c_void_p), ("d_lora_b", ctypes.c_void_p), ("rank", ctypes.c_uint32),
                ("lora_scale", ctypes.c_float)]


class Q4Chain:
    """A retained chain of device-pointer projections replayed as one HIP graph
    (spaceslug_q4_chain_create / _run / _destroy). The buffers named by the steps must
    outlive the chain; refill their contents between runs, never move them."""

    def __init__(self, session: "BackendSession", handle: int, steps: int) -> None:
        self._session = session
        self._handle = handle
        self.steps = steps

    def run(self, stream: int = 0) -> None:
        if not self._handle:
            raise BackendError("Q4Chain is closed")
        lib = self._session._native()
        self._session._check(lib.spaceslug_q4_chain_run(ctypes.c_void_p(self._handle), ctypes.c_void_p(stream)),
                             "q4_chain_run")

    def close(self) -> None:
        if self._handle:
            self._session._native().spaceslug_q4_chain_destroy(ctypes.c_void_p(self._handle))
            self._handle = 0

    def __enter__(self) -> "Q4Chain":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def __del__(self) -> None:  # best effort; explicit close() is preferred
        try:
            self.close()
        except Exception:
            pass


class BackendSession:
    """Runtime session bound to libspaceslug_runtime.so (HIP, gfx950)."""

    def __init__(self, runtime_revision: str = "spaceslug-main_amd", library: str | Path | None = None) -> None:
        self.runtime_revision = runtime_revision
        self._library_path = Path(library) if library else library_path()
        self._library: ctypes.CDLL | None = None

    # -- loading -----------------------------------------------------------------------------
    def _native(self) -> ctypes.CDLL:
        if self._library is None:
            if not self._library_path.is_file():
                raise BackendError(f"runtime shared library is missing: {self._library_path}")
            try:
                lib = ctypes.CDLL(str(self._library_path))
                vector_add = lib.spaceslug_vector_add
                vector_add.argtypes = [_f32p, _f32p, _f32p, ctypes.c_size_t]
                vector_add.restype = ctypes.c_int
                sgemm = lib.spaceslug_sgemm
                sgemm.argtypes = [_f32p, _f32p, _f32p, _u32, _u32, _u32, _f32p]
                sgemm.restype = ctypes.c_int
            except (OSError, AttributeError) as exc:
                raise BackendError(f"failed to bind runtime library {self._library_path}: {exc}") from exc
            if hasattr(lib, "spaceslug_last_error"):
                lib.spaceslug_last_error.argtypes = []
                lib.spaceslug_last_error.restype = ctypes.c_char_p
            if hasattr(lib, "spaceslug_q4gemm_capability"):
                lib.spaceslug_q4gemm_capability.argtypes = []
                lib.spaceslug_q4gemm_capability.restype = ctypes.c_char_p
            if hasattr(lib, "spaceslug_q4gemm"):
                lib.spaceslug_q4gemm.argtypes = [_f32p, _u8p, _f32p, _f32p, _u32, _u32, _u32]
                lib.spaceslug_q4gemm.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4gemm_lora"):
                lib.spaceslug_q4gemm_lora.argtypes = [_f32p, _u8p, _f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32, _u32,
                                                      ctypes.c_float]
                lib.spaceslug_q4gemm_lora.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4gemm_device"):
                lib.spaceslug_q4gemm_device.argtypes = [ctypes.c_void_p] * 4 + [_u32, _u32, _u32, ctypes.c_void_p]
                lib.spaceslug_q4gemm_device.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4gemm_device_noalloc"):
                lib.spaceslug_q4gemm_device_noalloc.argtypes = [ctypes.c_void_p] * 4 + [_u32, _u32, _u32,
                                                                                       ctypes.c_void_p]
                lib.spaceslug_q4gemm_device_noalloc.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4gemm_lora_device"):
                lib.spaceslug_q4gemm_lora_device.argtypes = ([ctypes.c_void_p] * 6 + [_u32] * 4 +
                                                             [ctypes.c_float, ctypes.c_void_p])
                lib.spaceslug_q4gemm_lora_device.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4_weight_create"):
                lib.spaceslug_q4_weight_create.argtypes = [_u8p, _f32p, _u32, _u32]
                lib.spaceslug_q4_weight_create.restype = ctypes.c_void_p
                lib.spaceslug_q4_weight_destroy.argtypes = [ctypes.c_void_p]
                lib.spaceslug_q4_weight_destroy.restype = None
                lib.spaceslug_q4gemm_run.argtypes = [ctypes.c_void_p, _f32p, _f32p, _u32]
                lib.spaceslug_q4gemm_run.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4_quantize"):
                lib.spaceslug_q4_quantize.argtypes = [_f32p, _u8p, _f32p, _u32, _u32]
                lib.spaceslug_q4_quantize.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4_quantize_device"):
                lib.spaceslug_q4_quantize_device.argtypes = [ctypes.c_void_p] * 3 + [_u32, _u32, ctypes.c_void_p]
                lib.spaceslug_q4_quantize_device.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_cq4_matmul"):
                lib.spaceslug_cq4_matmul.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _u32, ctypes.c_void_p]
                lib.spaceslug_cq4_matmul.restype = ctypes.c_int
                lib.spaceslug_cq4_matmul_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _u32, ctypes.c_void_p,
                                                            ctypes.c_void_p]
                lib.spaceslug_cq4_matmul_device.restype = ctypes.c_int
            if hasattr(lib, "spaceslug_q4_chain_create"):
                lib.spaceslug_q4_chain_create.argtypes = [ctypes.POINTER(Q4Step), _u32]
                lib.spaceslug_q4_chain_create.restype = ctypes.c_void_p
                lib.spaceslug_q4_chain_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
                lib.spaceslug_q4_chain_run.restype = ctypes.c_int
                lib.spaceslug_q4_chain_destroy.argtypes = [ctypes.c_void_p]
                lib.spaceslug_q4_chain_destroy.restype = None
            self._library = lib
        return self._library

    def _last_error(self) -> str:
        lib = self._native()
        if hasattr(lib, "spaceslug_last_error"):
            msg = lib.spaceslug_last_error()
            return msg.decode() if msg else ""
        return ""

    def _check(self, code: int, name: str) -> None:
        if code != OK:
            raise BackendError(f"native {name} returned {code}: {self._last_error()}")

    def _require(self, symbol: str) -> ctypes.CDLL:
        lib = self._native()
        if not hasattr(lib, symbol):
            raise BackendError(f"runtime library does not export {symbol}")
        return lib

    def capability(self) -> str:
        lib = self._require("spaceslug_q4gemm_capability")
        return lib.spaceslug_q4gemm_capability().decode()

    # -- reference-compatible entry points -----------------------------------------------------
    def execute_vector_add(self, left: Sequence[float], right: Sequence[float]) -> ExecutionResult:
        if len(left) != len(right):
            raise BackendError("vector_add inputs must have equal length")
        started = time.perf_counter()
        lib = self._native()
        ll, rr = _f32(left, len(left), "left"), _f32(right, len(right), "right")
        out = np.empty_like(ll)
        self._check(lib.spaceslug_vector_add(ll.ctypes.data_as(_f32p), rr.ctypes.data_as(_f32p),
                                             out.ctypes.data_as(_f32p), ll.size), "vector_add")
        return ExecutionResult("ok", "vector_add", "spaceslug-hip", self.runtime_revision, None, False,
                               {"operation_count": 1, "host_elapsed_seconds": time.perf_counter() - started},
                               {"first": float(out[0]) if out.size else None,
                                "last": float(out[-1]) if out.size else None, "count": int(out.size)})

    def sgemm_values(self, a: Any, b: Any, m: int, n: int, k: int) -> np.ndarray:
        """fp32 C = A * B through spaceslug_sgemm (m % 64, n % 64, k % 32)."""
        if m % 64 or n % 64 or k % 32 or m <= 0 or n <= 0 or k <= 0:
            raise BackendError("native sgemm dimensions or input lengths are invalid")
        lib = self._native()
        aa, bb = _f32(a, m * k, "a"), _f32(b, k * n, "b")
        cc = np.empty(m * n, dtype=np.float32)
        err = ctypes.c_float()
        self._check(lib.spaceslug_sgemm(aa.ctypes.data_as(_f32p), bb.ctypes.data_as(_f32p), cc.ctypes.data_as(_f32p),
                                        m, n, k, ctypes.byref(err)), "sgemm")
        return cc.reshape(m, n)

    def execute_sgemm_native(self, a: Any, b: Any, m: int, n: int, k: int, *,
                             cpu_reference: Any | None = None) -> ExecutionResult:
        values = self.sgemm_values(a, b, m, n, k)
        metrics = self._parity(values, cpu_reference, 1e-3)
        return ExecutionResult("ok" if metrics.get("status", "pass") == "pass" else "error", "sgemm", "spaceslug-hip",
                               self.runtime_revision, None, False, metrics,
                               {"m": m, "n": n, "k": k, "first": float(values.flat[0]), "values": values})

    # -- int4 projection -------------------------------------------------------------------------
    def q4gemm_values(self, x: Any, w_packed: Any, w_scales: Any, m: int, n: int, k: int) -> np.ndarray:
        """y[m][n] = x[m][k] * dequant(W) through spaceslug_q4gemm (drop-in for _native_sgemm_values)."""
        lib = self._require("spaceslug_q4gemm")
        if k % 32 or m <= 0 or n <= 0 or k <= 0:
            raise BackendError("native q4gemm needs m >= 1, n >= 1 and k % 32 == 0")
        xx = _f32(x, m * k, "x")
        ww = _u8(w_packed, n * (k // 2), "w_packed")
        ss = _f32(w_scales, n * (k // 32), "w_scales")
        yy = np.empty(m * n, dtype=np.float32)
        self._check(lib.spaceslug_q4gemm(xx.ctypes.data_as(_f32p), ww.ctypes.data_as(_u8p), ss.ctypes.data_as(_f32p),
                                         yy.ctypes.data_as(_f32p), m, n, k), "q4gemm")
        return yy.reshape(m, n)

    def q4gemm_lora_values(self, x: Any, w_packed: Any, w_scales: Any, lora_a: Any, lora_b: Any, m: int, n: int,
                           k: int, rank: int, scale: float) -> np.ndarray:
        """y = x * dequant(W) + scale * (x * lora_a) * lora_b in one call (spaceslug_q4gemm_lora)."""
        lib = self._require("spaceslug_q4gemm_lora")
        if k % 32 or m <= 0 or n <= 0 or k <= 0 or rank <= 0:
            raise BackendError("native q4gemm_lora needs m, n, rank >= 1 and k % 32 == 0")
        xx = _f32(x, m * k, "x")
        ww = _u8(w_packed, n * (k // 2), "w_packed")
        ss = _f32(w_scales, n * (k // 32), "w_scales")
        aa = _f32(lora_a, k * rank, "lora_a")
        bb = _f32(lora_b, rank * n, "lora_b")
        yy = np.empty(m * n, dtype=np.float32)
        self._check(lib.spaceslug_q4gemm_lora(xx.ctypes.data_as(_f32p), ww.ctypes.data_as(_u8p),
                                              ss.ctypes.data_as(_f32p), aa.ctypes.data_as(_f32p),
                                              bb.ctypes.data_as(_f32p), yy.ctypes.data_as(_f32p), m, n, k, rank,
                                              float(scale)), "q4gemm_lora")
        return yy.reshape(m, n)

    def execute_q4gemm_native(self, x: Any, w_packed: Any, w_scales: Any, m: int, n: int, k: int, *,
                              cpu_reference: Any | None = None, tolerance: float = 1e-5) -> ExecutionResult:
        started = time.perf_counter()
        values = self.q4gemm_values(x, w_packed, w_scales, m, n, k)
        metrics = self._parity(values, cpu_reference, tolerance)
        metrics["host_elapsed_seconds"] = time.perf_counter() - started
        return ExecutionResult("ok" if metrics.get("status", "pass") == "pass" else "error", "q4gemm",
                               "spaceslug-hip", self.runtime_revision, None, False, metrics,
                               {"m": m, "n": n, "k": k, "values": values})

    def execute_q4gemm_lora_native(self, x: Any, w_packed: Any, w_scales: Any, lora_a: Any, lora_b: Any, m: int,
                                   n: int, k: int, rank: int, alpha: float, *, cpu_reference: Any | None = None,
                                   tolerance: float = 1e-5) -> ExecutionResult:
        """LoRA scale = alpha / rank (lora.py:22)."""
        values = self.q4gemm_lora_values(x, w_packed, w_scales, lora_a, lora_b, m, n, k, rank, alpha / rank)
        metrics = self._parity(values, cpu_reference, tolerance)
        return ExecutionResult("ok" if metrics.get("status", "pass") == "pass" else "error", "q4gemm_lora",
                               "spaceslug-hip", self.runtime_revision, None, False, metrics,
                               {"m": m, "n": n, "k": k, "rank": rank, "values": values})

    def create_q4_weight(self, w_packed: Any, w_scales: Any, n: int, k: int) -> Q4Weight:
        lib = self._require("spaceslug_q4_weight_create")
        if k % 32 or n <= 0 or k <= 0:
            raise BackendError("q4 weight needs n >= 1 and k % 32 == 0")
        ww = _u8(w_packed, n * (k // 2), "w_packed")
        ss = _f32(w_scales, n * (k // 32), "w_scales")
        handle = lib.spaceslug_q4_weight_create(ww.ctypes.data_as(_u8p), ss.ctypes.data_as(_f32p), n, k)
        if not handle:
            raise BackendError(f"native spaceslug_q4_weight_create failed: {self._last_error()}")
        return Q4Weight(self, handle, n, k)

    # -- device-pointer entry points (e.g. torch tensors: tensor.data_ptr(), stream.cuda_stream) -----
    def q4gemm_device(self, d_x: int, d_w_packed: int, d_w_scales: int, d_y: int, m: int, n: int, k: int,
                      stream: int = 0) -> None:
        lib = self._require("spaceslug_q4gemm_device")
        code = lib.spaceslug_q4gemm_device(ctypes.c_void_p(d_x), ctypes.c_void_p(d_w_packed),
                                           ctypes.c_void_p(d_w_scales), ctypes.c_void_p(d_y), m, n, k,
                                           ctypes.c_void_p(stream))
        self._check(code, "q4gemm_device")

    def q4gemm_device_noalloc(self, d_x: int, d_w_packed: int, d_w_scales: int, d_y: int, m: int, n: int, k: int,
                              stream: int = 0) -> None:
        """q4gemm_device with the library's fixed per-device scratch: allocates nothing; calls that
        overlap on one device race on that scratch."""
        lib = self._require("spaceslug_q4gemm_device_noalloc")
        code = lib.spaceslug_q4gemm_device_noalloc(ctypes.c_void_p(d_x), ctypes.c_void_p(d_w_packed),
                                                   ctypes.c_void_p(d_w_scales), ctypes.c_void_p(d_y), m, n, k,
                                                   ctypes.c_void_p(stream))
        self._check(code, "q4gemm_device_noalloc")

    def q4gemm_lora_device(self, d_x: int, d_w_packed: int, d_w_scales: int, d_lora_a: int, d_lora_b: int, d_y: int,
                           m: int, n: int, k: int, rank: int, scale: float, stream: int = 0) -> None:
        lib = self._require("spaceslug_q4gemm_lora_device")
        code = lib.spaceslug_q4gemm_lora_device(ctypes.c_void_p(d_x), ctypes.c_void_p(d_w_packed),
                                                ctypes.c_void_p(d_w_scales), ctypes.c_void_p(d_lora_a),
                                                ctypes.c_void_p(d_lora_b), ctypes.c_void_p(d_y), m, n, k, rank,
                                                float(scale), ctypes.c_void_p(stream))
        self._check(code, "q4gemm_lora_device")

    def create_q4_chain(self, steps: Sequence[dict[str, Any]]) -> Q4Chain:
        """Records device-pointer projections into one replayable HIP graph. Each step is a dict with
        d_x, d_w_packed, d_w_scales, d_y (device addresses), m, n, k and optionally d_lora_a, d_lora_b,
        rank, lora_scale."""
        lib = self._require("spaceslug_q4_chain_create")
        arr = (Q4Step * max(1, len(steps)))()
        for i, s in enumerate(steps):
            arr[i] = Q4Step(s["d_x"], s["d_w_packed"], s["d_w_scales"], s["d_y"], s["m"], s["n"], s["k"],
                            s.get("d_lora_a") or None, s.get("d_lora_b") or None, s.get("rank", 0),
                            float(s.get("lora_scale", 0.0)))
        handle = lib.spaceslug_q4_chain_create(arr, len(steps))
        if not handle:
            raise BackendError(f"native spaceslug_q4_chain_create failed: {self._last_error()}")
        return Q4Chain(self, handle, len(steps))

    # -- CQ4 codebook matmul (cactus_quant_matmul) ---------------------------------------------------
    def cq4_matmul_values(self, *, bits: int, K: int, N: int, group_size: int, num_groups: int, flags: int,
                          codebook: Any, norms: Any, packed_indices: Any, a: Any, m: int,
                          input_scale: Any = None, input_scale_recip: Any = None, left_signs: Any = None,
                          right_signs: Any = None, permutation: Any = None, rotation: Any = None) -> np.ndarray:
        """fp16 (uint16 bit patterns) C [m][N] = cactus_quant_matmul semantics, synchronous host arrays.
        fp16 arrays are uint16 bit patterns; signs int8; permutation uint32; packed_indices uint8."""
        lib = self._require("spaceslug_cq4_matmul")
        keep = {}

        def arr(x: Any, dtype: Any) -> int | None:
            if x is None:
                return None
            v = np.ascontiguousarray(x, dtype=dtype)
            keep[id(v)] = v
            return v.ctypes.data

        s = CQ4MatrixStruct(bits, K, N, group_size, num_groups, flags, arr(codebook, np.uint16),
                            arr(input_scale, np.uint16), arr(input_scale_recip, np.uint16), arr(norms, np.uint16),
                            arr(packed_indices, np.uint8), arr(left_signs, np.int8), arr(right_signs, np.int8),
                            arr(permutation, np.uint32), arr(rotation, np.uint16), None, None)
        aa = np.ascontiguousarray(a, dtype=np.uint16)
        if m > 0 and aa.size != m * K:
            raise BackendError(f"a must hold m*K = {m * K} fp16 values")
        c = np.zeros((max(m, 1), N), np.uint16)
        self._check(lib.spaceslug_cq4_matmul(ctypes.addressof(s), aa.ctypes.data, m, c.ctypes.data), "cq4_matmul")
        return c

    def cq4_matmul_device(self, matrix: CQ4MatrixStruct, d_a: int, m: int, d_c: int, stream: int = 0) -> None:
        """`matrix` holds device addresses in its array fields."""
        lib = self._require("spaceslug_cq4_matmul_device")
        self._check(lib.spaceslug_cq4_matmul_device(ctypes.addressof(matrix), ctypes.c_void_p(d_a), m,
                                                    ctypes.c_void_p(d_c), ctypes.c_void_p(stream)),
                    "cq4_matmul_device")

    # -- fp32 -> int4 group-32 quantizer ----------------------------------------------------------
    def q4_quantize_values(self, w: Any, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
        """fp32 w[k][n] (row-major) -> (packed uint8 [n, k/2], scales float32 [n, k/32]) through
        spaceslug_q4_quantize (rule in include/runtime_abi.h)."""
        lib = self._require("spaceslug_q4_quantize")
        if k % 32 or n <= 0 or k <= 0:
            raise BackendError("native q4_quantize needs n >= 1 and k % 32 == 0")
        ww = _f32(w, k * n, "w")
        packed = np.empty((n, k // 2), dtype=np.uint8)
        scales = np.empty((n, k // 32), dtype=np.float32)
        self._check(lib.spaceslug_q4_quantize(ww.ctypes.data_as(_f32p), packed.ctypes.data_as(_u8p),
                                              scales.ctypes.data_as(_f32p), n, k), "q4_quantize")
        return packed, scales

    def q4_quantize_device(self, d_w: int, d_w_packed: int, d_w_scales: int, n: int, k: int,
                           stream: int = 0) -> None:
        lib = self._require("spaceslug_q4_quantize_device")
        code = lib.spaceslug_q4_quantize_device(ctypes.c_void_p(d_w), ctypes.c_void_p(d_w_packed),
                                                ctypes.c_void_p(d_w_scales), n, k, ctypes.c_void_p(stream))
        self._check(code, "q4_quantize_device")

    # -- helpers -----------------------------------------------------------------------------------
    @staticmethod
    def _parity(values: np.ndarray, cpu_reference: Any | None, tolerance: float) -> dict[str, Any]:
        if cpu_reference is None:
            return {"parity": "not-run"}
        ref = np.asarray(cpu_reference, dtype=np.float64)
        if ref.size != values.size:
            raise BackendError("CPU reference length does not match GPU output")
        return {"parity": "cpu-reference", **compare_float_arrays(values, ref, tolerance=tolerance)}
