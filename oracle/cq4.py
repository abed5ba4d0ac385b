"""CQ4 codebook matmul: the oracle's Python front end and a matrix builder (test infrastructure only).

`CQ4Matrix` holds the numpy arrays of one matrix and produces the C struct with
the field order of CactusQuantMatrixBridge (vulkan-runtime/src/cactus/
cactus_x86_bridge.h), which describes the matrix to this oracle (cq4_oracle.c),
to the reference's compiled bridge in oracle/_ref/ (when built) and to the
product's spaceslug_cq4_matmul alike. Fixture generators restate the reference
test's (vulkan-runtime/tests/test_cq4.cpp:66-160 and m6c1_common.h:33-42) so the
reference's five fixtures can be rebuilt bit for bit.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from oracle import oracle as _o

FLAG_ORTHOGONAL = 1 << 2
FLAG_INTERLEAVED_4ROW = 1 << 3
REF_LIB = Path(__file__).resolve().parent / "_ref" / "libcactus_ref.so"

_u16p = ctypes.POINTER(ctypes.c_uint16)


class CQ4Struct(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_uint32), ("K", ctypes.c_uint32), ("N", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32), ("num_groups", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("codebook", ctypes.c_void_p), ("input_scale", ctypes.c_void_p),
                ("input_scale_recip", ctypes.c_void_p), ("norms", ctypes.c_void_p),
                ("packed_indices", ctypes.c_void_p), ("left_signs", ctypes.c_void_p),
                ("right_signs", ctypes.c_void_p), ("permutation", ctypes.c_void_p), ("rotation", ctypes.c_void_p),
                ("expanded", ctypes.c_void_p), ("norm_f32", ctypes.c_void_p)]


ARRAYS = ("codebook", "input_scale", "input_scale_recip", "norms", "packed_indices", "left_signs", "right_signs",
          "permutation", "rotation")


@dataclass
class CQ4Matrix:
    bits: int
    K: int
    N: int
    group_size: int
    num_groups: int
    flags: int
    codebook: np.ndarray                       # uint16 (fp16 bits) [2^bits]
    norms: np.ndarray                          # uint16, stored layout
    packed_indices: np.ndarray                 # uint8
    input_scale: np.ndarray | None = None      # uint16 [K]
    input_scale_recip: np.ndarray | None = None
    left_signs: np.ndarray | None = None       # int8 [group_size]
    right_signs: np.ndarray | None = None
    permutation: np.ndarray | None = None      # uint32 [group_size]
    rotation: np.ndarray | None = None         # uint16 [K][K]
    indices: np.ndarray | None = field(default=None, repr=False)  # logical [N][K] (for tests)

    def struct(self, pointers: dict[str, int] | None = None) -> CQ4Struct:
        """Host struct (pointers into these arrays), or device struct when `pointers` maps names to addresses."""
        s = CQ4Struct(self.bits, self.K, self.N, self.group_size, self.num_groups, self.flags)
        for name in ARRAYS:
            a = getattr(self, name)
            if pointers is not None:
                setattr(s, name, pointers.get(name) if a is not None else None)
            elif a is not None:
                setattr(s, name, a.ctypes.data)
        return s


def lcg(s: int) -> int:
    return (s * 1664525 + 1013904223) & 0xFFFFFFFF


def gen_f32(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    """m6c1_common.h:33-42 (fp32 arithmetic)."""
    out = np.empty(n, np.float32)
    s = seed
    lo32, span = np.float32(lo), np.float32(hi) - np.float32(lo)
    for i in range(n):
        s = lcg(s)
        u = np.float32(s >> 8) * np.float32(1.0 / 16777216.0)
        out[i] = lo32 + u * span
    return out


def gen_signs(n: int, seed: int) -> np.ndarray:
    """test_cq4.cpp:86-94."""
    out = np.empty(n, np.int8)
    s = seed
    for i in range(n):
        s = lcg(s)
        out[i] = 1 if (s >> 8) & 1 else -1
    return out


def gen_permutation(n: int, seed: int) -> np.ndarray:
    """test_cq4.cpp:76-84 (Fisher-Yates with the LCG)."""
    p = np.arange(n, dtype=np.uint32)
    s = seed
    for i in range(n, 1, -1):
        s = lcg(s)
        j = (s >> 8) % i
        p[i - 1], p[j] = p[j], p[i - 1]
    return p


def f16(values: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits, round to nearest even."""
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def pack_lsb(idx: np.ndarray, bits: int, group_size: int) -> np.ndarray:
    """Logical indices [N][K] -> LSB-first bit packing per (row, group) (cactus_x86.cpp:24-43)."""
    N, K = idx.shape
    ng = K // group_size
    pgb = (group_size * bits + 7) // 8
    out = np.zeros(N * ng * pgb, np.uint8)
    for n in range(N):
        for g in range(ng):
            base = (n * ng + g) * pgb
            for k in range(group_size):
                bit = k * bits
                v = int(idx[n, g * group_size + k])
                out[base + bit // 8] |= (v << (bit % 8)) & 0xFF
                if bit % 8 + bits > 8:
                    out[base + bit // 8 + 1] |= v >> (8 - bit % 8)
    return out


def pack_interleaved(idx: np.ndarray, group_size: int) -> np.ndarray:
    """Logical 4-bit indices [N][K] -> 4-row panels per group (test_cq4.cpp:107-130)."""
    N, K = idx.shape
    ng = K // group_size
    pgb = group_size // 2
    out = np.zeros((N // 4) * ng * 4 * pgb, np.uint8)
    for p in range(N // 4):
        for g in range(ng):
            base = (p * ng + g) * 4 * pgb
            for r in range(4):
                for k in range(group_size):
                    b = base + (k // 8) * 16 + r * 4 + (k & 3)
                    v = int(idx[p * 4 + r, g * group_size + k]) & 0xF
                    out[b] |= (v << 4) if (k & 4) else v
    return out


def panel_norms(logical: np.ndarray, N: int, ng: int) -> np.ndarray:
    """[n*ng+g] -> panel-major [(n/4*ng+g)*4 + n%4] (test_cq4.cpp:137-146)."""
    out = np.empty_like(logical)
    for n in range(N):
        for g in range(ng):
            out[((n // 4) * ng + g) * 4 + (n & 3)] = logical[n * ng + g]
    return out


def reference_fixture(name: str) -> tuple[CQ4Matrix, np.ndarray, int]:
    """The five fixtures of test_cq4.cpp:480-484 (run_fixture, :365-425): (matrix, A fp16 bits [M][K], M)."""
    table = {"cq4_interleaved": (64, 64, 128, 1, True, False, False, False),
             "cq4_hadamard_signs": (64, 64, 128, 1, False, True, True, False),
             "cq4_orthogonal": (64, 64, 64, 1, False, False, False, True),
             "cq4_interleaved_multigroup_m1": (1, 64, 128, 4, True, False, False, False),
             "cq4_interleaved_m1_n512": (1, 512, 128, 4, True, False, False, False)}
    M, N, gs, ng, inter, signs_perm, use_scale, orth = table[name]
    bits, K = 4, gs * ng
    seed = 0x0C170000 if orth else 0x0C170100
    codebook = f16(gen_f32(16, seed + 1, -1.0, 1.0))
    norms = f16(gen_f32(N if orth else N * ng, seed + 2, 0.5, 1.5))
    if inter and not orth:
        norms = panel_norms(norms, N, ng)
    scale = recip = None
    if orth or not use_scale:
        recip = f16(gen_f32(K, seed + 3, 0.5, 1.5))
    else:
        scale = f16(gen_f32(K, seed + 3, 0.5, 1.5))
    left = right = perm = None
    if signs_perm:
        left, right, perm = gen_signs(gs, seed + 4), gen_signs(gs, seed + 5), gen_permutation(gs, seed + 6)
    idx = np.empty((N, K), np.uint32)
    s = seed + 7
    for n in range(N):
        for k in range(K):
            s = lcg(s)
            idx[n, k] = (s >> 8) % 16
    packed = pack_interleaved(idx, gs) if inter else pack_lsb(idx, 4, K)
    rotation = f16(gen_f32(K * K, seed + 8, -0.5, 0.5)) if orth else None
    A = f16(gen_f32(M * K, seed + 9, -1.0, 1.0)).reshape(M, K)
    flags = (FLAG_INTERLEAVED_4ROW if inter else 0) | (FLAG_ORTHOGONAL if orth else 0)
    W = CQ4Matrix(bits, K, N, gs, ng, flags, codebook, norms, packed, scale, recip, left, right, perm, rotation, idx)
    return W, A, M


def random_matrix(rng: np.random.Generator, *, bits: int, K: int, N: int, group_size: int, interleaved: bool = False,
                  orthogonal: bool = False, signs: bool = False, perm: bool = False, scale: str = "recip"
                  ) -> CQ4Matrix:
    """A matrix with random fp16 codebook/norms/scales and random indices, in either layout."""
    gs, ng = (K, 1) if orthogonal else (group_size, K // group_size)
    codebook = f16(rng.uniform(-1, 1, 1 << bits))
    logical = f16(rng.uniform(0.5, 1.5, N * ng))
    norms = panel_norms(logical, N, ng) if interleaved else logical
    idx = rng.integers(0, 1 << bits, size=(N, K)).astype(np.uint32)
    packed = pack_interleaved(idx, gs) if interleaved else pack_lsb(idx, bits, gs)
    sc = f16(rng.uniform(0.5, 1.5, K))
    W = CQ4Matrix(bits, K, N, group_size if not orthogonal else K, ng, 0, codebook, norms, packed, indices=idx)
    if scale == "recip":
        W.input_scale_recip = sc
    elif scale == "scale":
        W.input_scale = sc
    if interleaved:
        W.flags |= FLAG_INTERLEAVED_4ROW
    if orthogonal:
        W.flags |= FLAG_ORTHOGONAL
        W.rotation = f16(rng.uniform(-0.5, 0.5, K * K) / np.sqrt(K))
    else:
        if signs:
            W.left_signs = np.where(rng.integers(0, 2, gs) > 0, 1, -1).astype(np.int8)
            W.right_signs = np.where(rng.integers(0, 2, gs) > 0, 1, -1).astype(np.int8)
        if perm:
            W.permutation = rng.permutation(gs).astype(np.uint32)
    return W


def _bind(L: ctypes.CDLL) -> ctypes.CDLL:
    if not getattr(L, "_cq4_bound", False):
        L.oracle_cq4_matmul.argtypes = [ctypes.POINTER(CQ4Struct), _u16p, ctypes.c_uint32,
                                        ctypes.POINTER(ctypes.c_double)]
        L.oracle_cq4_matmul.restype = ctypes.c_int
        L.oracle_cq4_transform.argtypes = [ctypes.POINTER(CQ4Struct), _u16p, ctypes.c_uint32,
                                           ctypes.POINTER(ctypes.c_double)]
        L.oracle_cq4_transform.restype = ctypes.c_int
        L.oracle_f16_to_double.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_double.restype = ctypes.c_double
        L._cq4_bound = True
    return L


def matmul(W: CQ4Matrix, A: np.ndarray, M: int) -> np.ndarray:
    """Oracle C[m][n] in double (not rounded)."""
    L = _bind(_o.lib())
    A = np.ascontiguousarray(A, np.uint16)
    C = np.empty((M, W.N), np.float64)
    s = W.struct()
    if L.oracle_cq4_matmul(ctypes.byref(s), A.ctypes.data_as(_u16p), M,
                           C.ctypes.data_as(ctypes.POINTER(ctypes.c_double))) != 0:
        raise ValueError("oracle_cq4_matmul: invalid matrix")
    return C


def transform(W: CQ4Matrix, A: np.ndarray, M: int) -> np.ndarray:
    L = _bind(_o.lib())
    A = np.ascontiguousarray(A, np.uint16)
    out = np.empty((M, W.K), np.float64)
    s = W.struct()
    if L.oracle_cq4_transform(ctypes.byref(s), A.ctypes.data_as(_u16p), M,
                              out.ctypes.data_as(ctypes.POINTER(ctypes.c_double))) != 0:
        raise ValueError("oracle_cq4_transform: invalid matrix")
    return out


def reference_available() -> bool:
    return REF_LIB.is_file()


def reference_matmul(W: CQ4Matrix, A: np.ndarray, M: int) -> np.ndarray:
    """The reference's own cactus_bridge_quant_matmul (oracle/_ref build): fp16 bits [M][N]."""
    L = ctypes.CDLL(str(REF_LIB))
    fn = L.cactus_bridge_quant_matmul
    fn.argtypes = [ctypes.POINTER(CQ4Struct), _u16p, ctypes.c_uint32, _u16p]
    fn.restype = None
    A = np.ascontiguousarray(A, np.uint16)
    C = np.zeros((M, W.N), np.uint16)
    s = W.struct()
    fn(ctypes.byref(s), A.ctypes.data_as(_u16p), M, C.ctypes.data_as(_u16p))
    return C


def fp16_ulps(got_bits: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """Distance, in units of fp16 spacing at the reference value, between fp16 results and double references."""
    got = np.asarray(got_bits, np.uint16).view(np.float16).astype(np.float64)
    ref = np.asarray(ref, np.float64)
    _, e = np.frexp(np.maximum(np.abs(ref), 2.0 ** -14))
    spacing = np.ldexp(1.0, e - 11)  # fp16 has 11 significant bits
    return np.abs(got - ref) / spacing
