"""CQ4 codebook matmul: pinning the CPU oracle (oracle/cq4_oracle.c) and the C-ABI's argument checks.

The oracle restates cactus_quant_matmul (vulkan-runtime/src/cactus/cactus_x86.cpp:
133-240, 384-397) in double precision. It is pinned by
  - the reference's own library, compiled from its sources into oracle/_ref/ (when
    present), on the reference test's five fixtures (test_cq4.cpp:480-484, rebuilt
    from its generators) and on random matrices of every bit width and layout: the
    reference rounds an fp32 sum to fp16, so the oracle's double result, rounded to
    fp16, must equal it except where fp32 rounding decides (and stay within the
    reference test's own bar everywhere);
  - an independent numpy restatement: Sylvester Hadamard matrix from scipy, a dense
    decoded weight matrix from the logical indices, and one matrix product;
  - a closed form: orthogonal mode with an identity rotation and the codebook
    v - 8 is the int4 GEMM of the q4 oracle with one scale per column.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import scipy.linalg

from oracle import cq4

FIXTURES = ["cq4_interleaved", "cq4_hadamard_signs", "cq4_orthogonal", "cq4_interleaved_multigroup_m1",
            "cq4_interleaved_m1_n512"]

needs_ref = pytest.mark.skipif(not cq4.reference_available(), reason="oracle/_ref not built (no reference sources)")


def reference_bar(got_bits: np.ndarray, ref: np.ndarray) -> bool:
    """test_cq4.cpp:422 via m6c1_common.h:286-304: fail only where |d| > 2e-2 and |d| > 1e-2 |ref|."""
    g = got_bits.view(np.float16).astype(np.float64)
    err = np.abs(g - ref)
    return bool(np.all((err <= 2e-2) | (err <= 1e-2 * np.abs(ref))))


def decoded_dense(W: cq4.CQ4Matrix) -> np.ndarray:
    """[K][N] float64: codebook value * norm, from the logical indices (test-side restatement)."""
    cb = W.codebook.view(np.float16).astype(np.float64)
    orth = bool(W.flags & cq4.FLAG_ORTHOGONAL)
    inter = bool(W.flags & cq4.FLAG_INTERLEAVED_4ROW)
    gs, ng = (W.K, 1) if orth else (W.group_size, W.num_groups)
    norms = W.norms.view(np.float16).astype(np.float64)
    out = np.empty((W.K, W.N))
    for n in range(W.N):
        for g in range(ng):
            ni = ((n // 4) * ng + g) * 4 + (n & 3) if inter else n * ng + g
            out[g * gs:(g + 1) * gs, n] = cb[W.indices[n, g * gs:(g + 1) * gs]] * norms[ni]
    return out


def numpy_transform(W: cq4.CQ4Matrix, A: np.ndarray) -> np.ndarray:
    a = A.view(np.float16).astype(np.float64)
    if W.input_scale_recip is not None:
        a = a * W.input_scale_recip.view(np.float16).astype(np.float64)
    elif W.input_scale is not None:
        a = a / W.input_scale.view(np.float16).astype(np.float64)
    if W.flags & cq4.FLAG_ORTHOGONAL:
        return a @ W.rotation.view(np.float16).astype(np.float64).reshape(W.K, W.K)
    gs = W.group_size
    H = scipy.linalg.hadamard(gs).astype(np.float64) / np.sqrt(gs)  # Sylvester order = the in-place butterflies
    out = np.empty_like(a)
    for g in range(W.num_groups):
        x = a[:, g * gs:(g + 1) * gs]
        if W.left_signs is not None:
            x = x * W.left_signs
        y = x @ H.T
        if W.right_signs is not None:
            y = y * W.right_signs
        if W.permutation is not None:
            y = y[:, W.permutation]
        out[:, g * gs:(g + 1) * gs] = y
    return out


def random_case(seed: int, **kw) -> tuple[cq4.CQ4Matrix, np.ndarray, int]:
    rng = np.random.default_rng(seed)
    m = kw.pop("m", 5)
    W = cq4.random_matrix(rng, **kw)
    A = cq4.f16(rng.uniform(-1, 1, (m, W.K)))
    return W, A, m


RANDOM = [dict(bits=4, K=256, N=24, group_size=64, signs=True, perm=True, scale="scale"),
          dict(bits=3, K=256, N=20, group_size=128, signs=True),
          dict(bits=2, K=128, N=12, group_size=32, perm=True),
          dict(bits=1, K=64, N=8, group_size=64, scale="none"),
          dict(bits=4, K=512, N=16, group_size=128, interleaved=True),
          dict(bits=4, K=96, N=8, group_size=96, orthogonal=True),
          dict(bits=3, K=64, N=8, group_size=64, orthogonal=True, scale="none"),
          dict(bits=4, K=256, N=8, group_size=256, signs=True, perm=True, m=1)]


@needs_ref
@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_matches_reference_library_on_its_fixtures(name):
    W, A, M = cq4.reference_fixture(name)
    ref16 = cq4.reference_matmul(W, A, M)
    mine = cq4.matmul(W, A, M)
    assert reference_bar(ref16, mine)
    assert np.mean(ref16 == cq4.f16(mine)) >= 0.99


@needs_ref
@pytest.mark.parametrize("case", range(len(RANDOM)))
def test_oracle_matches_reference_library_on_random_matrices(case):
    W, A, M = random_case(100 + case, **dict(RANDOM[case]))
    ref16 = cq4.reference_matmul(W, A, M)
    mine = cq4.matmul(W, A, M)
    assert reference_bar(ref16, mine)
    assert np.mean(ref16 == cq4.f16(mine)) >= 0.98


@pytest.mark.parametrize("case", range(len(RANDOM)))
def test_oracle_matches_numpy_restatement(case):
    W, A, M = random_case(200 + case, **dict(RANDOM[case]))
    t = cq4.transform(W, A, M)
    np.testing.assert_allclose(t, numpy_transform(W, A), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(cq4.matmul(W, A, M), t @ decoded_dense(W), rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_rebuild_matches_numpy_restatement(name):
    W, A, M = cq4.reference_fixture(name)
    np.testing.assert_allclose(cq4.matmul(W, A, M), numpy_transform(W, A) @ decoded_dense(W), rtol=1e-11, atol=1e-11)


def test_orthogonal_identity_rotation_is_the_int4_gemm():
    from oracle import oracle as o

    rng = np.random.default_rng(7)
    K, N, M = 128, 16, 3
    W = cq4.random_matrix(rng, bits=4, K=K, N=N, group_size=K, orthogonal=True, scale="none")
    W.codebook = cq4.f16(np.arange(16) - 8.0)                        # value = index - 8: an int4 nibble
    W.rotation = cq4.f16(np.eye(K))
    A = cq4.f16(rng.uniform(-1, 1, (M, K)))
    v = W.indices.astype(np.int64) - 8                                # [N][K]
    packed = o.pack_q4(v.T.astype(np.int8))                           # the q4 layout of the same weights
    norms = W.norms.view(np.float16).astype(np.float32)
    scales = np.repeat(norms[:, None], K // 32, axis=1)               # one scale per column, every group
    want = o.q4gemm_packed(A.view(np.float16).astype(np.float32), packed, scales)
    np.testing.assert_allclose(cq4.matmul(W, A, M), want, rtol=1e-12, atol=1e-12)


def test_index_extraction_exhaustive():
    rng = np.random.default_rng(3)
    for bits in (1, 2, 3, 4):
        idx = rng.integers(0, 1 << bits, size=(1, 64)).astype(np.uint32)
        packed = cq4.pack_lsb(idx, bits, 64)
        L = cq4._bind(cq4._o.lib())
        L.oracle_cq4_index_lsb.argtypes = [ctypes.POINTER(ctypes.c_uint8), ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_cq4_index_lsb.restype = ctypes.c_uint32
        got = [L.oracle_cq4_index_lsb(packed.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), k, bits) for k in range(64)]
        assert got == list(idx[0])
    idx = rng.integers(0, 16, size=(4, 32)).astype(np.uint32)
    panel = cq4.pack_interleaved(idx, 32)
    L.oracle_cq4_index_interleaved.argtypes = [ctypes.POINTER(ctypes.c_uint8), ctypes.c_uint32, ctypes.c_uint32]
    L.oracle_cq4_index_interleaved.restype = ctypes.c_uint32
    for r in range(4):
        got = [L.oracle_cq4_index_interleaved(panel.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), r, k)
               for k in range(32)]
        assert got == list(idx[r])


def test_f16_decode_exhaustive():
    L = cq4._bind(cq4._o.lib())
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float64)
    got = np.array([L.oracle_f16_to_double(int(b)) for b in bits])
    finite = np.isfinite(want)
    assert np.array_equal(got[finite], want[finite])
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.array_equal(np.isinf(got), np.isinf(want))


# -- the C-ABI rejects what it does not define, before touching a device ----------------------------

def test_abi_cq4_validation(session):
    from spaceslug_amd import BackendError

    W, A, M = random_case(1, **dict(RANDOM[0]))
    base = dict(bits=W.bits, K=W.K, N=W.N, group_size=W.group_size, num_groups=W.num_groups, flags=W.flags,
                codebook=W.codebook, norms=W.norms, packed_indices=W.packed_indices, a=A, m=M,
                input_scale=W.input_scale, left_signs=W.left_signs, right_signs=W.right_signs,
                permutation=W.permutation)
    bad = [dict(bits=0), dict(bits=5), dict(m=0), dict(m=65536), dict(num_groups=3), dict(group_size=48, num_groups=16,
           K=768), dict(group_size=512, num_groups=1, K=512), dict(flags=cq4.FLAG_INTERLEAVED_4ROW, bits=3),
           dict(codebook=None), dict(permutation=np.full(64, 64, np.uint32)),
           dict(flags=cq4.FLAG_ORTHOGONAL)]  # orthogonal without a rotation
    for change in bad:
        args = {**base, **change}
        if "K" in change or "m" in change:
            args["a"] = np.zeros((max(1, args["m"]), args["K"]), np.uint16)
        with pytest.raises(BackendError, match="returned 1"):
            session.cq4_matmul_values(**args)
