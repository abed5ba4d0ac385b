"""Pins for the CPU oracle (runs without a GPU).

Each check is independent of the oracle's own formula: published constants,
hand-derived bytes from the layout comments, exact rational arithmetic, an
integer GEMM done by numpy, and algebraic invariants of the contraction.
"""
from __future__ import annotations

import struct
from fractions import Fraction

import numpy as np
import pytest

from cases import make_case, reference_kat_case

# Numerical Recipes (2nd ed., sec. 7.1, "ranqd1"): the quick-and-dirty generator
# idum = 1664525 * idum + 1013904223 started from idum = 0 yields these values.
NR_SEQUENCE_FROM_ZERO = [0x3C6EF35F, 0x47502932, 0xD1CCF6E9, 0xAAF95334, 0x6252E503, 0x9F2EC686,
                         0x57FE6C2D, 0xA3D95FA8, 0x81FDBEE7, 0x94F0AF1A, 0xCBF633B1]


def test_lcg_matches_numerical_recipes(oracle):
    s = 0
    for expected in NR_SEQUENCE_FROM_ZERO:
        s = oracle.lcg_next(s)
        assert s == expected


def test_generate_int4_from_published_sequence(oracle):
    # (s >> 8) % 16 is the third-lowest hex digit of each published value, minus 8.
    expected = [0x3 - 8, 0x9 - 8, 0x6 - 8, 0x3 - 8, 0x5 - 8, 0x6 - 8, 0xC - 8, 0xF - 8, 0xE - 8, 0xF - 8, 0x3 - 8]
    assert oracle.generate_int4(11, 0).tolist() == expected


def test_generate_floats_unit_interval_is_top_24_bits(oracle):
    v = oracle.generate_floats(len(NR_SEQUENCE_FROM_ZERO), 0, 0.0, 1.0)
    assert (v.astype(np.float64) * 2.0**24).tolist() == [float(s >> 8) for s in NR_SEQUENCE_FROM_ZERO]


def test_generate_floats_range_and_determinism(oracle):
    a = oracle.generate_floats(100000, 0x13579BDF, 0.01, 0.05)
    b = oracle.generate_floats(100000, 0x13579BDF, 0.01, 0.05)
    assert np.array_equal(a, b)
    assert a.min() >= np.float32(0.01) and a.max() <= np.float32(0.05)
    assert abs(float(a.mean()) - 0.03) < 1e-3


def test_generate_int4_covers_all_values_uniformly(oracle):
    v = oracle.generate_int4(160000, 0x9ABCDEF0)
    counts = np.bincount(v.astype(np.int64) + 8, minlength=16)
    assert v.min() == -8 and v.max() == 7
    assert np.all(np.abs(counts - 10000) < 600)


def test_generate_normal_moments(oracle):
    z = oracle.generate_normal(1_000_001, 0x12345678, 0.0, 1.0).astype(np.float64)
    assert abs(z.mean()) < 5e-3
    assert abs(z.std() - 1.0) < 5e-3
    assert np.isfinite(z).all()
    # fourth moment of N(0,1) is 3
    assert abs((z**4).mean() - 3.0) < 0.05
    w = oracle.generate_normal(10_000, 0x12345678, 0.0, 0.02).astype(np.float64)
    assert np.allclose(w, oracle.generate_normal(10_000, 0x12345678, 0.0, 1.0).astype(np.float64) * 0.02, rtol=1e-6,
                       atol=1e-9)


def test_pack_hand_derived_bytes(oracle):
    # q4gemm.comp:9-16: nibble = v & 0xF (-8 -> 0x8, -1 -> 0xF, 0 -> 0x0, 7 -> 0x7), even k low
    # nibble, odd k high nibble, byte index n*(K/2) + k/2.
    b = np.array([[-8, 1],
                  [7, -1],
                  [0, -2],
                  [-1, 3]], dtype=np.int8)
    packed = oracle.pack_q4(b)
    assert packed.ravel().tolist() == [0x78, 0xF0, 0xF1, 0x3E]
    # Byte pb lives in 32-bit word pb >> 2, lane pb & 3 (little-endian): the reference's word.
    assert struct.unpack("<I", packed.tobytes())[0] == 0x3EF1F078


def test_pack_matches_reference_word_formula_all_lanes(oracle):
    # Build the reference's uint32 words with its own arithmetic (word = pb >> 2,
    # lane = pb & 3, bits shift + lane*8) from the layout comments, for every nibble
    # value in both positions and all four byte lanes, then compare byte images.
    K, N = 32, 16
    vals = np.arange(-8, 8, dtype=np.int8)
    b = np.empty((K, N), dtype=np.int8)
    for n in range(N):
        for k in range(K):
            b[k, n] = vals[(k * 5 + n * 3 + (k // 2) * 7) % 16]
    words = [0] * (K * N // 8)
    for n in range(N):
        for k in range(K):
            nib = int(b[k, n]) & 0xF
            pb = n * (K // 2) + (k >> 1)
            words[pb >> 2] |= nib << ((k & 1) * 4 + (pb & 3) * 8)
    ref_bytes = struct.pack("<%dI" % len(words), *words)
    assert oracle.pack_q4(b).tobytes() == ref_bytes
    # every (value, position, lane) combination occurred
    seen = {(int(b[k, n]), k & 1, (n * (K // 2) + (k >> 1)) & 3) for n in range(N) for k in range(K)}
    assert len(seen) == 16 * 2 * 4


def test_pack_unpack_roundtrip_exhaustive(oracle):
    # all 256 (low, high) nibble pairs in one column
    lo, hi = np.meshgrid(np.arange(-8, 8), np.arange(-8, 8), indexing="ij")
    col = np.stack([lo.ravel(), hi.ravel()], axis=1).ravel().astype(np.int8)  # k-order
    b = col.reshape(-1, 1)
    packed = oracle.pack_q4(b)
    assert sorted(packed.ravel().tolist()) == list(range(256))
    assert np.array_equal(oracle.unpack_q4(packed, b.shape[0], 1), b)
    rnd = oracle.generate_int4(96 * 40, 7).reshape(96, 40)
    assert np.array_equal(oracle.unpack_q4(oracle.pack_q4(rnd), 96, 40), rnd)


def test_pack_rejects_odd_k(oracle):
    with pytest.raises(ValueError):
        oracle.pack_q4(np.zeros((3, 2), dtype=np.int8))


def _exact(a, b, s):
    M, K = a.shape
    N = b.shape[1]
    out = []
    for m in range(M):
        row = []
        for n in range(N):
            acc = Fraction(0)
            for k in range(K):
                acc += Fraction(float(a[m, k])) * int(b[k, n]) * Fraction(float(s[n, k // 32]))
            row.append(acc)
        out.append(row)
    return out


@pytest.mark.parametrize("shape", [(1, 1, 32), (2, 3, 64), (3, 2, 96)])
def test_reference_against_exact_rationals(oracle, shape):
    M, N, K = shape
    c = make_case(M, N, K)
    got = oracle.q4gemm_ref(c.x, c.b, c.scales)
    exact = _exact(c.x, c.b, c.scales)
    for m in range(M):
        for n in range(N):
            absum = sum(abs(float(c.x[m, k]) * int(c.b[k, n]) * float(c.scales[n, k // 32])) for k in range(K))
            bound = K * 2.0**-53 * absum
            assert abs(Fraction(got[m, n]) - exact[m][n]) <= Fraction(bound)


def test_reference_integer_gemm_matches_numpy(oracle):
    # With every scale 1 and integer activations the contraction is an integer GEMM.
    M, N, K = 7, 33, 128
    rng = np.random.default_rng(3)
    a = rng.integers(-50, 51, size=(M, K)).astype(np.float32)
    b = oracle.generate_int4(K * N, 11).reshape(K, N)
    s = np.ones((N, K // 32), dtype=np.float32)
    want = a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(oracle.q4gemm_ref(a, b, s), want.astype(np.float64))
    assert np.array_equal(oracle.q4gemm_packed(a, oracle.pack_q4(b), s), want.astype(np.float64))


def test_reference_unit_vector_selects_dequantized_row(oracle):
    M, N, K = 1, 24, 96
    c = make_case(M, N, K)
    for k in (0, 1, 31, 32, 33, 95):
        e = np.zeros((1, K), dtype=np.float32)
        e[0, k] = 1.0
        want = c.b[k, :].astype(np.float64) * c.scales[:, k // 32].astype(np.float64)
        assert np.array_equal(oracle.q4gemm_ref(e, c.b, c.scales)[0], want)
        assert np.array_equal(oracle.q4gemm_packed(e, c.packed, c.scales)[0], want)


def test_reference_single_nonzero_nibble_selects_column_and_group(oracle):
    M, N, K = 3, 5, 64
    c = make_case(M, N, K)
    b = np.zeros((K, N), dtype=np.int8)
    b[40, 3] = -8  # column 3, group 1
    got = oracle.q4gemm_packed(c.x, oracle.pack_q4(b), c.scales)
    want = np.zeros((M, N))
    want[:, 3] = c.x[:, 40].astype(np.float64) * -8.0 * float(c.scales[3, 1])
    assert np.array_equal(got, want)


def test_reference_invariants(oracle):
    c = make_case(4, 20, 128)
    base = oracle.q4gemm_ref(c.x, c.b, c.scales)
    # power-of-two scaling of activations or scales is exact
    assert np.array_equal(oracle.q4gemm_ref(c.x * np.float32(2), c.b, c.scales), 2 * base)
    assert np.array_equal(oracle.q4gemm_ref(c.x, c.b, c.scales * np.float32(0.5)), 0.5 * base)
    # negating the weights (all but -8, which has no int4 negation) negates the result
    b2 = np.where(c.b == -8, 0, c.b).astype(np.int8)
    assert np.array_equal(oracle.q4gemm_ref(c.x, (-b2).astype(np.int8), c.scales),
                          -oracle.q4gemm_ref(c.x, b2, c.scales))
    # linearity in x
    c2 = make_case(4, 20, 128, seed_a=99)
    lin = oracle.q4gemm_ref(c.x + c2.x, c.b, c.scales)
    assert np.allclose(lin, base + oracle.q4gemm_ref(c2.x, c.b, c.scales), rtol=1e-6, atol=1e-6)
    # columns are independent: permuting weight columns permutes outputs exactly
    perm = np.random.default_rng(5).permutation(20)
    assert np.array_equal(oracle.q4gemm_ref(c.x, c.b[:, perm], c.scales[perm]), base[:, perm])


def test_packed_reference_bit_identical_to_unpacked(oracle):
    c = make_case(17, 40, 96)
    ref = oracle.q4gemm_ref(c.x, c.b, c.scales)
    assert np.array_equal(oracle.q4gemm_packed(c.x, c.packed, c.scales), ref)
    assert np.array_equal(oracle.q4gemm_packed(c.x, c.packed, c.scales, threads=4), ref)
    assert np.array_equal(oracle.q4gemm_packed(c.x, c.packed, c.scales, rows=(5, 12)), ref[5:12])


def test_reference_kat_inputs_are_consistent(oracle):
    c = reference_kat_case()
    assert c.x.min() >= -1.0 and c.x.max() < 1.0
    assert c.scales.min() >= 0.5 and c.scales.max() <= 1.5
    ref = oracle.q4gemm_ref(c.x, c.b, c.scales)
    assert np.array_equal(oracle.q4gemm_packed(c.x, c.packed, c.scales, threads=4), ref)


def test_lora_reference(oracle):
    M, N, K, R = 3, 8, 64, 4
    c = make_case(M, N, K)
    la = oracle.generate_normal(K * R, 1, 0.0, 0.02).reshape(K, R)
    lb = oracle.generate_normal(R * N, 2, 0.0, 0.02).reshape(R, N)
    base = oracle.q4gemm_packed(c.x, c.packed, c.scales)
    # zero adapter leaves the base projection untouched
    assert np.array_equal(oracle.q4gemm_lora(c.x, c.packed, c.scales, np.zeros_like(la), lb, 2.0), base)
    got = oracle.q4gemm_lora(c.x, c.packed, c.scales, la, lb, 2.0)
    # exact rational delta
    for m in range(M):
        for n in range(N):
            delta = Fraction(0)
            for r in range(R):
                t = sum(Fraction(float(c.x[m, k])) * Fraction(float(la[k, r])) for k in range(K))
                delta += t * Fraction(float(lb[r, n]))
            assert abs(got[m, n] - base[m, n] - 2.0 * float(delta)) <= 1e-12 * (1 + abs(float(delta)))


def test_compare_metric(oracle):
    exp = np.array([0.5, 10.0, -3.0, 0.0])
    assert oracle.compare(exp.astype(np.float32), exp, 1e-3)["status"] == "pass"
    # |err| / max(1, |ref|): 2e-3 at |ref| = 0.5 fails, 5e-3 at |ref| = 10 passes (5e-4)
    act = np.array([0.502, 10.005, -3.0, 0.0], dtype=np.float32)
    rep = oracle.compare(act, exp, 1e-3)
    assert rep["status"] == "fail" and rep["first_bad_index"] == 0 and rep["bad_count"] == 1
    assert abs(rep["max_relative_error"] - 2e-3) < 1e-6
    act2 = np.array([0.5, 10.005, -3.0, 0.0], dtype=np.float32)
    assert oracle.compare(act2, exp, 1e-3)["status"] == "pass"
    nan = np.array([0.5, np.nan, -3.0, 0.0], dtype=np.float32)
    rep = oracle.compare(nan, exp, 1e-3)
    assert rep["status"] == "fail" and rep["first_bad_index"] == 1


def test_reference_nonfinite_x_follows_ieee(oracle):
    """An infinite x term is x * (v * s) as q4gemm_ref forms it (test_q4gemm.cpp:102-119):
    NaN against a zero nibble, +-inf with the sign of x * v otherwise; opposite infinities in
    one row give NaN, and a NaN anywhere in the row gives NaN. Hand-derived for K = 64."""
    K, N = 64, 4
    b = np.zeros((K, N), dtype=np.int8)
    b[0] = [0, 3, -2, 5]     # x[0] = +inf meets these nibbles
    b[40] = [1, 1, 2, -1]    # x[40] = -inf in row 1 (second group) meets these
    b[7] = [7, -8, 1, 1]     # a finite term everywhere
    scales = np.full((N, K // 32), 0.5, dtype=np.float32)
    x = np.zeros((3, K), dtype=np.float32)
    x[0, 0] = np.inf
    x[0, 7] = 2.0
    x[1, 0] = np.inf
    x[1, 40] = -np.inf
    x[2, 7] = np.nan
    got = oracle.q4gemm_packed(x, oracle.pack_q4(b), scales)
    nan, inf = np.nan, np.inf
    want = np.array([[nan, inf, -inf, inf],      # column 0: inf * 0
                     [nan, nan, -inf, inf],      # col 1: +inf*3, -inf*1; col 2: +inf*-2, -inf*2
                     [nan, nan, nan, nan]])
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    np.testing.assert_array_equal(got[fin], want[fin])
