"""CPU checks of the one-row GEMV's integer recoding of x (q4_gemv_pipe_kernel).

The kernel writes X = rint(x * 2^(30 - e_g)) (e_g: max|x| of the 32-value group
< 2^e_g) as eight signed base-16 digits, packs digit j of eight consecutive
values into the nibbles of one word, and forms sum_k v_k X_k as 65536 H + L with
v_dot8_i32_i4. These tests pin the arithmetic facts the kernel relies on: the
digit recoding is exact over the whole range of X, the two partial sums cannot
leave the range where int32 and float are exact, and the representation error
of x stays within 2^-30 of the group's largest magnitude, which keeps whole
projections inside the 1e-5 bar on inputs built to stress it.
"""
from __future__ import annotations

import numpy as np

import cases

BIAS = 0x88888888
DIGITS = 8
FRAC = 30


def signed_nibble(n: np.ndarray) -> np.ndarray:
    n = np.asarray(n, dtype=np.int64) & 0xF
    return np.where(n >= 8, n - 16, n)


def digit_words(X: np.ndarray) -> np.ndarray:
    """X int64 [..., 8] -> uint32 [..., DIGITS]: nibble t of word j = digit j of X[t], as the kernel packs them."""
    Y = ((X.astype(np.int64) + BIAS) & 0xFFFFFFFF) ^ BIAS
    words = np.zeros(X.shape[:-1] + (DIGITS,), dtype=np.int64)
    for j in range(DIGITS):
        for t in range(8):
            words[..., j] |= ((Y[..., t] >> (4 * j)) & 0xF) << (4 * t)
    return words.astype(np.uint32)


def dot8(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Signed 4-bit dot product of two packed words (what v_dot8_i32_i4 computes)."""
    a = a.astype(np.int64)
    b = b.astype(np.int64)
    return sum(signed_nibble(a >> (4 * t)) * signed_nibble(b >> (4 * t)) for t in range(8))


def test_digits_reconstruct_every_x():
    rng = np.random.default_rng(0)
    X = np.concatenate([rng.integers(-(2**30), 2**30 + 1, size=20000),
                        [-(2**30), 2**30, 0, -1, 1, 2**30 - 1, -(2**30) + 1, 0x7777777, -0x8888888]])
    Y = (X + BIAS) & 0xFFFFFFFF
    assert np.all((X + BIAS >= 0) & (X + BIAS < 2**32))        # no wrap: Y is X + bias exactly
    d = np.stack([((Y >> (4 * j)) & 0xF) - 8 for j in range(DIGITS)], axis=-1)
    assert d.min() >= -8 and d.max() <= 7
    assert np.array_equal((d * (16 ** np.arange(DIGITS))).sum(axis=-1), X)
    # the nibble stored is (hex digit of Y) xor 8, whose two's complement value is the digit
    assert np.array_equal(signed_nibble((Y[:, None] >> (4 * np.arange(DIGITS))) ^ 8), d)


def test_partial_sums_stay_exact():
    # largest |H| (or |L|): every v = -8 and every digit -8 over 32 values and four digits
    bound = 32 * 8 * 8 * sum(16**j for j in range(4))
    assert bound == 32 * 8 * 34952 and bound < 2**24
    # brute force on extreme words: 65536 H + L equals sum v X exactly
    rng = np.random.default_rng(1)
    for _ in range(200):
        v = rng.choice([-8, -7, 0, 7], size=32)
        X = rng.choice([-(2**30), 2**30, 0, 12345, -(2**29) - 7], size=32)
        wv = np.zeros(4, np.int64)
        for w in range(4):
            for t in range(8):
                wv[w] |= (int(v[8 * w + t]) & 0xF) << (4 * t)
        xd = digit_words(X.reshape(4, 8))                    # [word, digit]
        H = L = 0
        for j in range(DIGITS - 1, -1, -1):
            part = int(sum(dot8(wv[w], xd[w, j]) for w in range(4)))
            if j >= 4:
                H = H * 16 + part
                assert abs(H) < 2**24
            else:
                L = L * 16 + part
                assert abs(L) < 2**24
        assert 65536 * H + L == int(np.dot(v, X))


def recoded(x: np.ndarray) -> np.ndarray:
    m, k = x.shape
    g = x.reshape(m, k // 32, 32).astype(np.float64)
    e = np.frexp(np.abs(g).max(axis=2).astype(np.float32))[1].astype(np.float64)
    X = np.rint(g * np.exp2(FRAC - e)[..., None])
    assert np.abs(X).max() <= 2**FRAC
    return (X * np.exp2(e - FRAC)[..., None]).reshape(m, k)


def test_representation_error_bound():
    c = cases.make_case(4, 1, 4096)
    x = c.x.copy()
    x[:, 100] = 1e4
    x[:, 200:232] *= 1e-38
    xr = recoded(x)
    gmax = np.repeat(np.abs(x.reshape(4, 128, 32)).max(axis=2), 32, axis=1).astype(np.float64)
    assert np.all(np.abs(xr - x) <= gmax * 2.0**-FRAC)


def test_stress_inputs_stay_within_the_bar():
    """Groups of zeros, subnormals, 1e30, an outlier among small values and exact powers of
    two, and outlier channels up to 1e4: the recoding alone moves results by far less than 1e-5."""
    n, k = 300, 4096
    c = cases.make_case(2, n, k)
    dq = c.b.astype(np.float64) * np.repeat(c.scales.T.astype(np.float64), 32, axis=0)
    x = c.x.copy()
    x[:, 0:32] = 0.0
    x[:, 32:64] *= 1e-41
    x[:, 64:96] *= 1e30
    x[:, 96:128] *= 1e-3
    x[:, 100] = 1000.0
    x[:, 128:160] = np.float32(2.0) ** np.arange(-8, 24, dtype=np.float32)
    x[:, [1007, 2049, 4000]] = 1e4
    ref = x.astype(np.float64) @ dq
    got = recoded(x) @ dq
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) < 1e-6
