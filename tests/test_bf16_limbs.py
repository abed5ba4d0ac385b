"""Arithmetic facts behind the bf16-limb MFMA paths, checked on the CPU.

The wide int4 GEMM (v_mfma_f32_32x32x16_bf16) and the CQ4 MFMA GEMM (v_mfma_f32_16x16x32_bf16) feed
the matrix cores with x split into three bf16 limbs (split_bf16_limbs in q4_device.hpp: b0 = x
truncated to its top 8 significant bits,
b1 = (x - b0) truncated the same way, b2 = x - b0 - b1) and, for CQ4, each fp16 codebook value split
into two limbs (top 8 significant bits and the rest). The kernels' products are exact when
  - b0 + b1 + b2 == x (both subtractions exact, b2 representable in bf16), which holds for every
    fp32 x whose lowest significant bit is at least 2^-133, bf16's subnormal resolution: all x with
    |x| >= 2^-110, and zero. Below that the split drops at most 2^-133 of x (absolute), which is far
    below any output's bar of 1e-5 * max(1, |ref|);
  - every limb is a bf16 (its fp32 bit pattern has 16 zero low bits);
  - a limb times a weight v/16 (v in -8..7), or times a codebook limb, is exact in fp32.
These are checked here over random values of every magnitude, subnormals, the extremes of the fp32
range, and all finite fp16 values. The split is restated in numpy from the rule above.
"""
from __future__ import annotations

import numpy as np


def split3(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    x = np.asarray(x, np.float32)
    mask = np.uint32(0xFFFF0000)
    b0 = (x.view(np.uint32) & mask).view(np.float32)
    r1 = (x - b0).astype(np.float32)
    b1 = (r1.view(np.uint32) & mask).view(np.float32)
    b2 = (r1 - b1).astype(np.float32)
    return b0, b1, b2


def is_bf16(v: np.ndarray) -> bool:
    return bool(np.all((np.asarray(v, np.float32).view(np.uint32) & np.uint32(0xFFFF)) == 0))


def test_three_limbs_sum_exactly_to_x_down_to_bf16_resolution():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    special = np.array([0.0, -0.0, 1.0, -1.0, np.finfo(np.float32).max, -np.finfo(np.float32).max,
                        np.finfo(np.float32).tiny, np.float32(2.0**-149), np.float32(-(2.0**-149)),
                        np.float32(2.0**-126 - 2.0**-149), np.float32(1.0 + 2.0**-23), np.float32(3.0e38),
                        np.float32(1e-30), np.float32(-7.123456e-41)], np.float32)
    x = np.concatenate([x, special, rng.standard_normal(100_000).astype(np.float32)])
    b0, b1, b2 = split3(x)
    # the kernels keep the high 16 bits of each limb's fp32 pattern
    k0, k1, k2 = (((v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)) for v in (b0, b1, b2))
    assert is_bf16(b0) and is_bf16(b1)
    total = k0.astype(np.float64) + k1.astype(np.float64) + k2.astype(np.float64)
    exact = (np.abs(x) >= np.float32(2.0**-110)) | (x == 0)
    assert exact.sum() > 300_000
    assert np.array_equal(b2[exact], k2[exact])  # b2 is a bf16 there
    assert np.array_equal(total[exact], x.astype(np.float64)[exact])
    assert np.max(np.abs(total[~exact] - x.astype(np.float64)[~exact])) <= 2.0**-133
    # truncation: no limb exceeds x in magnitude, so nothing rounds past the fp32 range
    assert np.all(np.abs(b0) <= np.abs(x))


def test_limb_times_weight_is_exact_in_fp32():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(50_000) * np.exp2(rng.integers(-60, 60, 50_000))).astype(np.float32)
    weights = (np.arange(-8, 8, dtype=np.float32) / 16.0).astype(np.float32)
    assert is_bf16(weights)
    for limb in split3(x):
        prod64 = limb.astype(np.float64)[:, None] * weights.astype(np.float64)[None, :]
        prod32 = (limb[:, None] * weights[None, :]).astype(np.float32)
        assert np.array_equal(prod32.astype(np.float64), prod64)


def test_fp16_codebook_values_split_into_two_exact_bf16_limbs():
    h = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = h[np.isfinite(h)].astype(np.float32)
    assert v.size == 63488
    mask = np.uint32(0xFFFF0000)
    hi = (v.view(np.uint32) & mask).view(np.float32)
    lo = (v - hi).astype(np.float32)
    assert is_bf16(hi) and is_bf16(lo)
    assert np.array_equal(hi.astype(np.float64) + lo.astype(np.float64), v.astype(np.float64))
    # an activation limb times a codebook limb is exact in fp32 (8 + 8 significant bits)
    rng = np.random.default_rng(3)
    a = split3(rng.standard_normal(2000).astype(np.float32))
    for limb in a:
        for c in (hi[::31], lo[::31]):
            p64 = limb.astype(np.float64)[:, None] * c.astype(np.float64)[None, :]
            p32 = (limb[:, None] * c[None, :]).astype(np.float32)
            # exact unless the product underflows the fp32 range (values far below any output's spacing)
            normal = np.abs(p64) >= np.finfo(np.float32).tiny
            assert np.array_equal(p32.astype(np.float64)[normal], p64[normal])


def test_a_dropped_limb_is_detected():
    """The exactness check above is sensitive: leaving out the smallest limb breaks it."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(10_000).astype(np.float32)
    b0, b1, _ = split3(x)
    assert not np.array_equal(b0.astype(np.float64) + b1.astype(np.float64), x.astype(np.float64))
