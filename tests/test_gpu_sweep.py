"""Seeded random shapes through every int4 GEMM path against the oracle, at the stated tolerances.

One decode GEMV row (K up to 4096, and 4128..32768 on its K-split form), the small-batch kernel
(2..32 rows, K up to 6400), the wide and mid-size MFMA kernels (33..700 rows, K up to 8192, with
and without K-splits), and LoRA calls on both sides of 32 rows (ranks 1..64), each drawn with the
workload distributions (N(0, 1) x, scales
in [0.01, 0.05]) or the reference KAT's ranges (x in [-1, 1), scales in [0.5, 1.5);
test_q4gemm.cpp:168-176). Bars: 1e-5 up to 32 rows (exact group sums), 6e-6 * sqrt(K / 32)
(at least 1e-5) above, as the header states them.
"""
from __future__ import annotations

import math
import os
import random

import numpy as np
import pytest

from cases import lora_factors, make_case

pytestmark = pytest.mark.gpu

KINDS = ("gemv", "small", "wide", "mid", "lora", "lora_small")


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def draw(rng: random.Random, kind: str) -> tuple[int, int, int]:
    if kind == "gemv":
        return 1, rng.randint(1, 3000), 32 * rng.randint(1, 128)
    if kind == "small":
        return rng.randint(2, 32), rng.randint(1, 1500), 32 * rng.randint(1, 200)
    if kind == "mid":
        return rng.randint(33, 700), rng.randint(1, 900), 64 * rng.randint(1, 64)
    if kind == "lora_small":
        return rng.randint(1, 32), rng.randint(1, 600), 32 * rng.randint(1, 130)
    return rng.randint(33, 700), rng.randint(1, 900), 32 * rng.randint(1, 256)


def cases(seed: int, count: int):
    rng = random.Random(seed)
    out = []
    for i in range(count):
        kind = KINDS[i % len(KINDS)]
        m, n, k = draw(rng, kind)
        dist = rng.choice(("normal", "uniform"))
        rank = rng.randint(1, 64) if kind.startswith("lora") else 0
        out.append((kind, m, n, k, dist, rank, rng.getrandbits(32), rng.getrandbits(32), rng.getrandbits(32)))
    return out


@pytest.mark.parametrize("case", cases(0x5EED, 72), ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-{c[4]}-r{c[5]}")
def test_random_shapes_match_oracle(session, oracle, gpu, case):
    kind, m, n, k, dist, rank, sa, sb, ss = case
    note(f"sweep {kind} m={m} n={n} k={k} {dist} r={rank}")
    scale_range = (0.01, 0.05) if dist == "normal" else (0.5, 1.5)
    c = make_case(m, n, k, x_dist=dist, scale_range=scale_range, seed_a=sa, seed_b=sb, seed_s=ss)
    bar = 1e-5 if m <= 32 else max(1e-5, 6e-6 * math.sqrt(k / 32))
    threads = min(16, os.cpu_count() or 1)
    if rank:
        la, lb = lora_factors(k, n, rank)
        scale = 32.0 / rank
        got = session.q4gemm_lora_values(c.x, c.packed, c.scales, la, lb, m, n, k, rank, scale)
        want = oracle.q4gemm_lora(c.x, c.packed, c.scales, la, lb, scale, threads=threads)
    else:
        got = session.q4gemm_values(c.x, c.packed, c.scales, m, n, k)
        want = oracle.q4gemm_packed(c.x, c.packed, c.scales, threads=threads)
    assert got.shape == (m, n) and np.all(np.isfinite(got))
    rep = oracle.compare(got, want, bar)
    assert rep["status"] == "pass", (case, rep["max_relative_error"], bar)


def long_k_cases(seed: int, count: int):
    rng = random.Random(seed)
    return [(rng.randint(1, 5000), 32 * rng.randint(129, 1024), rng.choice(("normal", "uniform")), rng.getrandbits(32),
             rng.getrandbits(32), rng.getrandbits(32)) for _ in range(count)]


@pytest.mark.parametrize("case", long_k_cases(0x10C4, 16), ids=lambda c: f"gemv-1x{c[0]}x{c[1]}-{c[2]}")
def test_random_long_k_rows_match_oracle(session, oracle, gpu, case):
    """One row with K from 4128 to 32768 (the K-split decode GEMV), at the 1e-5 bar."""
    n, k, dist, sa, sb, ss = case
    note(f"sweep gemv-long m=1 n={n} k={k} {dist}")
    scale_range = (0.01, 0.05) if dist == "normal" else (0.5, 1.5)
    c = make_case(1, n, k, x_dist=dist, scale_range=scale_range, seed_a=sa, seed_b=sb, seed_s=ss)
    got = session.q4gemm_values(c.x, c.packed, c.scales, 1, n, k)
    want = oracle.q4gemm_packed(c.x, c.packed, c.scales, threads=min(16, os.cpu_count() or 1))
    assert got.shape == (1, n) and np.all(np.isfinite(got))
    rep = oracle.compare(got, want, 1e-5)
    assert rep["status"] == "pass", (case, rep["max_relative_error"])
