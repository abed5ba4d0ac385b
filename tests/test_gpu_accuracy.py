"""Accuracy on the reference KAT's own input ranges, at the sizes where an fp32 group sum fails.

The reference's KAT and bench draw x uniform in [-1, 1) and scales uniform in [0.5, 1.5)
(vulkan-runtime/tests/test_q4gemm.cpp:168-176, bench/bench_q4gemm.cpp:36-47). There each 32-value
group's partial sum is ~15, ~30x the workload configurations' (scales 0.01-0.05), while outputs near
zero are held to an absolute 1e-5 by the metric |gpu - ref| / max(1, |ref|) (test_q4gemm.cpp:380).

Up to 32 rows every path forms each group sum exactly in integers (the one- and two-row decode GEMV
with v_dot8 on hex digits of x, the small-batch GEMM with int8 MFMAs on byte digits of x) and sums the
groups in double. The only approximation left is x's 31-bit fixed point per group (at most 2^-30 of
the group's largest |x| per value), so these cases are held to 2e-7: a few fp32 roundings of y
itself. An fp32 group sum measured 2e-5 to 8e-5 on the same inputs, so a return of one fails here.

Above 32 rows the bf16-limb MFMA path rounds each group sum once per MFMA in fp32 (its stated
tolerance): the error grows like sqrt(K / 32) and is held to 6e-6 * sqrt(K / 32) on these ranges,
and to 1e-5 on the workload distributions at the same sizes.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

from cases import make_case

pytestmark = pytest.mark.gpu

EXACT_TOL = 2e-7
KAT_RANGES = dict(x_dist="uniform", x_range=(-1.0, 1.0), scale_range=(0.5, 1.5))


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def bf16_limb_tol(k: int) -> float:
    return 6e-6 * math.sqrt(k / 32)


def run_and_check(session, oracle, c, tol: float, label: str) -> float:
    got = session.q4gemm_values(c.x, c.packed, c.scales, c.m, c.n, c.k)
    want = oracle.q4gemm_packed(c.x, c.packed, c.scales, threads=16)
    rep = oracle.compare(got, want, tol)
    note(f"{label} max_rel={rep['max_relative_error']:.3e} (bar {tol:.1e})")
    assert rep["status"] == "pass", rep
    return rep["max_relative_error"]


@pytest.mark.parametrize("m,k", [(1, 1024), (1, 4096), (1, 8192), (2, 1024), (2, 4096), (4, 1024), (4, 4096),
                                 (3, 8192), (16, 1024), (16, 4096), (32, 1024), (32, 4096), (32, 8192),
                                 (24, 640), (7, 2080), (1, 14336), (1, 32768), (2, 8192), (2, 11008), (2, 16384)])
def test_small_batch_exact_on_kat_ranges(session, oracle, gpu, m, k):
    """Every path up to 32 rows, including the decode GEMV's K-split forms (one row up to K = 32768, two
    rows up to 16384), whose per-wavefront partials are added in double."""
    n = 2048 if k <= 4096 else 1024
    note(f"kat ranges m={m} n={n} k={k}")
    c = make_case(m, n, k, **KAT_RANGES)
    run_and_check(session, oracle, c, EXACT_TOL, f"kat-ranges {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(64, 2048, 1024), (64, 2048, 4096), (1024, 2048, 4096), (64, 1024, 8192),
                                   (1024, 1024, 1024)])
def test_bf16_limb_path_stated_tolerance(session, oracle, gpu, m, n, k):
    """Above 32 rows: the stated tolerance 6e-6 * sqrt(K/32) on the KAT's ranges (largest K tested 8192:
    9.6e-5), and the 1e-5 bar on the workload distributions at the same shapes."""
    note(f"bf16 limbs m={m} n={n} k={k}")
    c = make_case(m, n, k, **KAT_RANGES)
    run_and_check(session, oracle, c, bf16_limb_tol(k), f"bf16 kat-ranges {m}x{n}x{k}")
    w = make_case(m, n, k)
    run_and_check(session, oracle, w, 1e-5, f"bf16 workload {m}x{n}x{k}")


def test_small_batch_groups_of_very_different_magnitude(session, oracle, gpu):
    """Rows whose groups span 1e-30 .. 1e30, subnormals, exact powers of two and an outlier among small
    values: the fixed point is per (row, group), so a group's precision does not depend on another
    group's or another row's magnitude. Held to the exact bar at 5 and 32 rows."""
    rng = np.random.default_rng(7)
    for m in (5, 32):
        k, n = 512, 300
        c = make_case(m, n, k, **KAT_RANGES)
        x = c.x.copy()
        g = k // 32
        mags = np.array([1e-30, 1e-3, 1.0, 1e30, 2.0 ** -140, 1e5, 3.0, 1e-12], dtype=np.float64)
        for row in range(m):
            for gi in range(g):
                x[row, 32 * gi:32 * gi + 32] *= np.float32(mags[(row + gi) % len(mags)])
        x[:, 5] = np.float32(2.0 ** 20)           # an outlier in an otherwise small group
        x[:, 40:72] = np.float32(0.0)              # an all-zero group
        x[0, 100:132] = np.float32(2.0) ** rng.integers(-20, 20, 32).astype(np.float32)
        c.x = x.astype(np.float32)
        note(f"magnitudes m={m} n={n} k={k}")
        run_and_check(session, oracle, c, EXACT_TOL, f"magnitudes {m}x{n}x{k}")
