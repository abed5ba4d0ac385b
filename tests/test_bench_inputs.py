"""bench.py's input generators for the reference's own benchmark configuration
(bench_q4gemm.cpp: M=N=K=1024, its LCG seeds and ranges) against the oracle's restatement of the
reference generators (test_q4gemm.cpp:58-99, pinned in test_oracle.py): identical bytes."""
from __future__ import annotations

import numpy as np

import bench
from cases import make_case


def test_lcg_stream_matches_the_recurrence():
    s = 0x12345678
    want = []
    for _ in range(10_000):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        want.append(s)
    assert np.array_equal(bench.lcg_stream(10_000, 0x12345678), np.array(want, dtype=np.uint64))


def test_reference_bench_inputs_match_the_oracle_generators():
    got = bench.reference_bench_inputs(1024)
    c = make_case(1024, 1024, 1024, x_dist="uniform", x_range=(-1.0, 1.0), scale_range=(0.5, 1.5))
    assert np.array_equal(got["x"], c.x)
    assert np.array_equal(got["packed"], c.packed)
    assert np.array_equal(got["scales"], c.scales)
