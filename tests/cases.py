"""Seeded input builders for the int4 GEMM parity cases (uses the oracle's generators).

Default seeds are the reference KAT's (vulkan-runtime/tests/test_q4gemm.cpp:168-176):
0x12345678 for A, 0x9abcdef0 for the int4 values (drawn k-major, b[k*N + n]),
0x13579bdf for the scales (n-major). The workload configurations use N(0, 1)
activations and scales uniform in [0.01, 0.05].
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import oracle as o

SEED_A = 0x12345678
SEED_B = 0x9ABCDEF0
SEED_S = 0x13579BDF
SEED_LA = 0x2468ACE0
SEED_LB = 0x0F1E2D3C


@dataclass
class Case:
    m: int
    n: int
    k: int
    x: np.ndarray        # float32 [m, k]
    b: np.ndarray        # int8 [k, n] (logical int4 values)
    packed: np.ndarray   # uint8 [n, k/2]
    scales: np.ndarray   # float32 [n, k/32]


def make_case(m: int, n: int, k: int, *, x_dist: str = "normal", scale_range=(0.01, 0.05), x_range=(-1.0, 1.0),
              seed_a: int = SEED_A, seed_b: int = SEED_B, seed_s: int = SEED_S) -> Case:
    if x_dist == "normal":
        x = o.generate_normal(m * k, seed_a, 0.0, 1.0)
    else:
        x = o.generate_floats(m * k, seed_a, x_range[0], x_range[1])
    b = o.generate_int4(k * n, seed_b).reshape(k, n)
    scales = o.generate_floats(n * (k // 32), seed_s, scale_range[0], scale_range[1]).reshape(n, k // 32)
    packed = o.pack_q4(b)
    return Case(m, n, k, x.reshape(m, k), b, packed, scales)


def reference_kat_case() -> Case:
    """test_q4gemm.cpp:40-42,168-176: M=N=K=256, A ~ U[-1, 1), scales ~ U[0.5, 1.5)."""
    return make_case(256, 256, 256, x_dist="uniform", x_range=(-1.0, 1.0), scale_range=(0.5, 1.5))


def lora_factors(k: int, n: int, rank: int, std: float = 0.02) -> tuple[np.ndarray, np.ndarray]:
    la = o.generate_normal(k * rank, SEED_LA, 0.0, std).reshape(k, rank)
    lb = o.generate_normal(rank * n, SEED_LB, 0.0, std).reshape(rank, n)
    return la, lb
