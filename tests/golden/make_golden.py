"""Writes the int4 GEMM golden fixtures of this directory from the C oracle.

The reference holds no stored vectors for this path (its only check is the
procedural 256^3 KAT of vulkan-runtime/tests/test_q4gemm.cpp:160-176, tolerance
1e-3), so these fixtures freeze the oracle's double-precision results on seeded
inputs. Each file holds the inputs it needs (except the 256^3 KAT, whose inputs
are regenerated from the reference's seeds by the NR LCG, test_q4gemm.cpp:58-80)
and the expected output in float64.

Run from the repository root after building the oracle:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

from oracle import oracle as o  # noqa: E402
import cases  # noqa: E402


def _save(name: str, **arrays) -> None:
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, **arrays)
    print(f"{path.name}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def tiny() -> None:
    """The Tiny projection shape (M=128, K=64, N=64), N(0,1) x, scales U[0.01, 0.05]."""
    c = cases.make_case(128, 64, 64)
    _save("tiny_m128_k64_n64", x=c.x, packed=c.packed, scales=c.scales, y=o.q4gemm_ref(c.x, c.b, c.scales))


def kat256() -> None:
    """Reference KAT, test_q4gemm.cpp:168-176: inputs regenerate from the seeds; y only."""
    c = cases.reference_kat_case()
    y = o.q4gemm_ref(c.x, c.b, c.scales)
    _save("kat_m256_k256_n256", y=y.astype(np.float32), y_row_sums=y.sum(axis=1),
          packed_checksum=np.array([int(c.packed.astype(np.uint64).sum())], dtype=np.uint64))


def ragged() -> None:
    """Shapes no 16/64 tiling divides: exercises every bounds clamp of the kernels."""
    for (m, n, k) in [(1, 37, 96), (3, 50, 160), (5, 33, 32), (17, 70, 224), (33, 129, 128)]:
        c = cases.make_case(m, n, k, x_dist="uniform", scale_range=(0.01, 0.05), seed_a=0x1000 + m,
                            seed_b=0x2000 + n, seed_s=0x3000 + k)
        _save(f"ragged_m{m}_k{k}_n{n}", x=c.x, packed=c.packed, scales=c.scales,
              y=o.q4gemm_ref(c.x, c.b, c.scales))


def extremes() -> None:
    """All nibbles -8 (sign extension) or 7 with the largest scale, and a lone nonzero nibble per column."""
    m, n, k = 4, 48, 256
    x = o.generate_floats(m * k, 0x5151, -1.0, 1.0).reshape(m, k)
    scales = np.full((n, k // 32), 0.05, dtype=np.float32)
    b = np.full((k, n), -8, dtype=np.int8)
    b[:, n // 2:] = 7
    _save("extreme_m4_k256_n48", x=x, packed=o.pack_q4(b), scales=scales, y=o.q4gemm_ref(x, b, scales))
    b = np.zeros((k, n), dtype=np.int8)
    for col in range(n):
        b[(col * 37) % k, col] = (-8, 7, -1, 3)[col % 4]
    scales = o.generate_floats(n * (k // 32), 0x5252, 0.5, 1.5).reshape(n, k // 32)
    _save("lone_nibble_m4_k256_n48", x=x, packed=o.pack_q4(b), scales=scales, y=o.q4gemm_ref(x, b, scales))


def lora() -> None:
    """Fused LoRA epilogue: y = x * dequant(W) + (alpha / r) * (x * A) * B, alpha = 32, r = 8."""
    m, n, k, r = 24, 80, 128, 8
    c = cases.make_case(m, n, k)
    la, lb = cases.lora_factors(k, n, r)
    scale = 32.0 / r
    _save("lora_m24_k128_n80_r8", x=c.x, packed=c.packed, scales=c.scales, la=la, lb=lb,
          lora_scale=np.array([scale], dtype=np.float32),
          y=o.q4gemm_lora(c.x, c.packed, c.scales, la, lb, scale))


def main() -> None:
    tiny()
    kat256()
    ragged()
    extremes()
    lora()


if __name__ == "__main__":
    main()
