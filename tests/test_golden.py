"""The committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle still reproduces every fixture bit for bit (a regression guard on
the oracle), the fixture inputs regenerate from their seeds, and an independent
float64 numpy computation (dequantise with numpy's own nibble arithmetic, then a
BLAS matrix product) agrees with every expected output to 1e-12 relative.
GPU: the HIP path through the C-ABI matches each fixture at the 1e-5 bar
(the reference's own 256^3 KAT at its 1e-3 bar plus a 3e-5 bound).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import cases

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = sorted(p.stem for p in GOLDEN.glob("*.npz") if not p.stem.startswith("kat_"))
TOL = 1e-5


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz") as z:  # allow_pickle stays False
        return {k: z[k] for k in z.files}


def numpy_dequant(packed: np.ndarray, scales: np.ndarray, k: int) -> np.ndarray:
    """W [k, n] in float64 from the packed bytes, with numpy only: low nibble = even k, two's complement."""
    lo = (packed & 0x0F).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    nib = np.empty((packed.shape[0], k), dtype=np.int16)
    nib[:, 0::2] = lo
    nib[:, 1::2] = hi
    nib = np.where(nib >= 8, nib - 16, nib)
    return (nib.astype(np.float64) * np.repeat(scales.astype(np.float64), 32, axis=1)).T


def numpy_expected(f: dict) -> np.ndarray:
    k = f["x"].shape[1]
    y = f["x"].astype(np.float64) @ numpy_dequant(f["packed"], f["scales"], k)
    if "la" in f:
        y += float(f["lora_scale"][0]) * ((f["x"].astype(np.float64) @ f["la"].astype(np.float64))
                                          @ f["lb"].astype(np.float64))
    return y


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(1.0, np.abs(want))))


def test_fixture_set_is_complete():
    assert "tiny_m128_k64_n64" in FIXTURES
    assert any(n.startswith("lora_") for n in FIXTURES)
    assert len([n for n in FIXTURES if n.startswith("ragged_")]) >= 5
    assert (GOLDEN / "kat_m256_k256_n256.npz").is_file()


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_fixture(oracle, name):
    f = load(name)
    if "la" in f:
        y = oracle.q4gemm_lora(f["x"], f["packed"], f["scales"], f["la"], f["lb"], float(f["lora_scale"][0]))
    else:
        y = oracle.q4gemm_packed(f["x"], f["packed"], f["scales"])
    assert y.dtype == np.float64 and y.shape == f["y"].shape
    assert np.array_equal(y, f["y"]), name


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_matches_independent_numpy(name):
    f = load(name)
    assert rel_err(numpy_expected(f), f["y"]) <= 1e-12, name


def test_seeded_fixtures_regenerate_from_seeds(oracle):
    f = load("tiny_m128_k64_n64")
    c = cases.make_case(128, 64, 64)
    assert np.array_equal(c.x, f["x"]) and np.array_equal(c.packed, f["packed"])
    assert np.array_equal(c.scales, f["scales"])


def test_reference_kat_fixture(oracle):
    f = load("kat_m256_k256_n256")
    c = cases.reference_kat_case()
    assert int(c.packed.astype(np.uint64).sum()) == int(f["packed_checksum"][0])
    y = oracle.q4gemm_ref(c.x, c.b, c.scales)
    assert np.array_equal(y.astype(np.float32), f["y"])
    assert np.array_equal(y.sum(axis=1), f["y_row_sums"])
    f_np = {"x": c.x, "packed": c.packed, "scales": c.scales}
    assert rel_err(numpy_expected(f_np), y) <= 1e-12


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_gpu_matches_fixture(session, gpu, name):
    f = load(name)
    m, k = f["x"].shape
    n = f["packed"].shape[0]
    print(f"[gpu-case] golden {name}", flush=True)
    if "la" in f:
        r = f["la"].shape[1]
        got = session.q4gemm_lora_values(f["x"], f["packed"], f["scales"], f["la"], f["lb"], m, n, k, r,
                                         float(f["lora_scale"][0]))
    else:
        got = session.q4gemm_values(f["x"], f["packed"], f["scales"], m, n, k)
    err = rel_err(np.asarray(got).reshape(m, n), f["y"])
    print(f"[gpu-case] golden {name} max_rel={err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.gpu
def test_gpu_matches_reference_kat_fixture(session, gpu):
    f = load("kat_m256_k256_n256")
    c = cases.reference_kat_case()
    print("[gpu-case] golden kat 256^3", flush=True)
    got = np.asarray(session.q4gemm_values(c.x, c.packed, c.scales, 256, 256, 256)).reshape(256, 256)
    # stored in float32: their rounding (<= 2^-24 relative) is far below both bars
    err = rel_err(got, f["y"].astype(np.float64))
    print(f"[gpu-case] golden kat max_rel={err:.3e}", flush=True)
    assert err <= 1e-3
    assert err <= TOL
