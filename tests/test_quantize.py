"""fp32 -> int4 group-32 quantizer and the .ssq4 weight file.

CPU: the oracle's quantizer agrees bit for bit with an independent numpy
restatement of the rule; exactly representable groups (v * 2^e with the -8 end
present) come back exactly; the rounding error bound holds; zero and
non-finite groups; the file format round trip, its fail-closed checks and the
C-ABI argument validation. GPU: spaceslug_q4_quantize is bit-identical to the
oracle, and quantize -> q4gemm matches the oracle's GEMM at the 1e-5 bar.
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest

import cases
from spaceslug_amd import q4file

f32p = ctypes.POINTER(ctypes.c_float)
u8p = ctypes.POINTER(ctypes.c_uint8)


def numpy_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The rule restated with numpy only (argmax keeps the first maximum; IEEE float32 division; rint)."""
    w = np.asarray(w, dtype=np.float32)
    K, N = w.shape
    G = K // 32
    blocks = w.reshape(G, 32, N)                                   # [g, t, n]
    idx = np.argmax(np.abs(blocks), axis=1)                        # first largest magnitude
    m = np.take_along_axis(blocks, idx[:, None, :], axis=1)[:, 0, :]
    scale = (-m * np.float32(0.125)).astype(np.float32)            # [g, n]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(blocks / scale[:, None, :]).astype(np.float32)
    q = np.clip(np.nan_to_num(q, nan=0.0), -8, 7).astype(np.int64)
    finite = np.all(np.isfinite(blocks), axis=1)                  # [g, n]
    bad = ~finite | (scale == 0)
    q[np.broadcast_to(bad[:, None, :], q.shape)] = 0
    scale = np.where(finite, np.where(scale == 0, np.float32(0), scale), np.float32(np.nan))
    nib = (q.reshape(K, N) & 0xF).astype(np.uint8)                 # [k, n]
    packed = (nib[0::2, :] | (nib[1::2, :] << 4)).T.copy()         # [n, k/2]
    return packed, scale.T.astype(np.float32).copy()


def weights(k: int, n: int, seed: int = 11) -> np.ndarray:
    from oracle import oracle as o

    return o.generate_normal(k * n, seed, 0.0, 0.02).reshape(k, n)


def same(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


@pytest.mark.parametrize("k,n", [(32, 1), (64, 7), (256, 33), (4096, 40)])
def test_oracle_matches_numpy_restatement(oracle, k, n):
    w = weights(k, n)
    p_o, s_o = oracle.q4_quantize(w)
    p_n, s_n = numpy_quantize(w)
    assert np.array_equal(p_o, p_n)
    assert same(s_o, s_n)


def test_exactly_representable_groups_round_trip(oracle):
    rng = np.random.default_rng(3)
    k, n = 128, 24
    v = rng.integers(-8, 8, size=(k, n))
    v[0::32, :] = -8                                   # each group's extreme value is -8 and comes first
    e = rng.integers(-20, 5, size=(k // 32, n)).astype(np.float64)
    w = (v * np.repeat(2.0 ** e, 32, axis=0)).astype(np.float32)
    packed, scales = oracle.q4_quantize(w)
    assert np.array_equal(scales, (2.0 ** e).T.astype(np.float32))
    assert np.array_equal(oracle.unpack_q4(packed, k, n), v.astype(np.int8))


def test_rounding_error_bound(oracle):
    w = weights(512, 64, seed=5)
    packed, scales = oracle.q4_quantize(w)
    v = oracle.unpack_q4(packed, 512, 64).astype(np.float64)
    s = np.repeat(scales.T.astype(np.float64), 32, axis=0)
    err = np.abs(w - v * s)
    clamped = (w / s) > 7.5                           # the opposite-sign extreme (+8 -> 7)
    assert np.all(err[~clamped] <= np.abs(s[~clamped]) * 0.5 * (1 + 1e-6))
    assert np.all(err[clamped] <= np.abs(s[clamped]) * (1 + 1e-6))
    # the group extreme is represented exactly as -8 * scale
    assert np.all(np.min(v.reshape(16, 32, 64) * np.sign(-scales.T[:, None, :]), axis=1) >= -8)


def test_ties_zero_and_nonfinite_groups(oracle):
    w = np.zeros((64, 3), np.float32)
    w[3, 0], w[9, 0] = 0.5, -0.5                       # tie: the first (0.5) sets the sign -> scale -1/16
    w[40, 1] = np.nan                                  # non-finite groups: a NaN anywhere, an infinity
    w[70 % 64, 2] = np.inf
    packed, scales = oracle.q4_quantize(w)
    assert scales[0, 0] == np.float32(-0.0625)
    v = oracle.unpack_q4(packed, 64, 3)
    assert v[3, 0] == -8 and v[9, 0] == 7              # +8 clamps to 7
    assert scales[1, 0] == 0.0 and np.signbit(scales[1, 0]) == 0 and not np.any(v[:32, 1])
    assert np.isnan(scales[1, 1]) and not np.any(v[32:, 1])
    assert np.isnan(scales[2, 0]) and scales[2, 1] == 0.0 and not np.any(v[:32, 2])
    p_n, s_n = numpy_quantize(w)
    assert np.array_equal(packed, p_n) and same(scales, s_n)


# -- the .ssq4 file ----------------------------------------------------------------------------------------

def test_file_round_trip(oracle, tmp_path):
    w = weights(256, 40)
    packed, scales = oracle.q4_quantize(w)
    t = q4file.Q4Tensor(40, 256, packed, scales)
    path = tmp_path / "w.ssq4"
    q4file.save(path, t)
    header = q4file.read_header(path)
    assert header["n"] == 40 and header["k"] == 256 and header["group"] == 32
    assert header["packed_offset"] % 256 == 0 and header["scales_offset"] % 256 == 0
    back = q4file.load(path)
    assert np.array_equal(back.packed, packed) and same(back.scales, scales)
    assert back.quantizer == q4file.QUANTIZER


def test_file_fails_closed(oracle, tmp_path):
    packed, scales = oracle.q4_quantize(weights(64, 8))
    path = tmp_path / "w.ssq4"
    q4file.save(path, q4file.Q4Tensor(8, 64, packed, scales))
    raw = bytearray(path.read_bytes())

    def write(b: bytes) -> None:
        path.write_bytes(b)

    bad = bytearray(raw); bad[0:4] = b"XXXX"; write(bytes(bad))
    with pytest.raises(q4file.Q4FormatError, match="not an SSQ4"):
        q4file.load(path)
    bad = bytearray(raw); bad[4:8] = struct.pack("<I", 2); write(bytes(bad))
    with pytest.raises(q4file.Q4FormatError, match="unknown SSQ4 version"):
        q4file.load(path)
    bad = bytearray(raw); bad[-1] ^= 0xFF; write(bytes(bad))
    with pytest.raises(q4file.Q4FormatError, match="checksum"):
        q4file.load(path)
    write(bytes(raw[:-100]))
    with pytest.raises(q4file.Q4FormatError, match="truncated"):
        q4file.load(path)
    hlen = struct.unpack("<I", raw[8:12])[0]
    header = raw[12:12 + hlen].decode().replace('"group": 32', '"group": 64')
    bad = bytearray(raw); bad[12:12 + hlen] = header.encode(); write(bytes(bad))
    with pytest.raises(q4file.Q4FormatError, match="group"):
        q4file.load(path)


def test_abi_quantize_validates_before_device(runtime_lib_path):
    L = ctypes.CDLL(str(runtime_lib_path))
    L.spaceslug_last_error.restype = ctypes.c_char_p
    w = np.zeros(64 * 4, np.float32)
    p = np.zeros(4 * 32, np.uint8)
    s = np.zeros(4 * 2, np.float32)
    wp, pp, sp = w.ctypes.data_as(f32p), p.ctypes.data_as(u8p), s.ctypes.data_as(f32p)
    assert L.spaceslug_q4_quantize(None, pp, sp, 4, 64) == 1
    assert L.spaceslug_q4_quantize(wp, pp, sp, 4, 48) == 1
    assert L.spaceslug_q4_quantize(wp, pp, sp, 0, 64) == 1
    w[5] = np.inf
    assert L.spaceslug_q4_quantize(wp, pp, sp, 4, 64) == 1
    assert b"non-finite" in L.spaceslug_last_error()


# -- GPU --------------------------------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("k,n", [(32, 1), (96, 300), (4096, 257), (8192, 64)])
def test_gpu_quantizer_bit_identical(session, oracle, gpu, k, n):
    print(f"[gpu-case] quantize k={k} n={n}", flush=True)
    w = weights(k, n, seed=k + n)
    w[:32, 0] = 0.0                                    # an all-zero group
    if n > 1:
        w[32 % k:32 % k + 1, 1] = -w[0, 1]             # keep a sign tie somewhere
    packed, scales = session.q4_quantize_values(w, n, k)
    p_o, s_o = oracle.q4_quantize(w)
    assert np.array_equal(packed, p_o)
    assert same(scales, s_o)


@pytest.mark.gpu
def test_gpu_quantizer_device_entry_and_gemm(session, oracle, gpu):
    import torch

    print("[gpu-case] quantize on device then q4gemm", flush=True)
    m, n, k = 16, 512, 1024
    w = weights(k, n, seed=77)
    w_t = torch.from_numpy(w).to("cuda:0")
    p_t = torch.empty((n, k // 2), dtype=torch.uint8, device="cuda:0")
    s_t = torch.empty((n, k // 32), dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream()
    session.q4_quantize_device(w_t.data_ptr(), p_t.data_ptr(), s_t.data_ptr(), n, k, st.cuda_stream)
    st.synchronize()
    p_o, s_o = oracle.q4_quantize(w)
    assert np.array_equal(p_t.cpu().numpy(), p_o) and same(s_t.cpu().numpy(), s_o)
    c = cases.make_case(m, n, k)
    y = session.q4gemm_values(c.x, p_t.cpu().numpy(), s_t.cpu().numpy(), m, n, k)
    ref = oracle.q4gemm_packed(c.x, p_o, s_o)
    rep = oracle.compare(y, ref, 1e-5)
    assert rep["status"] == "pass", rep
    # and the quantised projection tracks the fp32 one to int4 accuracy (a step of |m|/8 per group:
    # about 11% relative RMS error per weight for normal weights, and the same on the outputs)
    dense = c.x.astype(np.float64) @ w.astype(np.float64)
    assert np.linalg.norm(ref - dense) <= 0.15 * np.linalg.norm(dense)


@pytest.mark.gpu
def test_gpu_quantize_file_cli_round_trip(session, oracle, gpu, tmp_path):
    print("[gpu-case] q4file CLI", flush=True)
    w = weights(256, 96, seed=9)
    np.save(tmp_path / "w.npy", w)
    assert q4file.main(["quantize", "--input", str(tmp_path / "w.npy"), "--output", str(tmp_path / "w.ssq4")]) == 0
    t = q4file.load(tmp_path / "w.ssq4")
    p_o, s_o = oracle.q4_quantize(w)
    assert np.array_equal(t.packed, p_o) and same(t.scales, s_o)
    assert q4file.main(["info", str(tmp_path / "w.ssq4")]) == 0
