"""Versioned on-disk format for int4 group-32 weights in the kernels' packed layout (".ssq4").

The reference keeps its int4 weights only in memory (its tests generate them,
vulkan-runtime/tests/test_q4gemm.cpp:71-99) and asks that quantization metadata
be explicit and that unknown schema versions fail closed
(docs/ARTIFACT_FORMAT.md:35-38,50-55). This file format carries exactly the bytes
spaceslug_q4gemm reads, with that metadata:

    offset 0   4 bytes  magic b"SSQ4"
    offset 4   u32 LE   format version (1)
    offset 8   u32 LE   byte length L of the JSON header
    offset 12  L bytes  JSON header, UTF-8 (fields below)
    ...        zero padding to a multiple of 256
    packed     uint8[n][k/2]   (header "packed_offset", "packed_bytes")
    ...        zero padding to a multiple of 256
    scales     float32 LE [n][k/32] (header "scales_offset", "scales_bytes")

JSON fields: format ("spaceslug-int4-g32"), version, n, k, group (32), layout,
nibble, scale_dtype, quantizer (the rule that produced the values, or
"external"), packed_offset/packed_bytes, scales_offset/scales_bytes, and sha256
of the packed and scale bytes. Reading checks every one of them; a mismatch,
an unknown version or a different format name raises Q4FormatError.

Command line:
    python -m spaceslug_amd.q4file quantize --input w.npy --output w.ssq4   (w: float32 [k, n])
    python -m spaceslug_amd.q4file info w.ssq4
"""
from __future__ import annotations

import argparse
import hashlib
import json
import struct
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

MAGIC = b"SSQ4"
VERSION = 1
FORMAT = "spaceslug-int4-g32"
GROUP = 32
ALIGN = 256
LAYOUT = "packed uint8[n][k/2]: byte n*(k/2) + k/2, even k in bits 0-3, odd k in bits 4-7; scales float32[n][k/32]"
NIBBLE = "two's complement, value in [-8, 7]"
QUANTIZER = ("per column and 32-value group: m = largest-magnitude value (first in k order), scale = -m/8, "
             "nibble = clamp(rint(w/scale), -8, 7); all-zero group: scale 0")


class Q4FormatError(ValueError):
    pass


@dataclass
class Q4Tensor:
    n: int
    k: int
    packed: np.ndarray   # uint8 [n, k/2]
    scales: np.ndarray   # float32 [n, k/32]
    quantizer: str = QUANTIZER

    def __post_init__(self) -> None:
        if self.k <= 0 or self.n <= 0 or self.k % GROUP:
            raise Q4FormatError(f"n={self.n}, k={self.k}: need n >= 1 and k % {GROUP} == 0")
        self.packed = np.ascontiguousarray(self.packed, dtype=np.uint8).reshape(self.n, self.k // 2)
        self.scales = np.ascontiguousarray(self.scales, dtype="<f4").reshape(self.n, self.k // GROUP)


def _align(v: int) -> int:
    return (v + ALIGN - 1) // ALIGN * ALIGN


def _sha(b: bytes | memoryview) -> str:
    return hashlib.sha256(b).hexdigest()


def save(path: str | Path, t: Q4Tensor) -> None:
    packed = t.packed.tobytes()
    scales = t.scales.astype("<f4").tobytes()
    header: dict[str, Any] = {"format": FORMAT, "version": VERSION, "n": t.n, "k": t.k, "group": GROUP,
                              "layout": LAYOUT, "nibble": NIBBLE, "scale_dtype": "float32-le",
                              "quantizer": t.quantizer, "packed_bytes": len(packed), "scales_bytes": len(scales),
                              "sha256": {"packed": _sha(packed), "scales": _sha(scales)}}
    # offsets depend on the header length, which depends on the offsets' digits: iterate to a fixed point
    header["packed_offset"] = header["scales_offset"] = 0
    for _ in range(4):
        blob = json.dumps(header, sort_keys=True).encode("utf-8")
        packed_offset = _align(12 + len(blob))
        scales_offset = _align(packed_offset + len(packed))
        if header["packed_offset"] == packed_offset and header["scales_offset"] == scales_offset:
            break
        header["packed_offset"], header["scales_offset"] = packed_offset, scales_offset
    blob = json.dumps(header, sort_keys=True).encode("utf-8")
    if _align(12 + len(blob)) != header["packed_offset"]:
        raise Q4FormatError("internal: header layout did not converge")
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<II", VERSION, len(blob)) + blob)
        f.write(b"\0" * (header["packed_offset"] - 12 - len(blob)))
        f.write(packed)
        f.write(b"\0" * (header["scales_offset"] - header["packed_offset"] - len(packed)))
        f.write(scales)


def read_header(path: str | Path) -> dict[str, Any]:
    with open(path, "rb") as f:
        head = f.read(12)
        if len(head) < 12 or head[:4] != MAGIC:
            raise Q4FormatError(f"{path}: not an SSQ4 file")
        version, hlen = struct.unpack("<II", head[4:12])
        if version != VERSION:
            raise Q4FormatError(f"{path}: unknown SSQ4 version {version} (this reader knows {VERSION})")
        try:
            header = json.loads(f.read(hlen).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise Q4FormatError(f"{path}: unreadable header: {e}") from None
    if not isinstance(header, dict):
        raise Q4FormatError(f"{path}: header is not an object")
    expect = {"format": FORMAT, "version": VERSION, "group": GROUP, "scale_dtype": "float32-le", "layout": LAYOUT,
              "nibble": NIBBLE}
    for key, value in expect.items():
        if header.get(key) != value:
            raise Q4FormatError(f"{path}: header field {key!r} is {header.get(key)!r}, expected {value!r}")
    n, k = header.get("n"), header.get("k")
    if not (isinstance(n, int) and isinstance(k, int) and n >= 1 and k >= GROUP and k % GROUP == 0):
        raise Q4FormatError(f"{path}: bad shape n={n!r} k={k!r}")
    if header.get("packed_bytes") != n * (k // 2) or header.get("scales_bytes") != 4 * n * (k // GROUP):
        raise Q4FormatError(f"{path}: section sizes do not match n={n}, k={k}")
    return header


def load(path: str | Path, verify: bool = True) -> Q4Tensor:
    header = read_header(path)
    n, k = header["n"], header["k"]
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    po, pb, so, sb = (header["packed_offset"], header["packed_bytes"], header["scales_offset"],
                      header["scales_bytes"])
    if po % ALIGN or so % ALIGN or so < po + pb or raw.size < so + sb:
        raise Q4FormatError(f"{path}: truncated or misplaced sections")
    packed = np.array(raw[po:po + pb])
    scales = np.array(raw[so:so + sb]).view("<f4")
    if verify:
        if _sha(packed.tobytes()) != header["sha256"]["packed"] or _sha(scales.tobytes()) != header["sha256"]["scales"]:
            raise Q4FormatError(f"{path}: checksum mismatch")
    return Q4Tensor(n, k, packed, scales.astype(np.float32), header.get("quantizer", "external"))


def quantize(session: Any, w: np.ndarray) -> Q4Tensor:
    """fp32 w [k, n] -> Q4Tensor through the GPU quantizer (spaceslug_q4_quantize)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise Q4FormatError("w must be a [k, n] matrix")
    k, n = w.shape
    packed, scales = session.q4_quantize_values(w, n, k)
    return Q4Tensor(n, k, packed, scales)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m spaceslug_amd.q4file", description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    q = sub.add_parser("quantize", help="quantize a float32 [k, n] .npy matrix on the GPU and write .ssq4")
    q.add_argument("--input", required=True)
    q.add_argument("--output", required=True)
    i = sub.add_parser("info", help="print and verify an .ssq4 header")
    i.add_argument("path")
    args = ap.parse_args(argv)
    if args.cmd == "info":
        header = read_header(args.path)
        load(args.path)  # verifies sizes and checksums
        print(json.dumps(header, indent=2, sort_keys=True))
        return 0
    from .backend import BackendSession

    w = np.load(args.input, allow_pickle=False)
    t = quantize(BackendSession(), w)
    save(args.output, t)
    print(f"{args.output}: n={t.n} k={t.k} ({t.packed.nbytes + t.scales.nbytes} bytes of weights)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
