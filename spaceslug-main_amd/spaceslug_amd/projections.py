"""Device-resident int4 projections of the tiny projected-attention forward.

The reference runs every projection of its tiny forward through the fp32 GEMM
ABI and re-stages the weights on each call (python/spaceslug/backend.py:1707-1738:
Q, K, V and the output projection as 128x64x64 `spaceslug_sgemm` calls, the LM head
as 128x320x64 with the vocabulary padded to 320; sgemm_api.cpp:31-53 creates a
context and copies A, B and C every time). Its LoRA forward adds a separate
`spaceslug_lora_delta` call per projection and a host-side add
(backend.py:794-799, 812-816; B pre-scaled by alpha/rank, lora.py:21-23).

Here the five weight matrices are quantized once on the GPU
(`spaceslug_q4_quantize_device`), stay resident, and the projections run on the
int4 path:
  - Q, K and V read the same states, so their weights are stored as one [3h][h/2]
    matrix (the packed layout is indexed by output column first, so concatenating
    along n stacks rows) and computed by one launch. With LoRA, the three adapters
    become one of rank 3r: A = [A_q | A_k | A_v] and B block diagonal, whose zero
    blocks contribute exact zeros;
  - the output projection (with its adapter) and the LM head run back to back as
    one retained chain (`spaceslug_q4_chain_*`): one HIP graph launch, no host
    round trip between them.
Attention between the two halves is not part of the int4 path: `forward_logits`
takes it as a callable. Outputs are those of the int4 weights (the quantizer's
rule), not of the fp32 matrices they came from.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Mapping

import numpy as np

from .backend import BackendError, BackendSession

ROWS = 128          # the reference pads the token states to 128 rows (backend.py:1714)
VOCAB_PADDED = 320  # and the LM head to 320 columns (backend.py:1709, 1733)


@dataclass
class LoRAFactors:
    """One projection's adapter: A [h][r], B [r][h]; the delta is (alpha / r) * x A B (lora.py:21-23)."""

    a: np.ndarray
    b: np.ndarray


class TinyProjections:
    """Int4 projections of the tiny forward on device-resident weights.

    query, key, value, output: float32 [h][h] (row k, column n, as the reference's
    `mat(model.query)`); lm_head: float32 [h][vocab]. adapters: optional mapping of
    "query", "key", "value", "output" to LoRAFactors of one rank r, with `alpha`.
    """

    def __init__(self, session: BackendSession, query: Any, key: Any, value: Any, output: Any, lm_head: Any, *,
                 adapters: Mapping[str, LoRAFactors] | None = None, alpha: float = 0.0,
                 vocab_padded: int = VOCAB_PADDED, rows: int = ROWS) -> None:
        import torch

        if not torch.cuda.is_available():
            raise BackendError("TinyProjections needs a HIP device")
        self._torch = torch
        self._session = session
        mats = [np.ascontiguousarray(m, dtype=np.float32) for m in (query, key, value, output)]
        h = mats[0].shape[0]
        if any(m.shape != (h, h) for m in mats) or h % 32:
            raise BackendError("query/key/value/output must be [h][h] with h % 32 == 0")
        lm = np.ascontiguousarray(lm_head, dtype=np.float32)
        if lm.ndim != 2 or lm.shape[0] != h or lm.shape[1] > vocab_padded:
            raise BackendError(f"lm_head must be [h][vocab] with vocab <= {vocab_padded}")
        self.h, self.rows, self.vocab, self.vocab_padded = h, rows, lm.shape[1], vocab_padded
        lm_p = np.zeros((h, vocab_padded), np.float32)
        lm_p[:, :self.vocab] = lm
        dev = torch.device("cuda:0")
        self._dev = dev
        self._keep: list[Any] = []  # every device buffer a chain step points at

        self.weights = {"qkv": self._quantize(np.concatenate(mats[:3], axis=1)),
                        "output": self._quantize(mats[3]),
                        "lm_head": self._quantize(lm_p)}
        f32 = dict(dtype=torch.float32, device=dev)
        self._states = torch.zeros((rows, h), **f32)
        self._qkv = torch.empty((rows, 3 * h), **f32)
        self._context = torch.zeros((rows, h), **f32)
        self._projected = torch.empty((rows, h), **f32)
        self._logits = torch.empty((rows, vocab_padded), **f32)
        self._keep += [self._states, self._qkv, self._context, self._projected, self._logits]

        lora_qkv = lora_out = None
        if adapters:
            names = ("query", "key", "value", "output")
            if set(adapters) != set(names):
                raise BackendError(f"adapters must cover {names}")
            r = adapters["query"].a.shape[1]
            for n in names:
                if adapters[n].a.shape != (h, r) or adapters[n].b.shape != (r, h):
                    raise BackendError(f"adapter {n}: A must be [h][r] and B [r][h] with one r")
            a_cat = np.concatenate([adapters[n].a for n in names[:3]], axis=1)  # [h][3r]
            b_blk = np.zeros((3 * r, 3 * h), np.float32)                       # block diagonal
            for i, n in enumerate(names[:3]):
                b_blk[i * r:(i + 1) * r, i * h:(i + 1) * h] = adapters[n].b
            lora_qkv = (self._resident(a_cat), self._resident(b_blk), 3 * r, alpha / r)
            lora_out = (self._resident(adapters["output"].a), self._resident(adapters["output"].b), r, alpha / r)
        self.rank = lora_qkv[2] // 3 if lora_qkv else 0

        def step(x, name, y, m, n, k, lora=None) -> dict[str, Any]:
            wp, ws = self.weights[name]
            s = {"d_x": x.data_ptr(), "d_w_packed": wp.data_ptr(), "d_w_scales": ws.data_ptr(), "d_y": y.data_ptr(),
                 "m": m, "n": n, "k": k}
            if lora:
                s.update(d_lora_a=lora[0].data_ptr(), d_lora_b=lora[1].data_ptr(), rank=lora[2], lora_scale=lora[3])
            return s

        self._qkv_chain = session.create_q4_chain([step(self._states, "qkv", self._qkv, rows, 3 * h, h, lora_qkv)])
        self._head_chain = session.create_q4_chain([
            step(self._context, "output", self._projected, rows, h, h, lora_out),
            step(self._projected, "lm_head", self._logits, rows, vocab_padded, h),
        ])

    # -- set-up ------------------------------------------------------------------------------------
    def _resident(self, a: np.ndarray) -> Any:
        t = self._torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(self._dev)
        self._keep.append(t)
        return t

    def _quantize(self, w: np.ndarray) -> tuple[Any, Any]:
        torch = self._torch
        k, n = w.shape
        wd = self._resident(w)
        packed = torch.empty((n, k // 2), dtype=torch.uint8, device=self._dev)
        scales = torch.empty((n, k // 32), dtype=torch.float32, device=self._dev)
        stream = torch.cuda.current_stream()
        self._session.q4_quantize_device(wd.data_ptr(), packed.data_ptr(), scales.data_ptr(), n, k, stream.cuda_stream)
        stream.synchronize()
        self._keep += [packed, scales]
        return packed, scales

    def packed(self, name: str) -> tuple[np.ndarray, np.ndarray]:
        """The int4 weights ("qkv", "output" or "lm_head") as host copies: packed [n][k/2], scales [n][k/32]."""
        wp, ws = self.weights[name]
        return wp.cpu().numpy(), ws.cpu().numpy()

    # -- the projections ----------------------------------------------------------------------------
    def _load(self, buf: Any, values: Any) -> None:
        v = np.ascontiguousarray(values, dtype=np.float32)
        if v.ndim != 2 or v.shape[1] != self.h or v.shape[0] > self.rows:
            raise BackendError(f"expected [t][{self.h}] with t <= {self.rows}")
        pad = np.zeros((self.rows, self.h), np.float32)
        pad[:v.shape[0]] = v
        buf.copy_(self._torch.from_numpy(pad))

    def qkv(self, states: Any) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """Q, K, V [rows][h] of the (zero-padded) states, one launch."""
        self._load(self._states, states)
        stream = self._torch.cuda.current_stream()
        self._qkv_chain.run(stream.cuda_stream)
        stream.synchronize()
        out = self._qkv.cpu().numpy()
        h = self.h
        return out[:, :h].copy(), out[:, h:2 * h].copy(), out[:, 2 * h:].copy()

    def head(self, context: Any) -> np.ndarray:
        """Logits [rows][vocab_padded] = LM head of the output projection of `context`, one graph launch."""
        self._load(self._context, context)
        stream = self._torch.cuda.current_stream()
        self._head_chain.run(stream.cuda_stream)
        stream.synchronize()
        return self._logits.cpu().numpy()

    def projected(self) -> np.ndarray:
        """The output projection [rows][h] the last head() call fed to the LM head."""
        return self._projected.cpu().numpy()

    def forward_logits(self, states: Any, attention: Callable[[np.ndarray, np.ndarray, np.ndarray, int], Any]
                       ) -> np.ndarray:
        """The tiny forward's last-token logits (backend.py:1734): projections here, `attention(q, k, v, t)`
        -> context [>= t][h] supplied by the caller."""
        t = np.asarray(states).shape[0]
        q, k, v = self.qkv(states)
        context = np.asarray(attention(q, k, v, t), dtype=np.float32)
        logits = self.head(context[:self.rows])
        return logits[t - 1, :self.vocab].copy()

    def close(self) -> None:
        for c in (getattr(self, "_qkv_chain", None), getattr(self, "_head_chain", None)):
            if c is not None:
                c.close()
        self._keep = []
