"""Retained projection chains (spaceslug_q4_chain_*) and the tiny forward's int4 projections.

Chains: replays of one recorded graph must equal the same calls made eagerly, bit for
bit, on every replay, with the inputs refilled and other GPU work done between
replays (a graph that only works on its first replay would pass a single check).
The steps cover a fused Q/K/V shape, a step reading what the previous one wrote, a
LoRA step and a K-split step that needs the chain's own workspace.

Tiny projections (backend.py:1707-1738, 776-816): every projection against the
oracle at the 1e-5 bar on the int4 weights the GPU quantizer produced (which are
themselves bit-identical to the oracle's quantizer), and the whole forward's
last-token logits against a double-precision pipeline with the same attention.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-5


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def rand(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def test_chain_replays_equal_eager_calls(session, oracle, gpu):
    import torch

    note("chain replays vs eager")
    rng = np.random.default_rng(5)
    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731

    def weights(n, k, seed):
        p, s = oracle.q4_quantize(rand(np.random.default_rng(seed), k, n, scale=0.05))
        return t(p), t(s)

    shapes = {"qkv": (128, 192, 64), "out": (128, 64, 64), "lm": (128, 320, 64), "lora": (40, 256, 512),
              "split": (64, 2048, 4096)}
    w = {name: weights(n, k, i) for i, (name, (m, n, k)) in enumerate(shapes.items())}
    x_qkv = t(rand(rng, 128, 64))
    ctx = t(rand(rng, 128, 64))
    x_lora = t(rand(rng, 40, 512))
    x_split = t(rand(rng, 64, 4096))
    la, lb = t(rand(rng, 512, 8, scale=0.02)), t(rand(rng, 8, 256, scale=0.02))
    ys = {name: torch.empty((m, n), dtype=torch.float32, device=dev) for name, (m, n, k) in shapes.items()}
    inputs = {"qkv": x_qkv, "out": ctx, "lm": ys["out"], "lora": x_lora, "split": x_split}

    def step(name):
        m, n, k = shapes[name]
        s = {"d_x": inputs[name].data_ptr(), "d_w_packed": w[name][0].data_ptr(), "d_w_scales": w[name][1].data_ptr(),
             "d_y": ys[name].data_ptr(), "m": m, "n": n, "k": k}
        if name == "lora":
            s.update(d_lora_a=la.data_ptr(), d_lora_b=lb.data_ptr(), rank=8, lora_scale=4.0)
        return s

    order = ["qkv", "out", "lm", "lora", "split"]
    chain = session.create_q4_chain([step(n) for n in order])
    st = torch.cuda.current_stream()

    def eager():
        out = {}
        for name in order:
            m, n, k = shapes[name]
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            x = out["out"] if name == "lm" else inputs[name]
            if name == "lora":
                session.q4gemm_lora_device(x.data_ptr(), w[name][0].data_ptr(), w[name][1].data_ptr(), la.data_ptr(),
                                           lb.data_ptr(), y.data_ptr(), m, n, k, 8, 4.0, st.cuda_stream)
            else:
                session.q4gemm_device(x.data_ptr(), w[name][0].data_ptr(), w[name][1].data_ptr(), y.data_ptr(), m, n, k,
                                      st.cuda_stream)
            out[name] = y
        st.synchronize()
        return {k: v.cpu().numpy() for k, v in out.items()}

    try:
        for replay in range(3):
            for buf in (x_qkv, ctx, x_lora, x_split):
                buf.copy_(torch.from_numpy(rand(rng, *buf.shape)))
            for y in ys.values():
                y.fill_(float("nan"))
            want = eager()                       # eager GPU work between replays
            chain.run(st.cuda_stream)
            st.synchronize()
            for name in order:
                got = ys[name].cpu().numpy()
                assert np.array_equal(got, want[name]), (replay, name)
        # and against the oracle once, for the step that reads the previous step's output
        ref = oracle.q4gemm_packed(ys["out"].cpu().numpy(), w["lm"][0].cpu().numpy(), w["lm"][1].cpu().numpy())
        rep = oracle.compare(ys["lm"].cpu().numpy(), ref, TOL)
        assert rep["status"] == "pass", rep
    finally:
        chain.close()


def test_chain_rejects_run_on_closed_handle(session, gpu):
    import torch

    from spaceslug_amd import BackendError

    dev = torch.device("cuda:0")
    x = torch.zeros((1, 64), device=dev)
    wp = torch.zeros((8, 32), dtype=torch.uint8, device=dev)
    ws = torch.zeros((8, 2), device=dev)
    y = torch.zeros((1, 8), device=dev)
    chain = session.create_q4_chain([{"d_x": x.data_ptr(), "d_w_packed": wp.data_ptr(), "d_w_scales": ws.data_ptr(),
                                      "d_y": y.data_ptr(), "m": 1, "n": 8, "k": 64}])
    chain.run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    chain.close()
    chain.close()  # idempotent
    with pytest.raises(BackendError, match="closed"):
        chain.run()


def tiny_model(rng, h=64, vocab=259, rank=4):
    from spaceslug_amd.projections import LoRAFactors

    mats = {n: rand(rng, h, h, scale=0.125) for n in ("query", "key", "value", "output")}
    lm = rand(rng, h, vocab, scale=0.125)
    adapters = {n: LoRAFactors(rand(rng, h, rank, scale=0.05), rand(rng, rank, h, scale=0.05))
                for n in ("query", "key", "value", "output")}
    return mats, lm, adapters


def causal_attention(q, k, v, t):
    """Single-head causal softmax attention in double over the first t rows (scale 1/sqrt(h))."""
    q, k, v = (np.asarray(a, np.float64)[:t] for a in (q, k, v))
    s = q @ k.T / np.sqrt(q.shape[1])
    s = np.where(np.tril(np.ones((t, t), bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    out = np.zeros((128, q.shape[1]))
    out[:t] = p @ v
    return out


@pytest.mark.parametrize("with_lora", [False, True])
def test_tiny_projections_match_oracle(session, oracle, gpu, with_lora):
    from spaceslug_amd.projections import TinyProjections

    note(f"tiny projections lora={with_lora}")
    rng = np.random.default_rng(11)
    mats, lm, adapters = tiny_model(rng)
    alpha = 8.0
    tp = TinyProjections(session, mats["query"], mats["key"], mats["value"], mats["output"], lm,
                         adapters=adapters if with_lora else None, alpha=alpha)
    try:
        h, t = 64, 37
        # the GPU quantizer's weights are the oracle quantizer's, bit for bit
        p_qkv, s_qkv = tp.packed("qkv")
        po, so = oracle.q4_quantize(np.concatenate([mats["query"], mats["key"], mats["value"]], axis=1))
        assert np.array_equal(p_qkv, po) and np.array_equal(s_qkv.view(np.uint32), so.view(np.uint32))
        states = np.zeros((128, h), np.float32)
        states[:t] = rand(rng, t, h)
        q, k, v = tp.qkv(states[:t])
        if with_lora:
            names = ("query", "key", "value")
            a_cat = np.concatenate([adapters[n].a for n in names], axis=1)
            b_blk = np.zeros((12, 3 * h), np.float32)
            for i, n in enumerate(names):
                b_blk[4 * i:4 * i + 4, h * i:h * i + h] = adapters[n].b
            ref = oracle.q4gemm_lora(states, p_qkv, s_qkv, a_cat, b_blk, alpha / 4)
        else:
            ref = oracle.q4gemm_packed(states, p_qkv, s_qkv)
        rep = oracle.compare(np.concatenate([q, k, v], axis=1), ref, TOL)
        note(f"qkv max_rel={rep['max_relative_error']:.3e}")
        assert rep["status"] == "pass", rep
        assert not np.any(q[t:]) and not np.any(v[t:])  # zero-padded rows stay exactly zero

        context = causal_attention(q, k, v, t).astype(np.float32)
        logits = tp.head(context)
        p_o, s_o = tp.packed("output")
        p_lm, s_lm = tp.packed("lm_head")
        if with_lora:
            proj = oracle.q4gemm_lora(context, p_o, s_o, adapters["output"].a, adapters["output"].b, alpha / 4)
        else:
            proj = oracle.q4gemm_packed(context, p_o, s_o)
        # the LM head's input is the GPU's own projection output (what the chain feeds it)
        proj_gpu = tp.projected()
        rep = oracle.compare(proj_gpu, proj, TOL)
        assert rep["status"] == "pass", rep
        rep = oracle.compare(logits, oracle.q4gemm_packed(proj_gpu, p_lm, s_lm), TOL)
        note(f"head max_rel={rep['max_relative_error']:.3e}")
        assert rep["status"] == "pass", rep
        assert not np.any(logits[:, 259:])  # padded vocabulary columns are zero weights

        # whole forward vs a double pipeline on the same int4 weights and the same attention
        last = tp.forward_logits(states[:t], causal_attention)
        qkv_d = ref
        ctx_d = causal_attention(qkv_d[:, :h], qkv_d[:, h:2 * h], qkv_d[:, 2 * h:], t)
        if with_lora:
            proj_d = oracle.q4gemm_lora(ctx_d.astype(np.float32), p_o, s_o, adapters["output"].a,
                                        adapters["output"].b, alpha / 4)
        else:
            proj_d = oracle.q4gemm_packed(ctx_d.astype(np.float32), p_o, s_o)
        logits_d = oracle.q4gemm_packed(proj_d.astype(np.float32), p_lm, s_lm)[t - 1, :259]
        rep = oracle.compare(last, logits_d, TOL)
        note(f"forward max_rel={rep['max_relative_error']:.3e}")
        assert rep["status"] == "pass", rep
    finally:
        tp.close()
