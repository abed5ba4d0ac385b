"""Calls from several host threads at once: the host-pointer entry points (one shared staging buffer per
device) and the device-pointer entry points on one stream per thread (one shared workspace per device,
ordered across streams by the library). ctypes releases the GIL for each call, so the threads enter the
library together. Every result is checked against the oracle, computed beforehand."""
from __future__ import annotations

import threading

import numpy as np
import pytest

from cases import lora_factors, make_case

pytestmark = pytest.mark.gpu

# (m, n, k, rank): GEMV (one row; K-split; two rows), small batch, K-split wide, mid-size tiles, LoRA on both
# sides of 32 rows
SHAPES = [(1, 3000, 4096, 0), (1, 2000, 14336, 0), (2, 900, 8192, 0), (7, 900, 1024, 0), (40, 300, 4128, 0),
          (100, 301, 512, 0), (64, 256, 1024, 8), (5, 700, 2048, 4)]
THREADS = 8
ROUNDS = 4


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def expected(oracle):
    out = []
    for i, (m, n, k, r) in enumerate(SHAPES):
        c = make_case(m, n, k, seed_a=0x1000 + i, seed_b=0x2000 + i, seed_s=0x3000 + i)
        if r:
            la, lb = lora_factors(k, n, r)
            want = oracle.q4gemm_lora(c.x, c.packed, c.scales, la, lb, 2.0)
        else:
            la = lb = None
            want = oracle.q4gemm_packed(c.x, c.packed, c.scales)
        out.append((c, la, lb, want))
    return out


def run_threads(worker):
    errors = []

    def body(t):
        try:
            worker(t)
        except Exception as e:  # reported to the main thread
            errors.append((t, repr(e)))

    threads = [threading.Thread(target=body, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors


def test_host_pointer_calls_from_threads(session, oracle, gpu):
    note(f"host-pointer calls from {THREADS} threads")
    cases = expected(oracle)

    def worker(t):
        for rnd in range(ROUNDS):
            i = (t + rnd) % len(SHAPES)
            m, n, k, r = SHAPES[i]
            c, la, lb, want = cases[i]
            if r:
                got = session.q4gemm_lora_values(c.x, c.packed, c.scales, la, lb, m, n, k, r, 2.0)
            else:
                got = session.q4gemm_values(c.x, c.packed, c.scales, m, n, k)
            rep = oracle.compare(got, want, 1e-5)
            assert rep["status"] == "pass", (t, rnd, SHAPES[i], rep["max_relative_error"])

    run_threads(worker)


def test_device_pointer_calls_from_threads_on_their_own_streams(session, oracle, gpu):
    import torch

    note(f"device-pointer calls from {THREADS} threads, one stream each")
    cases = expected(oracle)
    dev = []
    for c, la, lb, _ in cases:
        t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
        dev.append((t(c.x), t(c.packed), t(c.scales), t(la), t(lb)))
    torch.cuda.synchronize()

    def worker(t):
        stream = torch.cuda.Stream(device="cuda:0")
        for rnd in range(ROUNDS):
            i = (2 * t + rnd) % len(SHAPES)
            m, n, k, r = SHAPES[i]
            x, w, s, la, lb = dev[i]
            with torch.cuda.stream(stream):
                y = torch.empty((m, n), dtype=torch.float32, device="cuda:0")  # allocated on this stream
                if r:
                    session.q4gemm_lora_device(x.data_ptr(), w.data_ptr(), s.data_ptr(), la.data_ptr(), lb.data_ptr(),
                                               y.data_ptr(), m, n, k, r, 2.0, stream.cuda_stream)
                else:
                    session.q4gemm_device(x.data_ptr(), w.data_ptr(), s.data_ptr(), y.data_ptr(), m, n, k,
                                          stream.cuda_stream)
            stream.synchronize()
            rep = oracle.compare(y.cpu().numpy(), cases[i][3], 1e-5)
            assert rep["status"] == "pass", (t, rnd, SHAPES[i], rep["max_relative_error"])

    run_threads(worker)
