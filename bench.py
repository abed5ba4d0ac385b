#!/usr/bin/env python3
"""Benchmark of the MI355X int4-dequant GEMV/GEMM (libspaceslug_runtime.so, gfx950).

Headline (value): decode GEMV, M=1, K=4096, N=14336, int4 group-32 weights, 64
distinct weight copies (2.35 GB, far beyond the 256 MB last-level cache) resident
in HBM and swept in turn. One step = one sweep = 64 GEMV launches through the
C-ABI device entry point spaceslug_q4gemm_device on torch's current stream,
captured once into a HIP graph and replayed (the way a decode loop launches a
fixed sequence of projections); the same sweep launched call by call from the
host is timed too and reported as "gemv_other_launch".
value = algorithmic bytes of all timed launches / timed wall time on the GPU
(HIP events around the timed region, on the launch stream).

Algorithmic bytes per launch (each tensor once): packed nibbles K*N/2 + fp32
scales 4*N*K/32 + x 4*M*K + y 4*M*N. Flops per launch: 2*M*N*K.

Also reported in the same JSON line:
  - "roofline": achieved GB/s of the GEMV kernel vs MI355X's 8 TB/s HBM peak;
  - "prefill": the M=2048, K=4096, N=14336 GEMM in TFLOP/s (2*M*N*K / time, the second half of the
    headline metric). Its roofline is the matrix instruction the kernel runs: above 32 rows that is
    v_mfma_f32_16x16x32_bf16 on x split exactly into three bf16 limbs, so the matrix core executes
    3 * 2*M*N*K bf16 flops, priced against the 2.5 PFLOP/s dense bf16 peak (the fp32-equivalent rate
    and the 157.3 TFLOP/s fp32 MFMA peak are given beside it); at 32 rows or fewer the kernels run
    v_mfma_f32_16x16x4_f32, priced against 157.3 TFLOP/s;
  - "small_batch" (M=16, K=N=4096, 32 weight copies per step) and "lora"
    (M=512, K=N=4096, rank 16) throughput;
  - "cq4": the CQ4 codebook matmul on the reference's CQ4 benchmark shapes;
  - "launch_floor": the per-launch time of a near-empty kernel replayed the same way, and the
    fraction of the HBM peak that one launch of the GEMV's bytes could reach above it;
  - "cpu_baseline": the C CPU oracle (double-precision restatement of the
    reference's cpu_reference) on a bounded sample of the same GEMV workload,
    timed on this host's cores.
Inputs are synthetic (torch RNG on the GPU: N(0,1) activations, uniform
nibbles in [-8, 7], scales uniform in [0.01, 0.05]).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "spaceslug-main_amd"))
sys.path.insert(0, str(REPO))

METRIC = "int4 GEMV GB/s @M=1 & GEMM TFLOP/s @M=2048, % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
# The library runs GEMMs of more than 32 rows on the bf16 MFMA with x as three exact bf16 limbs.
WIDE_MIN_ROWS = 33
BF16_LIMBS = 3


def gemm_roofline(m: int, n: int, k: int, seconds_per_call: float) -> dict:
    """Roofline of the GEMM kernel that runs m x n x k: the matrix instruction's executed flops per second
    against that instruction's dense peak (LoRA's rank-r terms, under 1% of the work, are left out)."""
    tf = 2.0 * m * n * k / seconds_per_call / 1e12
    if m >= WIDE_MIN_ROWS:
        achieved = BF16_LIMBS * tf
        return {"bound": "mfma", "instruction": "v_mfma_f32_16x16x32_bf16 (x as 3 exact bf16 limbs)",
                "achieved": achieved, "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / BF16_MFMA_PEAK_TFLOPS, "fp32_equivalent_tflops": tf,
                "fp32_mfma_peak": FP32_MFMA_PEAK_TFLOPS}
    return {"bound": "mfma", "instruction": "v_mfma_f32_16x16x4_f32", "achieved": tf,
            "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tf / FP32_MFMA_PEAK_TFLOPS}


def algo_bytes(m: int, n: int, k: int, rank: int = 0) -> int:
    b = n * k // 2 + 4 * n * (k // 32) + 4 * m * k + 4 * m * n
    if rank:
        b += 4 * k * rank + 4 * rank * n
    return b


def algo_flops(m: int, n: int, k: int, rank: int = 0) -> int:
    f = 2 * m * n * k
    if rank:
        f += 2 * m * rank * (k + n)
    return f


def make_weights(torch, n: int, k: int, copies: int, gen, with_all: bool = False):
    """`copies` distinct weight matrices, stored back to back: copy i is rows [i*n, (i+1)*n) of one
    [copies*n, k/2] packed tensor (and of one scale tensor), so the same bytes also form one matrix
    of copies*n columns (the layout of concatenated projection weights)."""
    packed_all = torch.randint(0, 256, (copies * n, k // 2), dtype=torch.uint8, device="cuda", generator=gen)
    scales_all = torch.rand((copies * n, k // 32), dtype=torch.float32, device="cuda", generator=gen) * 0.04 + 0.01
    packed = [packed_all[i * n:(i + 1) * n] for i in range(copies)]
    scales = [scales_all[i * n:(i + 1) * n] for i in range(copies)]
    if with_all:
        return packed, scales, packed_all, scales_all
    return packed, scales


def time_region(torch, fn, steps: int, warmup: int) -> float:
    """Runs fn() warmup times untimed, then steps times between HIP events; returns ms per step."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def bench_gemv(torch, session, steps: int, warmup: int, copies: int = 64, launch: str = "hip-graph") -> dict:
    """The 64-copy sweep timed twice, launched from the host stream by stream and replayed as one HIP graph
    of the same 64 launches; `launch` picks which one is the headline."""
    m, n, k = 1, 14336, 4096
    gen = torch.Generator(device="cuda").manual_seed(1234)
    packed, scales, packed_all, scales_all = make_weights(torch, n, k, copies, gen, with_all=True)
    x = torch.randn((m, k), dtype=torch.float32, device="cuda", generator=gen)
    ys = [torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(copies)]
    y_all = torch.empty((m, copies * n), dtype=torch.float32, device="cuda")

    def sweep():
        st = torch.cuda.current_stream().cuda_stream
        for i in range(copies):
            session.q4gemm_device(x.data_ptr(), packed[i].data_ptr(), scales[i].data_ptr(), ys[i].data_ptr(), m, n,
                                  k, st)

    sweep()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sweep()
    bytes_per = algo_bytes(m, n, k)
    modes = {}
    for name, fn in (("stream", sweep), ("hip-graph", g.replay)):
        ms = time_region(torch, fn, steps, warmup)
        per_launch_s = ms * 1e-3 / copies
        modes[name] = {"ms_per_step": ms, "per_launch_us": per_launch_s * 1e6, "gbs": bytes_per / per_launch_s / 1e9}
    del g

    # The same 64 matrices read as one matrix of 64*n columns in a single launch: what the kernel
    # streams when one launch's ramp-up and drain are amortised (fused projections sharing x).
    def one_launch():
        session.q4gemm_device(x.data_ptr(), packed_all.data_ptr(), scales_all.data_ptr(), y_all.data_ptr(), m,
                              copies * n, k, torch.cuda.current_stream().cuda_stream)

    ms_all = time_region(torch, one_launch, max(3, steps // 5), 2)
    bytes_all = algo_bytes(m, copies * n, k)
    concat = {"n": copies * n, "bytes": bytes_all, "us_per_launch": round(ms_all * 1e3, 3),
              "gbs": round(bytes_all / (ms_all * 1e-3) / 1e9, 2),
              "frac": round(bytes_all / (ms_all * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    head = modes[launch]
    other = {name: {"us_per_launch": round(v["per_launch_us"], 3), "gbs": round(v["gbs"], 2)}
             for name, v in modes.items() if name != launch}
    return {"ms_per_step": head["ms_per_step"], "per_launch_us": head["per_launch_us"], "gbs": head["gbs"],
            "bytes_per_launch": bytes_per, "copies": copies, "launch": launch, "other_launch": other,
            "concatenated": concat, "tflops": algo_flops(m, n, k) * 1e-12 * 1e6 / head["per_launch_us"]}


def bench_gemm(torch, session, m: int, n: int, k: int, copies: int, steps: int, warmup: int, rank: int = 0) -> dict:
    gen = torch.Generator(device="cuda").manual_seed(99)
    packed, scales = make_weights(torch, n, k, copies, gen)
    x = torch.randn((m, k), dtype=torch.float32, device="cuda", generator=gen)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    if rank:
        la = torch.randn((k, rank), dtype=torch.float32, device="cuda", generator=gen) * 0.02
        lb = torch.randn((rank, n), dtype=torch.float32, device="cuda", generator=gen) * 0.02

    def step():
        st = torch.cuda.current_stream().cuda_stream
        for i in range(copies):
            if rank:
                session.q4gemm_lora_device(x.data_ptr(), packed[i].data_ptr(), scales[i].data_ptr(), la.data_ptr(),
                                           lb.data_ptr(), y.data_ptr(), m, n, k, rank, 32.0 / rank, st)
            else:
                session.q4gemm_device(x.data_ptr(), packed[i].data_ptr(), scales[i].data_ptr(), y.data_ptr(), m, n, k,
                                      st)

    ms = time_region(torch, step, steps, warmup)
    per_call = ms * 1e-3 / copies
    fl = algo_flops(m, n, k, rank)
    by = algo_bytes(m, n, k, rank)
    tf = fl / per_call / 1e12
    return {"m": m, "n": n, "k": k, "rank": rank, "copies": copies, "ms_per_call": per_call * 1e3,
            "tflops": tf, "gbs": by / per_call / 1e9, "flops_per_call": fl, "bytes_per_call": by,
            "roofline": gemm_roofline(m, n, k, per_call)}


def bench_cq4(torch, session, steps: int) -> dict:
    """The CQ4 codebook matmul on the reference's CQ4 benchmark shapes (vulkan-runtime/bench/bench_cq4gemm.cpp:
    bits 4, group 128, non-interleaved, input_scale_recip; 1024^3, 1x512x512, 1024x512x512), device-resident
    inputs, one spaceslug_cq4_matmul_device call per step. TFLOP/s = 2*M*N*K / time, as the reference counts it
    (transform and decode not counted)."""
    from spaceslug_amd.backend import CQ4MatrixStruct

    out = {}
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(7)
    for m, n, k in ((1024, 1024, 1024), (1, 512, 512), (1024, 512, 512)):
        gs = 128
        ng = k // gs
        half = lambda *shape: (torch.rand(shape, generator=gen, device=dev) + 0.5).half()  # noqa: E731
        codebook = (torch.rand(16, generator=gen, device=dev) * 2 - 1).half()
        norms = half(n * ng)
        recip = half(k)
        packed = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=gen)
        a = (torch.rand((m, k), generator=gen, device=dev) * 2 - 1).half()
        c = torch.empty((m, n), dtype=torch.float16, device=dev)
        s = CQ4MatrixStruct(4, k, n, gs, ng, 0, codebook.data_ptr(), None, recip.data_ptr(), norms.data_ptr(),
                            packed.data_ptr(), None, None, None, None, None, None)

        def step():
            session.cq4_matmul_device(s, a.data_ptr(), m, c.data_ptr(), torch.cuda.current_stream().cuda_stream)

        reps = 20 if m > 1 else 200
        ms = time_region(torch, lambda: [step() for _ in range(reps)], max(3, steps // 10), 2) / reps
        out[f"{m}x{n}x{k}"] = {"us_per_call": round(ms * 1e3, 3),
                               "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 3)}
    return out


def copy_reference(torch, steps: int) -> dict:
    """Per-launch time of a device-to-device copy (the runtime's own streaming kernel) of the GEMV's byte
    count, over 64 distinct source buffers swept like the weight copies, and of one 8x larger copy: the
    launch-size effect and the streaming rate next to which the decode GEMV's figure is read. Copies read
    and write, so their GB/s counts both directions."""
    out = {}
    for label, nbytes, copies in (("gemv_size", 36_700_160, 64), ("x8_size", 8 * 36_700_160, 8)):
        src = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(copies)]
        dst = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")

        def sweep():
            for b in src:
                dst.copy_(b)

        ms = time_region(torch, sweep, max(3, steps // 5), 2)
        us = ms * 1e3 / copies
        out[label] = {"bytes_read": nbytes, "bytes_written": nbytes, "us_per_launch": round(us, 3),
                      "gbs_read_plus_write": round(2 * nbytes / us / 1e3, 1)}
        del src, dst
        torch.cuda.empty_cache()
    out["kernel"] = "torch copy_ (device-to-device), same sweep pattern as the weights"
    return out


def launch_floor(torch, steps: int, bytes_per_launch: int) -> dict:
    """Per-launch time of a kernel with almost no work (torch fill_ of one float), 64 launches captured
    into one HIP graph and replayed like the GEMV sweep: the fixed cost every launch of the sweep pays
    (completion, cache maintenance between dependent kernels, dispatch). With it, the highest fraction of
    the HBM peak a single launch of `bytes_per_launch` bytes could reach is
    bytes / (floor + bytes / peak) / peak."""
    bufs = [torch.empty(1, dtype=torch.float32, device="cuda") for _ in range(64)]

    def sweep():
        for b in bufs:
            b.fill_(1.0)

    sweep()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sweep()
    ms = time_region(torch, g.replay, steps, 5)
    del g
    us = ms * 1e3 / len(bufs)
    ideal_us = bytes_per_launch / (HBM_PEAK_GBS * 1e3)
    return {"us_per_launch": round(us, 3), "kernel": "torch fill_ of 4 bytes, 64 launches replayed as one HIP graph",
            "gemv_ceiling_frac": round(ideal_us / (us + ideal_us), 4)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s: float) -> dict:
    """Times the C oracle (double, from the packed bytes) on whole GEMV calls of the same shape: over
    OMP_NUM_THREADS threads (parallel over columns; every output is summed in the same order as with one
    thread) for `budget_s`, then single-threaded for a quarter of that."""
    import numpy as np

    from oracle import oracle as o

    m, n, k = 1, 14336, 4096
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    threads = max(1, min(threads, os.cpu_count() or 1))
    rng = np.random.default_rng(7)
    # 16 distinct weight sets (590 MB, beyond any host last-level cache), used in turn
    pool = [(rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8),
             (rng.random((n, k // 32), dtype=np.float32) * 0.04 + 0.01).astype(np.float32)) for _ in range(16)]
    x = rng.standard_normal((m, k)).astype(np.float32)

    def run(nthreads: int, budget: float) -> tuple[int, float]:
        calls, elapsed = 0, 0.0
        while elapsed < budget or calls < 2:
            packed, scales = pool[calls % len(pool)]
            t0 = time.perf_counter()
            o.q4gemm_packed(x, packed, scales, threads=nthreads)
            elapsed += time.perf_counter() - t0
            calls += 1
        return calls, elapsed

    calls, elapsed = run(threads, budget_s)
    calls1, elapsed1 = run(1, budget_s / 4)
    gbs = algo_bytes(m, n, k) * calls / elapsed / 1e9
    gbs1 = algo_bytes(m, n, k) * calls1 / elapsed1 / 1e9
    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{calls} GEMV calls M=1 K=4096 N=14336 (16 random weight sets in turn), double-precision C oracle "
                      f"over {threads} OpenMP threads, {elapsed:.1f} s",
            "single_thread": {"value": gbs1, "unit": "GB/s", "cores": 1,
                              "sample": f"{calls1} calls of the same shape on one thread, {elapsed1:.1f} s"},
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count()}


def load_traffic() -> float | None:
    p = REPO / "profiles" / "q4_gemv_m1_k4096_n14336_traffic.json"
    if p.is_file():
        try:
            return float(json.loads(p.read_text())["hbm_bytes_per_launch"])
        except Exception:
            return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--launch", choices=("hip-graph", "stream"), default="hip-graph",
                    help="headline GEMV timing: the 64-launch sweep replayed as one HIP graph (default) or launched "
                         "call by call on the stream (both are measured and reported)")
    ap.add_argument("--gemv-only", action="store_true", help="skip the secondary GEMM configurations")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget (0 disables)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run 3 plain device copies of this many MiB (a known-traffic kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the int4 path is measured "
              f"on a single MI355X", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    from spaceslug_amd import BackendSession

    session = BackendSession()
    session.capability()  # fails loudly when the HIP library is missing

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copy calibration: 3 x {args.copy_calibration_mib} MiB read + write", file=sys.stderr, flush=True)
        del src, dst

    print(f"[bench] gemv sweep steps={args.steps} warmup={args.warmup} launch={args.launch}", file=sys.stderr,
          flush=True)
    gemv = bench_gemv(torch, session, args.steps, args.warmup, launch=args.launch)
    result = {
        "metric": METRIC,
        "value": round(gemv["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemv["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "int4 group-32 decode GEMV M=1 K=4096 N=14336, 64 weight copies swept per step",
                   "m": 1, "k": 4096, "n": 14336, "copies": 64, "launch": gemv["launch"],
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gemv["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv["gbs"] / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
                     "bytes_per_launch": gemv["bytes_per_launch"],
                     "avg_launch_us": round(gemv["per_launch_us"], 3)},
        "gemv_other_launch": gemv["other_launch"],
        "gemv_concatenated": gemv["concatenated"],
    }
    del gemv
    torch.cuda.empty_cache()
    print("[bench] copy reference", file=sys.stderr, flush=True)
    result["copy_reference"] = copy_reference(torch, args.steps)
    result["launch_floor"] = launch_floor(torch, args.steps, result["roofline"]["bytes_per_launch"])
    if not args.gemv_only:
        print("[bench] prefill 2048x4096x14336", file=sys.stderr, flush=True)
        pre = bench_gemm(torch, session, 2048, 14336, 4096, copies=1, steps=max(3, args.steps // 10), warmup=2)
        result["prefill"] = {"value": round(pre["tflops"], 3), "unit": "TFLOP/s",
                             "ms_per_call": round(pre["ms_per_call"], 4), "roofline": pre["roofline"]}
        torch.cuda.empty_cache()
        print("[bench] small batch 16x4096x4096 x32 copies", file=sys.stderr, flush=True)
        sb = bench_gemm(torch, session, 16, 4096, 4096, copies=32, steps=max(3, args.steps // 5), warmup=2)
        result["small_batch"] = {"value": round(sb["tflops"], 3), "unit": "TFLOP/s", "gbs": round(sb["gbs"], 2),
                                 "us_per_call": round(sb["ms_per_call"] * 1e3, 3), "roofline": sb["roofline"]}
        torch.cuda.empty_cache()
        print("[bench] lora 512x4096x4096 r16", file=sys.stderr, flush=True)
        lo = bench_gemm(torch, session, 512, 4096, 4096, copies=1, steps=max(3, args.steps // 5), warmup=2, rank=16)
        result["lora"] = {"value": round(lo["tflops"], 3), "unit": "TFLOP/s",
                          "us_per_call": round(lo["ms_per_call"] * 1e3, 3), "roofline": lo["roofline"]}
        torch.cuda.empty_cache()
        print("[bench] cq4 codebook matmul", file=sys.stderr, flush=True)
        result["cq4"] = bench_cq4(torch, session, args.steps)
    if args.cpu_seconds > 0:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
