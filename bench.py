"""Benchmark of the quantized-matmul hot path on one MI355X.

Metric: 4-bit qmv/qmm achieved HBM GB/s (% of peak) and
µs/call at K=5120 N=17408 (configs[1]; configs[0] is the reference's
CPU-runnable case).  One *step* is one quantized_matmul call at M=1 over
one of R rotated copies of the 4-bit weights (R copies exceed the 256 MB
Infinity Cache, so every step streams its weights from HBM, the reference's
own "cold chain" rule).  The K timed steps are one HIP graph replay,
bracketed by torch.cuda.synchronize(), so host launch overhead is out of
the measurement; inputs are resident in HBM before the timed region.

Printed JSON line (rank 0 only; one GPU):
  value      whole-job algorithmic GB/s over the timed region
  roofline   the dominant kernel's algorithmic bytes per launch over its
             average launch duration, from HIP events recorded on the
             launching stream around each launch in an eager pass that
             mirrors the timed steps; peak = 8000 GB/s (MI355X HBM3E)
  cpu_baseline  the C oracle (oracle/qmm_oracle.c, OpenMP) timed on this
             host's cores over a bounded sample of the same workload
  sweep      µs/call and GB/s for M = 1, 2, 4, 8, 16 on both config-2 shapes

Algorithmic bytes per call (M rows): packed weights N*K/2 + scales and
biases 2*2*N*K/64 + x 2*M*K + out 2*M*N.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
METRIC = "4-bit qmv/qmm achieved HBM GB/s (% peak) + µs/call, M=1..16, K=5120 N=17408"


def algo_bytes(M: int, N: int, K: int, bits: int = 4, gs: int = 64) -> int:
    return N * K * bits // 8 + 2 * 2 * N * (K // gs) + 2 * M * K + 2 * M * N


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=8, help="rotated weight copies (>256 MB total)")
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


def make_weights(torch, N, K, copies, seed=1, bits=4, gs=64):
    """R distinct random 4-bit weight copies on the GPU (synthetic, seeded).

    Codes are uniform random words; scales/biases are small bf16 values.  The
    kernel's work does not depend on the values, and the parity tests cover
    MLX-quantized N(0, 0.02) weights of the same shape.
    """
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    out = []
    for _ in range(copies):
        w = torch.randint(-2**31, 2**31 - 1, (N, K * bits // 32), dtype=torch.int32, device="cuda",
                          generator=g).view(torch.uint32)
        s = (torch.rand((N, K // gs), device="cuda", generator=g) * 0.002).to(torch.bfloat16)
        b = (torch.rand((N, K // gs), device="cuda", generator=g) * 0.02 - 0.01).to(torch.bfloat16)
        out.append((w, s, b))
    return out


def time_graph(torch, mq, xs, ws, steps, warmup):
    """Warmup eagerly, then capture `steps` calls (rotating weights) in one graph."""
    R = len(ws)
    for i in range(warmup):
        mq.quantized_matmul(xs[i % len(xs)], *ws[i % R])
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                outs.append(mq.quantized_matmul(xs[i % len(xs)], *ws[i % R]))
    torch.cuda.synchronize()
    graph.replay()                       # untimed replay: graph upload / first-touch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0), graph, outs


_SLEEP_CYCLES_PER_S = None


def _sleep_rate(torch):
    """Calibrate torch.cuda._sleep (a bounded spin kernel): cycles per second."""
    global _SLEEP_CYCLES_PER_S
    if _SLEEP_CYCLES_PER_S is None:
        torch.cuda.synchronize()
        torch.cuda._sleep(1_000_000)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        torch.cuda._sleep(10_000_000)
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_S = 10_000_000 / max(time.perf_counter() - t0, 1e-6)
    return _SLEEP_CYCLES_PER_S


def time_events(torch, mq, xs, ws, launches):
    """Per-launch durations from HIP events on the launching stream.

    A bounded GPU sleep sized to three times the host's enqueue time is
    queued first, so every launch and event is enqueued while the GPU is
    still busy; the launches then run back to back and each event pair
    brackets exactly one kernel.
    """
    R = len(ws)
    st = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(launches + 1)]
    # host enqueue cost per launch (measured, GPU idle afterwards is fine here)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(min(launches, 50)):
        mq.quantized_matmul(xs[i % len(xs)], *ws[i % R])
    per_launch = (time.perf_counter() - t0) / min(launches, 50)
    torch.cuda.synchronize()
    cycles = int(_sleep_rate(torch) * max(3 * per_launch * launches, 0.005))
    torch.cuda._sleep(min(cycles, 2_000_000_000))
    ev[0].record(st)
    for i in range(launches):
        mq.quantized_matmul(xs[i % len(xs)], *ws[i % R])
        ev[i + 1].record(st)
    torch.cuda.synchronize()
    d = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(launches)]) * 1e3   # us
    return d


def cpu_baseline(N, K, seconds):
    """The C oracle (same arithmetic as the oracle: bf16-exact dequant, fp32
    accumulation) on this host's cores, bounded to ~`seconds`."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cref
    threads = min(len(os.sched_getaffinity(0)), 16)
    rng = np.random.default_rng(3)
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = np.full((N, K // 64), 0x3B00, np.uint16)
    b = np.full((N, K // 64), 0xBC00, np.uint16)
    x = np.full((1, K), 0x3F80, np.uint16)
    cref.qmm(x, w, s, b, 64, 4, threads=threads)            # warm-up (page faults, OpenMP pool)
    reps, t0 = 0, time.perf_counter()
    while True:
        cref.qmm(x, w, s, b, 64, 4, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 200:
            break
    per = el / reps
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(algo_bytes(1, N, K) / per / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{reps} full M=1 calls K={K} N={N} (C oracle, OpenMP {threads} threads, "
                   f"{per * 1e3:.1f} ms/call) on {cpu_model or 'host CPU'}; MLX CPU "
                   "quantized_matmul is not installable here"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU sharding of "
                          "the quantized matmul is designed (N-split, no exchange) but not built",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import mlxturbo_amd as mq

    K, N = 5120, 17408
    ws = make_weights(torch, N, K, args.copies)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    xs = [torch.randn((1, K), device="cuda", generator=g).to(torch.bfloat16) for _ in range(4)]
    bytes_call = algo_bytes(1, N, K)

    elapsed, graph, _ = time_graph(torch, mq, xs, ws, args.steps, args.warmup)
    ms_per_step = elapsed * 1e3 / args.steps
    value = bytes_call * args.steps / elapsed / 1e9

    d = time_events(torch, mq, xs, ws, min(args.steps, 400))
    avg_us = float(np.mean(d))
    achieved = bytes_call / (avg_us * 1e-6) / 1e9

    sweep = {}
    if not args.no_sweep:
        for (KK, NN) in ((5120, 17408), (17408, 5120)):
            wsw = ws if (KK, NN) == (K, N) else make_weights(torch, NN, KK, args.copies, seed=2)
            for M in (1, 2, 4, 8, 16):
                xm = [torch.randn((M, KK), device="cuda", generator=g).to(torch.bfloat16)]
                dd = time_events(torch, mq, xm, wsw, 100)
                us = float(np.median(dd))
                sweep[f"K{KK}_N{NN}_M{M}"] = {
                    "us": round(us, 2),
                    "GBps": round(algo_bytes(M, NN, KK) / (us * 1e-6) / 1e9, 1),
                }
            del wsw
            torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline(N, K, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"config2 qmv: M=1 x K={K} -> N={N}, MLX affine 4-bit g64, bf16 "
                         f"scales/biases/activations, {args.copies} rotated weight copies "
                         f"({args.copies * bytes_call / 1e6:.0f} MB > 256 MB MALL), "
                         "one HIP graph of `steps` launches"),
            "M": 1, "K": K, "N": N, "bits": 4, "group_size": 64,
            "bytes_per_call": bytes_call,
            "pct_peak": round(100 * value / HBM_PEAK_GBS, 1),
            "us_per_call": round(ms_per_step * 1e3, 3),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "qmm_skinny_kernel<bf16,4,64>",
            "avg_launch_us": round(avg_us, 3),
        },
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
