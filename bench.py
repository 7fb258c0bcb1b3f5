"""Benchmark of the quantized-matmul hot path on one MI355X.

Metric: 4-bit qmv/qmm achieved HBM GB/s (% of peak) and
µs/call at K=5120 N=17408.  The headline workload is configs[1] at M=1 (the
decode qmv): one *step* is one quantized_matmul call over one of R rotated
copies of the 4-bit weights (R copies exceed the 256 MB Infinity Cache, so
every step streams its weights from HBM -- the reference's own "cold chain"
rule, the reference's CLAUDE.md:13-16).  Inputs are resident in HBM before
timing starts.

Timing: the K timed steps are captured in one HIP graph on a dedicated
stream; HIP events recorded on that same stream bracket one replay, with
torch.cuda.synchronize() on both sides.  One step is exactly one kernel
launch, so ``ms_per_step`` is also the dominant kernel's average launch
duration, the denominator of ``roofline.achieved``.

Algorithmic bytes per call (M rows, K, N, b bits, group 64, 16-bit T):
packed weights N*K*b/8 + scales and biases 2*2*N*K/64 + x 2*M*K + out 2*M*N.

``roofline`` carries two denominators: MI355X's published 8 TB/s (``peak``,
``frac``) and a plain streaming read of the same byte count measured the
same way on the same GPU (``measured_read``, ``frac_of_measured_read``;
mlxturbo_amd/csrc/read_probe.hip, a measurement helper outside the ABI).

``sweep`` reports the same measurement for configs 1, 2 (both shapes,
M = 1..16) and 5 (8-bit lm_head); ``cpu_baseline`` times the C restatement
of the oracle (oracle/qmm_oracle.c, OpenMP) on this host's cores over a
bounded sample of the headline workload, and ``cpu_sweep`` does the same
beside one case of each swept row family (skinny M=16, 8-bit lm_head, wide
M=512, gather decode and prefill) on a slice of N or of the pairs, scaled
to the whole call.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "4-bit qmv/qmm achieved HBM GB/s (% peak) + µs/call, M=1..16, K=5120 N=17408"
MALL_BYTES = 256 << 20


def algo_bytes(M: int, N: int, K: int, bits: int = 4, gs: int = 64) -> int:
    return N * K * bits // 8 + 2 * 2 * N * (K // gs) + 2 * M * K + 2 * M * N


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=0,
                   help="rotated weight copies (default: enough to exceed 2x the 256 MB MALL)")
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--copy-probe", type=int, default=0,
                   help="run a plain copy of this many bytes first (counter calibration)")
    p.add_argument("--case", default="",
                   help="run one sweep case only and print its result (for profiling): "
                        "wide<M> (configs[2]), gather_<proj>_<routing>_T<T> (configs[3] decode), "
                        "gather_glu_<routing>_T<T> (fused gate+up+SiLU), qmv<M> / qmvdown<M> "
                        "(configs[1] skinny), combine (MoE combine, 2048 x top-8 x 2048), "
                        "gather_prefill_<proj>_<routing> (2048 tokens), "
                        "moe_layer_<routing>_T<T> (whole decode MoE layer), "
                        "moe_block_<routing>_T<T> (decode MoE block: routing, layer, "
                        "shared-expert merge), "
                        "moe_layer_prefill_<routing>[_sortpath] (whole prefill MoE layer, "
                        "2048 tokens), "
                        "route<T> (MoE routing + shared gate), "
                        "mfma_ceiling (the measured bf16 MFMA ceiling and its clock)")
    return p.parse_args()


def run_case(torch, mq, case: str) -> dict:
    """One sweep entry by name, so a profiler sees only its kernels."""
    K, N = 5120, 17408
    banks = {"gate_up": (1024, 2048), "down": (2048, 512)}
    if case.startswith("qmv"):
        # qmv<M> (K=5120 N=17408) or qmvdown<M> (K=17408 N=5120), 4-bit g64
        down = case.startswith("qmvdown")
        M = int(case[7:] if down else case[3:])
        KK, NN = (N, K) if down else (K, N)
        r = measure_qmm(torch, mq, M, NN, KK, 4, 200, 20)
        return {"case": case, "us": round(r["us"], 2), "GBps": round(r["GBps"], 1)}
    if case == "combine":
        return {"case": case, **measure_combine(torch, mq, 2048, 8, 2048, 50, 3)}
    if case == "mfma_ceiling":
        return {"case": case, **measure_mfma_ceiling(torch)}
    if case.startswith("wide"):
        M = int(case[4:])
        r = measure_qmm(torch, mq, M, N, K, 4, 20 if M >= 2048 else 100, 10, copies=2)
        tflops = 2.0 * M * N * K / (r["us"] * 1e-6) / 1e12
        return {"case": case, "us": round(r["us"], 2), "TFLOPs": round(tflops, 1),
                "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    if case.startswith("gather_prefill_"):
        proj, routing = case[len("gather_prefill_"):].rsplit("_", 1)
        NN, KK = banks[proj]
        return {"case": case, **measure_gather_prefill(torch, mq, 2048, NN, KK, routing, 20, 3)}
    if case.startswith("route"):
        return {"case": case, **measure_route(torch, mq, int(case[len("route"):] or 1), 100, 5)}
    if case.startswith("moe_block_"):
        routing, t = case[len("moe_block_"):].rsplit("_T", 1)
        return {"case": case, **measure_moe_block(torch, mq, int(t), routing, 100, 5)}
    if case.startswith("moe_layer_prefill_"):
        routing = case[len("moe_layer_prefill_"):]
        sort = routing.endswith("_sortpath")
        routing = routing[:-len("_sortpath")] if sort else routing
        return {"case": case, **measure_moe_layer_prefill(torch, mq, 2048, routing, 20, 3,
                                                          tables=not sort)}
    if case.startswith("moe_layer_"):
        routing, t = case[len("moe_layer_"):].rsplit("_T", 1)
        return {"case": case, **measure_moe_layer(torch, mq, int(t), routing, 100, 5)}
    if case.startswith("gather_"):
        body, t = case[len("gather_"):].rsplit("_T", 1)
        proj, routing = body.rsplit("_", 1)
        NN, KK = banks["gate_up" if proj == "glu" else proj]
        return {"case": case, **measure_gather(torch, mq, int(t), NN, KK, routing, 100, 5,
                                               glu=proj == "glu")}
    raise SystemExit(f"unknown --case {case!r}")


def copies_for(nbytes: int, requested: int = 0) -> int:
    if requested:
        return requested
    return max(2, -(-2 * MALL_BYTES // nbytes))


def make_weights(torch, N, K, copies, seed=1, bits=4, gs=64):
    """`copies` distinct weight sets on the GPU: seeded N(0, 0.02) bf16
    matrices quantized by the library's own ``quantize`` (MLX's affine
    scheme), the weights the stated workload names.  The dense matrix is
    made and quantized in slabs of rows so that only the packed copies stay
    resident (the 8-bit lm_head is 2.5 GB of bf16 per copy)."""
    import mlxturbo_amd as mq
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    slab = max(1, min(N, (256 << 20) // (2 * K)))
    out = []
    for _ in range(copies):
        w = torch.empty((N, K * bits // 32), dtype=torch.uint32, device="cuda")
        s = torch.empty((N, K // gs), dtype=torch.bfloat16, device="cuda")
        b = torch.empty_like(s)
        for r0 in range(0, N, slab):
            r1 = min(N, r0 + slab)
            dense = (torch.randn((r1 - r0, K), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
            w[r0:r1], s[r0:r1], b[r0:r1] = mq.quantize(dense, gs, bits)
        out.append((w, s, b))
    return out


def time_graph(torch, fn, steps, warmup):
    """Warm up eagerly, capture `steps` calls in one graph, time one replay.

    Returns (elapsed seconds of the replay, per-step seconds).  The warm-up
    runs on the capture stream (so per-stream caches built there serve the
    capture), and events are recorded on that stream, the stream every
    launch in the graph runs on.
    """
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):          # warm-up on the capture stream
        for i in range(warmup):
            fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fn(i)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        graph.replay()                      # untimed replay: upload, first touch
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    elapsed = e0.elapsed_time(e1) * 1e-3
    del graph
    return elapsed, elapsed / steps


def measure_qmm(torch, mq, M, N, K, bits, steps, warmup, copies=0, seed=1):
    per = algo_bytes(M, N, K, bits)
    R = copies_for(N * K * bits // 8, copies)
    ws = make_weights(torch, N, K, R, seed=seed, bits=bits)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 100)
    xs = [torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16) for _ in range(2)]

    def fn(i):
        w, s, b = ws[i % R]
        mq.quantized_matmul(xs[i % 2], w, s, b, group_size=64, bits=bits)

    elapsed, per_step = time_graph(torch, fn, steps, warmup)
    del ws
    torch.cuda.empty_cache()
    return {"us": per_step * 1e6, "GBps": per / per_step / 1e9, "bytes": per, "copies": R,
            "elapsed": elapsed}


def recorded_traffic():
    """HBM bytes per launch of the headline kernel from the committed counter
    passes (profiles/qmv_b4_K5120_N17408_M1_traffic.md), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "qmv_b4_K5120_N17408_M1_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def zipf_routing(rng, T, top_k, E, s=1.1):
    """top_k distinct experts per token drawn from Zipf(s) over E (rank -> id
    through a fixed seeded permutation), as BASELINE configs[3] specifies."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = np.random.default_rng(12345).permutation(E)
    return np.stack([perm[rng.choice(E, size=top_k, replace=False, p=p)]
                     for _ in range(T)]).astype(np.int32)


def measure_gather(torch, mq, T, N, K, routing, steps, warmup, E=512, top_k=8, nroute=64, seed=4,
                   glu=False):
    """gather_qmm over an E-expert 4-bit bank for T tokens x top_k
    experts; `nroute` seeded routings rotate so weights stream from HBM.
    Algorithmic bytes count each distinct expert's weights once per call.
    glu: the N rows per expert are a gate and an up bank of N/2 rows each,
    through the fused gate+up+SiLU (gather_glu, N/2 outputs per pair)."""
    rng = np.random.default_rng(seed + T)
    routes = [(zipf_routing(rng, T, top_k, E) if routing == "zipf" else
               np.stack([rng.choice(E, size=top_k, replace=False) for _ in range(T)]).astype(np.int32))
              for _ in range(nroute)]
    nb = 2 if glu else 1
    banks = [tuple(t.view(E, N // nb, -1) for t in make_weights(torch, E * N // nb, K, 1,
                                                                 seed=seed + i)[0])
             for i in range(nb)]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((T, 1, 1, K), device="cuda", generator=g).to(torch.bfloat16)
    idx = [torch.from_numpy(r).cuda() for r in routes]
    per_expert = N * K // 2 + 4 * N * (K // 64)
    nbytes = [len(np.unique(r)) * per_expert + 2 * T * K + 2 * T * top_k * N // nb for r in routes]

    def fn(i):
        if glu:
            mq.gather_glu(x, *banks[0], *banks[1], rhs_indices=idx[i % nroute])
        else:
            mq.gather_qmm(x, *banks[0], rhs_indices=idx[i % nroute])

    elapsed, per_step = time_graph(torch, fn, steps, warmup)
    avg_bytes = sum(nbytes[i % nroute] for i in range(steps)) / steps
    uniq = sum(len(np.unique(r)) for r in routes) / nroute
    del banks
    torch.cuda.empty_cache()
    return {"us": round(per_step * 1e6, 2), "GBps": round(avg_bytes / per_step / 1e9, 1),
            "distinct_experts": round(uniq, 1)}


def measure_moe_layer(torch, mq, T, routing, steps, warmup, E=512, top_k=8, hidden=2048,
                      inter=512, nroute=64, seed=8):
    """One whole decode MoE layer of configs[3] (SwitchGLU with the fused
    gate+up+SiLU route and router scores): gather_glu, then the down
    projection with the combine folded in (one or two tokens) or the down
    gather_qmm and the combine epilogue; "launches" counts them.
    Algorithmic bytes: each distinct expert's gate, up and down weights
    once, plus activations."""
    from mlxturbo_amd import nn as mqnn
    rng = np.random.default_rng(seed + T)
    routes = [(zipf_routing(rng, T, top_k, E) if routing == "zipf" else
               np.stack([rng.choice(E, size=top_k, replace=False) for _ in range(T)]).astype(np.int32))
              for _ in range(nroute)]

    def bank(N, K, s):
        (w, sc, b), = make_weights(torch, E * N, K, 1, seed=s)
        return mqnn.QuantizedSwitchLinear(w.view(E, N, -1), sc.view(E, N, -1), b.view(E, N, -1))

    layer = mqnn.SwitchGLU(bank(inter, hidden, seed), bank(inter, hidden, seed + 1),
                           bank(hidden, inter, seed + 2), fuse_gate_up=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((T, hidden), device="cuda", generator=g).to(torch.bfloat16)
    scores = torch.softmax(torch.randn((T, top_k), device="cuda", generator=g), -1)
    idx = [torch.from_numpy(r).cuda() for r in routes]

    def per_expert(N, K):
        return N * K // 2 + 4 * N * (K // 64)

    pe = 2 * per_expert(inter, hidden) + per_expert(hidden, inter)
    act = 2 * T * hidden * 2 + 2 * T * top_k * (inter + hidden) * 2 + 4 * T * top_k
    nbytes = [len(np.unique(r)) * pe + act for r in routes]

    def fn(i):
        layer(x, idx[i % nroute], scores)

    n0 = mq.launch_count()
    fn(0)
    launches = mq.launch_count() - n0
    _, per_step = time_graph(torch, fn, steps, warmup)
    avg_bytes = sum(nbytes[i % nroute] for i in range(steps)) / steps
    del layer
    torch.cuda.empty_cache()
    return {"us": round(per_step * 1e6, 2), "GBps": round(avg_bytes / per_step / 1e9, 1),
            "distinct_experts": round(sum(len(np.unique(r)) for r in routes) / nroute, 1),
            "launches": int(launches)}


def measure_moe_block(torch, mq, T, routing, steps, warmup, E=512, top_k=8, hidden=2048,
                      inter=512, nroute=64, seed=11):
    """The decode MoE block after its router matmul as one timed unit
    (ops.moe_block): routing of float logits with the shared expert's gate,
    the fused gate+up+SiLU gather, the down projection with the combine and
    the shared-expert merge folded in.  Logits rotate over `nroute` sets:
    Gumbel noise plus log p_e, so the top-k is a draw without replacement
    from p (zipf(1.1) over the experts through a fixed permutation, or
    uniform).  Algorithmic bytes: each distinct expert's gate, up and down
    weights once, plus logits, activations and the shared expert's row."""
    rng = np.random.default_rng(seed + T)
    if routing == "zipf":
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
        logp = np.log(p / p.sum())[np.argsort(np.random.default_rng(12345).permutation(E))]
    else:
        logp = np.zeros(E)
    logit_sets = [(rng.gumbel(size=(T, E)) + logp).astype(np.float32) for _ in range(nroute)]
    logits = [torch.from_numpy(l).cuda() for l in logit_sets]
    experts = [np.unique(np.argsort(-l, axis=1, kind="stable")[:, :top_k]) for l in logit_sets]

    def bank(N, K, s):
        (w, sc, b), = make_weights(torch, E * N, K, 1, seed=s)
        return w.view(E, N, -1), sc.view(E, N, -1), b.view(E, N, -1)

    gate, up, down = bank(inter, hidden, seed), bank(inter, hidden, seed + 1), \
        bank(hidden, inter, seed + 2)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((T, hidden), device="cuda", generator=g).to(torch.bfloat16)
    sgw = (torch.randn((hidden,), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    shared = (torch.randn((T, hidden), device="cuda", generator=g) * 0.1).to(torch.bfloat16)

    def per_expert(N, K):
        return N * K // 2 + 4 * N * (K // 64)

    pe = 2 * per_expert(inter, hidden) + per_expert(hidden, inter)
    act = 4 * T * E + 2 * T * hidden * 3 + 2 * hidden + 2 * T * top_k * inter + 2 * T * hidden
    nbytes = [len(e) * pe + act for e in experts]

    def fn(i):
        mq.ops.moe_block(x, logits[i % nroute], top_k, gate, up, down, sgw=sgw, shared=shared)

    n0 = mq.launch_count()
    fn(0)
    launches = mq.launch_count() - n0
    _, per_step = time_graph(torch, fn, steps, warmup)
    avg_bytes = sum(nbytes[i % nroute] for i in range(steps)) / steps
    del gate, up, down
    torch.cuda.empty_cache()
    return {"us": round(per_step * 1e6, 2), "GBps": round(avg_bytes / per_step / 1e9, 1),
            "distinct_experts": round(sum(len(e) for e in experts) / nroute, 1),
            "launches": int(launches)}


def measure_moe_layer_prefill(torch, mq, T, routing, steps, warmup, E=512, top_k=8, hidden=2048,
                              inter=512, nroute=4, seed=9, tables=True):
    """One whole prefill MoE layer of configs[3] (SwitchGLU with router
    scores over T tokens x top_k experts): the segment tables built once and
    shared by the gate, up and down gathers (x read through each pair's
    token), one SwiGLU pass, one combine -- the reference's prefill path
    (fused.py:3283-3316).  tables=False times the sort path instead (two
    argsorts, the gathered x, three table builds, torch's SwiGLU, the
    combine through the inverse permutation).  Reported as dense-equivalent
    TFLOP/s of the three projections (2 P (2 inter hidden + hidden inter))
    and HBM GB/s of the algorithmic bytes (every expert's weights once plus
    activations); "launches" counts library kernels."""
    from mlxturbo_amd import nn as mqnn
    rng = np.random.default_rng(seed + T)
    routes = [(zipf_routing(rng, T, top_k, E) if routing == "zipf" else
               np.stack([rng.choice(E, size=top_k, replace=False) for _ in range(T)]).astype(np.int32))
              for _ in range(nroute)]

    def bank(N, K, s):
        (w, sc, b), = make_weights(torch, E * N, K, 1, seed=s)
        return mqnn.QuantizedSwitchLinear(w.view(E, N, -1), sc.view(E, N, -1), b.view(E, N, -1))

    layer = mqnn.SwitchGLU(bank(inter, hidden, seed), bank(inter, hidden, seed + 1),
                           bank(hidden, inter, seed + 2), prefill_tables=tables)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((T, hidden), device="cuda", generator=g).to(torch.bfloat16)
    scores = torch.softmax(torch.randn((T, top_k), device="cuda", generator=g), -1)
    idx = [torch.from_numpy(r).cuda() for r in routes]
    P = T * top_k

    def per_expert(N, K):
        return N * K // 2 + 4 * N * (K // 64)

    nbytes = (E * (2 * per_expert(inter, hidden) + per_expert(hidden, inter)) + 2 * T * hidden * 2
              + 2 * P * inter * 2 * 3 + 2 * P * hidden + 4 * P)
    flops = 2.0 * P * (2 * inter * hidden + hidden * inter)

    def fn(i):
        layer(x, idx[i % nroute], scores)

    n0 = mq.launch_count()
    fn(0)
    launches = mq.launch_count() - n0
    _, per_step = time_graph(torch, fn, steps, warmup)
    del layer
    torch.cuda.empty_cache()
    return {"us": round(per_step * 1e6, 2), "TFLOPs": round(flops / per_step / 1e12, 1),
            "GBps": round(nbytes / per_step / 1e9, 1), "launches": int(launches)}


def measure_gather_prefill(torch, mq, T, N, K, routing, steps, warmup, E=512, top_k=8, seed=5):
    """The prefill form of configs[3]: T tokens x top_k experts as one
    gather_qmm (x (P, 1, K) sorted by expert, sorted_indices=True, as mlx-lm's
    _gather_sort does); runs the expert-grouped MFMA tile kernel.  Reported
    as dense-equivalent TFLOP/s (2 * P * N * K per call)."""
    rng = np.random.default_rng(seed + T)
    idx = (zipf_routing(rng, T, top_k, E) if routing == "zipf" else
           np.stack([rng.choice(E, size=top_k, replace=False) for _ in range(T)]).astype(np.int32))
    (w, s, b), = make_weights(torch, E * N, K, 1, seed=seed)
    w, s, b = w.view(E, N, -1), s.view(E, N, -1), b.view(E, N, -1)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((T, 1, K), device="cuda", generator=g).to(torch.bfloat16)
    xs = x[torch.from_numpy(order // top_k).cuda()].contiguous()
    rhs = torch.from_numpy(flat[order].copy()).cuda()
    P = T * top_k

    def fn(i):
        mq.gather_qmm(xs, w, s, b, rhs_indices=rhs, sorted_indices=True)

    _, per_step = time_graph(torch, fn, steps, warmup)
    del w, s, b
    torch.cuda.empty_cache()
    tflops = 2.0 * P * N * K / per_step / 1e12
    return {"us": round(per_step * 1e6, 2), "TFLOPs": round(tflops, 1),
            "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "distinct_experts": int(len(np.unique(flat)))}


def measure_combine(torch, mq, rows, top_k, N, steps, warmup, seed=6):
    """MoE combine epilogue over an expert-sorted down-projection output of
    rows*top_k x N (the reference's prefill shape: 2048 tokens x top-8 x
    2048).  Bytes per call: y read once + out written once + inv and w."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    y = torch.randn((rows * top_k, N), device="cuda", generator=g).to(torch.bfloat16)
    inv = torch.argsort(torch.randperm(rows * top_k, device="cuda", generator=g)).to(torch.int32)
    w = torch.rand(rows * top_k, device="cuda", generator=g)

    def fn(i):
        mq.moe_combine(y, inv, w, rows, top_k)

    _, per_step = time_graph(torch, fn, steps, warmup)
    nbytes = 2 * rows * top_k * N + 2 * rows * N + 8 * rows * top_k
    return {"us": round(per_step * 1e6, 2), "GBps": round(nbytes / per_step / 1e9, 1)}


def measure_route(torch, mq, T, steps, warmup, E=512, top_k=8, H=2048, seed=9):
    """MoE routing of T tokens (config-4 router: 512 experts, top-8) with the
    shared-expert gate over the hidden size: one launch, latency-bound."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    logits = torch.randn((T, E), device="cuda", generator=g)
    x = torch.randn((T, H), device="cuda", generator=g).to(torch.bfloat16)
    sgw = (torch.randn((H,), device="cuda", generator=g) * 0.02).to(torch.bfloat16)

    def fn(i):
        mq.moe_route(logits, top_k, x, sgw)

    _, per_step = time_graph(torch, fn, steps, warmup)
    return {"us": round(per_step * 1e6, 2), "bytes": T * (4 * E + 2 * H) + 2 * H + T * 8 * top_k}


def measure_dequant(torch, mq, N, K, steps, warmup):
    R = copies_for(N * K // 2)
    ws = make_weights(torch, N, K, R, seed=7)
    per = N * K // 2 + 4 * N * (K // 64) + 2 * N * K

    def fn(i):
        w, s, b = ws[i % R]
        mq.dequantize(w, s, b, group_size=64, bits=4)

    _, per_step = time_graph(torch, fn, steps, warmup)
    del ws
    torch.cuda.empty_cache()
    return {"us": round(per_step * 1e6, 2), "GBps": round(per / per_step / 1e9, 1)}


def measure_stream_read(torch, nbytes, steps=200, warmup=10):
    """The second roofline denominator: a plain streaming read of `nbytes`
    (mlxturbo_amd/csrc/read_probe.hip, contiguous non-temporal 16-byte
    loads, four workgroups per CU: the fastest of a sweep over cache
    policies and grids) over rotated copies that exceed the MALL, timed the
    same way as the kernel (one HIP graph of `steps` launches).  What one
    MI355X reads per second at this size, launch and ramp included."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "mlxturbo_amd",
                                   "libmq_read_probe.so"))
    lib.mq_read_probe.restype = ctypes.c_int
    lib.mq_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_void_p]
    nbytes -= nbytes % 16
    R = copies_for(nbytes)
    bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(R)]
    sink = torch.empty(1024, dtype=torch.uint8, device="cuda")
    wgs = 4 * torch.cuda.get_device_properties(0).multi_processor_count

    def fn(i):
        rc = lib.mq_read_probe(bufs[i % R].data_ptr(), nbytes, sink.data_ptr(), wgs,
                               torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"mq_read_probe failed: {rc}")

    _, per_step = time_graph(torch, fn, steps, warmup)
    del bufs
    torch.cuda.empty_cache()
    return {"us": round(per_step * 1e6, 2), "GBps": round(nbytes / per_step / 1e9, 1),
            "bytes": nbytes, "how": "plain non-temporal 16-byte loads, 4 workgroups per CU, "
                                    "rotated copies, one HIP graph "
                                    "(mlxturbo_amd/csrc/read_probe.hip)"}


def measure_mfma_ceiling(torch, ms_target=10.0):
    """The measured ceiling of the MFMA rooflines: 8-wave workgroups, four per
    CU, each wave 4 chains of bf16 v_mfma_f32_32x32x16 on operands rewritten
    every round (mlxturbo_amd/csrc/read_probe.hip `mq_mfma_probe`), timed
    with HIP events after two warm-up launches; the shader clock they ran at
    is the median over workgroups of (cycles / 100 MHz real-time ticks).
    Under MFMA load the clock drops below its 2.4 GHz peak, and further with
    more bit activity, so this is what the matrix cores sustain here."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "mlxturbo_amd",
                                   "libmq_read_probe.so"))
    lib.mq_mfma_probe.restype = ctypes.c_int
    lib.mq_mfma_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_void_p]
    wgs = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(2048, dtype=torch.uint8, device="cuda")
    clk = torch.zeros(4 * wgs, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream()
    flop_per_iter = 4 * 32768.0 * 8 * wgs
    iters = int(ms_target * 1e-3 * 2.0e15 / flop_per_iter)
    for _ in range(2):
        if lib.mq_mfma_probe(iters, wgs, sink.data_ptr(), clk.data_ptr(), st.cuda_stream):
            raise RuntimeError("mq_mfma_probe failed")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    if lib.mq_mfma_probe(iters, wgs, sink.data_ptr(), clk.data_ptr(), st.cuda_stream):
        raise RuntimeError("mq_mfma_probe failed")
    e1.record(st)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3
    c = clk.view(wgs, 4).cpu().numpy().astype(np.float64)
    mhz = float(np.median((c[:, 1] - c[:, 0]) / np.maximum(c[:, 3] - c[:, 2], 1.0) * 100.0))
    return {"TFLOPs": round(flop_per_iter * iters / sec / 1e12, 1), "clock_MHz": round(mhz),
            "how": "bf16 32x32x16 MFMA loop on changing operands, 8 waves x 4 workgroups per CU "
                   "(mlxturbo_amd/csrc/read_probe.hip mq_mfma_probe)"}


def copy_probe(torch, nbytes, reps=4):
    """A plain device copy of known size, for calibrating rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters against the bytes actually moved."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def cpu_threads() -> tuple:
    """(threads used, cores the host's affinity mask shows).  The GPU box
    grants one GPU's share of the host (OMP_NUM_THREADS, 16 there) whatever
    the affinity mask shows, so the OpenMP legs use that share."""
    affinity = len(os.sched_getaffinity(0))
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        share = 0
    return (min(share, affinity) if share > 0 else affinity), affinity


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, seconds, max_reps=200):
    fn()                                                  # warm-up (page faults, thread pool)
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= max_reps:
            return el / reps, reps


def torch_cpu_qmm(torch, x, w, s, b, gs=64, bits=4):
    """torch-CPU dequantize -> matmul over MLX-format tensors (the second
    MLX-CPU substitute): codes unpacked with shifts and masks, s*q + b in
    float32 rounded to bf16 per weight, then a float32 matmul."""
    per = 32 // bits
    shifts = torch.arange(per, dtype=torch.int64) * bits
    codes = ((w.to(torch.int64).unsqueeze(-1) >> shifts) & ((1 << bits) - 1))
    codes = codes.reshape(w.shape[0], -1).to(torch.float32)
    deq = (codes.view(w.shape[0], -1, gs) * s.float().unsqueeze(-1)
           + b.float().unsqueeze(-1)).reshape(w.shape[0], -1)
    deq = deq.to(torch.bfloat16).float()
    return (x.float() @ deq.T).to(torch.bfloat16)


def cpu_baseline(N, K, seconds):
    """The C restatement of the oracle (bf16-exact dequant, fp32 accumulation,
    OpenMP) on this host's cores, bounded to about `seconds`, with all of the
    box's threads and with one; and a torch-CPU dequantize -> matmul of the
    same call.  MLX's CPU quantized_matmul is not installable here."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cref
    import torch
    threads, affinity = cpu_threads()
    rng = np.random.default_rng(3)
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = np.full((N, K // 64), 0x3B00, np.uint16)
    b = np.full((N, K // 64), 0xBC00, np.uint16)
    x = np.full((1, K), 0x3F80, np.uint16)
    per, reps = _timed(lambda: cref.qmm(x, w, s, b, 64, 4, threads=threads), seconds)
    per1, reps1 = _timed(lambda: cref.qmm(x, w, s, b, 64, 4, threads=1), seconds / 2, 20)
    tw = torch.from_numpy(w.view(np.int32))
    ts = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    tx = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    nt0 = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        per_t, reps_t = _timed(lambda: torch_cpu_qmm(torch, tx, tw, ts, tb), seconds / 2, 50)
    finally:
        torch.set_num_threads(nt0)
    nbytes = algo_bytes(1, N, K)
    model = cpu_model()
    return {
        "value": round(nbytes / per / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": model,
        "host_affinity_cores": affinity,
        "one_thread": {"value": round(nbytes / per1 / 1e9, 3), "unit": "GB/s",
                       "ms_per_call": round(per1 * 1e3, 2), "reps": reps1},
        "torch_cpu": {"value": round(nbytes / per_t / 1e9, 3), "unit": "GB/s",
                      "ms_per_call": round(per_t * 1e3, 2), "reps": reps_t, "threads": threads,
                      "what": "torch-CPU dequantize (bf16-rounded per weight) -> fp32 matmul"},
        "sample": (f"{reps} full M=1 calls K={K} N={N} (C oracle oracle/qmm_oracle.c, OpenMP "
                   f"{threads} threads = the box's CPU share, {per * 1e3:.1f} ms/call); "
                   f"1 thread {per1 * 1e3:.1f} ms/call; torch-CPU {per_t * 1e3:.1f} ms/call; "
                   "MLX's CPU quantized_matmul is not installable here"),
    }


def cpu_rows(seconds):
    """The C oracle beside each swept row family, on a bounded slice of the
    same workload (a fraction of N, or of the pairs), timed for about
    `seconds` and scaled to the whole call; units as in the GPU sweep."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cref
    threads, _ = cpu_threads()
    rng = np.random.default_rng(5)

    def timed(fn):
        fn()                                              # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds or reps >= 50:
                return el / reps

    def packed(N, K, bits, E=1):
        w = rng.integers(0, 2**32, size=(E * N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
        s = np.full((E * N, K // 64), 0x3B00, np.uint16)
        b = np.full((E * N, K // 64), 0xBC00, np.uint16)
        return w, s, b

    rows = {}
    # dense skinny / wide / lm_head: a 1/frac slice of N, scaled back up
    for key, (M, K, N, bits, frac, unit) in {
            "b4_K5120_N17408_M16": (16, 5120, 17408, 4, 8, "GBps"),
            "b8_K5120_N248320_M1": (1, 5120, 248320, 8, 16, "GBps"),
            "b4_K5120_N17408_M512": (512, 5120, 17408, 4, 32, "TFLOPs")}.items():
        n = N // frac
        w, s, b = packed(n, K, bits)
        x = np.full((M, K), 0x3F80, np.uint16)
        us = timed(lambda: cref.qmm(x, w, s, b, 64, bits, threads=threads)) * frac * 1e6
        r = {"us": round(us, 1), "sample": f"M={M} K={K} N={n} (1/{frac} of N), x{frac}"}
        if unit == "GBps":
            r["GBps"] = round(algo_bytes(M, N, K, bits) / us / 1e3, 3)
        else:
            r["TFLOPs"] = round(2.0 * M * N * K / us / 1e6, 4)
        rows[key] = r
    # MoE gather over the config-4 gate/up bank: decode T=8 (all 64 pairs) and
    # prefill T=2048 (1/64 of the 16384 pairs), zipf routing
    E, N, K = 512, 1024, 2048
    w, s, b = packed(N, K, 4, E)
    w, s, b = w.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1)
    for key, (T, frac) in {"gather_gate_up_zipf_T8": (8, 1),
                           "gather_prefill_gate_up_zipf_T2048": (2048, 64)}.items():
        idx = zipf_routing(np.random.default_rng(4 + T), T, 8, E).reshape(-1)
        P = idx.size // frac
        rhs = np.ascontiguousarray(idx[:P])
        lhs = np.arange(P, dtype=np.int32) // 8
        x = np.full((T, 1, K), 0x3F80, np.uint16)
        us = timed(lambda: cref.gather_qmm(x, w, s, b, lhs, rhs, 64, 4, threads=threads))
        us *= frac * 1e6
        U = len(np.unique(idx))
        r = {"us": round(us, 1), "sample": f"{P} of {idx.size} pairs, x{frac}"}
        if frac == 1:
            byt = U * (N * K // 2 + 4 * N * (K // 64)) + 2 * T * K + 2 * idx.size * N
            r["GBps"] = round(byt / us / 1e3, 3)
        else:
            r["TFLOPs"] = round(2.0 * idx.size * N * K / us / 1e6, 4)
        rows[key] = r
    return {"threads": threads, "kind": "port",
            "what": "C oracle (oracle/qmm_oracle.c, OpenMP): exact bf16 dequant per weight, "
                    "fp32 accumulation; gather loops over pairs as the reference's contract "
                    "defines it",
            "rows": rows}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the quantized matmul "
                          "shards along N without exchange, and no multi-GPU path is built",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import mlxturbo_amd as mq

    if args.copy_probe:
        copy_probe(torch, args.copy_probe)
    if args.case:
        print(json.dumps(run_case(torch, mq, args.case)))
        return
    K, N = 5120, 17408
    head = measure_qmm(torch, mq, 1, N, K, 4, args.steps, args.warmup, args.copies)
    value = head["GBps"]
    ms_per_step = head["us"] * 1e-3
    read = measure_stream_read(torch, head["bytes"])

    # every sweep row runs a fixed number of steps of its own, whatever
    # --steps says (--steps and --warmup are the headline's), so a row reads
    # the same from any command line
    sweep = {}
    if not args.no_sweep:
        for (KK, NN, bits, Ms) in ((4096, 4096, 4, (1,)), (5120, 17408, 4, (2, 4, 8, 16)),
                                   (17408, 5120, 4, (1, 2, 4, 8, 16, 32, 48)),
                                   (5120, 248320, 8, (1, 2, 4))):
            for M in Ms:
                r = measure_qmm(torch, mq, M, NN, KK, bits, 100, 5)
                sweep[f"b{bits}_K{KK}_N{NN}_M{M}"] = {
                    "us": round(r["us"], 2), "GBps": round(r["GBps"], 1),
                    "pct_peak": round(100 * r["GBps"] / HBM_PEAK_GBS, 1)}

        # config 3: prefill widths on the MFMA tile kernel (compute-bound)
        # configs[2] (512/2048/8192) plus points across the bandwidth/compute
        # crossover (M ~ 95 at the MFMA ridge; up to ~70 rows run as 32-row
        # skinny launches): HBM GB/s and TFLOP/s for each, and the fraction
        # of the measured MFMA ceiling
        ceiling = measure_mfma_ceiling(torch)
        sweep["mfma_ceiling"] = ceiling
        for M in (32, 64, 96, 256, 512, 2048, 8192):
            r = measure_qmm(torch, mq, M, N, K, 4, 20 if M >= 2048 else 100, 3, copies=2)
            tflops = 2.0 * M * N * K / (r["us"] * 1e-6) / 1e12
            sweep[f"b4_K{K}_N{N}_M{M}"] = {
                "us": round(r["us"], 2), "TFLOPs": round(tflops, 1),
                "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                "frac_of_measured_mfma": round(tflops / ceiling["TFLOPs"], 4),
                "GBps": round(r["GBps"], 1)}

        # the transposed (down-proj) shape at prefill widths: few column
        # tiles, K split over workgroups
        for M in (64, 512, 2048):
            r = measure_qmm(torch, mq, M, K, N, 4, 20 if M >= 2048 else 100, 3, copies=2)
            tflops = 2.0 * M * N * K / (r["us"] * 1e-6) / 1e12
            sweep[f"b4_K{N}_N{K}_M{M}"] = {
                "us": round(r["us"], 2), "TFLOPs": round(tflops, 1),
                "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                "GBps": round(r["GBps"], 1)}

        # config 4: MoE gather at decode/verify widths (gate/up and down banks)
        for routing in ("zipf", "uniform"):
            for T in (1, 4, 8):
                for name, (NN, KK) in (("gate_up", (1024, 2048)), ("down", (2048, 512))):
                    sweep[f"gather_{name}_{routing}_T{T}"] = measure_gather(
                        torch, mq, T, NN, KK, routing, 100, 5)
                # the same gate/up bytes through the fused gate+up+SiLU kernel
                sweep[f"gather_glu_{routing}_T{T}"] = measure_gather(
                    torch, mq, T, 1024, 2048, routing, 100, 5, glu=True)
                # the whole layer: gate+up+SiLU, down, router-weighted combine
                sweep[f"moe_layer_{routing}_T{T}"] = measure_moe_layer(
                    torch, mq, T, routing, 100, 5)
                # the block: routing + shared gate, the layer, the shared merge
                sweep[f"moe_block_{routing}_T{T}"] = measure_moe_block(
                    torch, mq, T, routing, 100, 5)
        for T in (1, 4, 8):
            sweep[f"moe_route_T{T}_E512_k8"] = measure_route(torch, mq, T, 100, 5)
        # config 4 banks at prefill width (2048 tokens): expert-grouped MFMA tiles
        for routing in ("zipf", "uniform"):
            for name, (NN, KK) in (("gate_up", (1024, 2048)), ("down", (2048, 512))):
                sweep[f"gather_prefill_{name}_{routing}_T2048"] = measure_gather_prefill(
                    torch, mq, 2048, NN, KK, routing, 20, 3)
            # the whole prefill layer (tables shared by its three gathers),
            # and the sort path it replaces
            sweep[f"moe_layer_prefill_{routing}_T2048"] = measure_moe_layer_prefill(
                torch, mq, 2048, routing, 20, 3)
            sweep[f"moe_layer_prefill_{routing}_T2048_sortpath"] = measure_moe_layer_prefill(
                torch, mq, 2048, routing, 20, 3, tables=False)
        sweep["moe_combine_T2048_k8_N2048"] = measure_combine(torch, mq, 2048, 8, 2048, 50, 3)
        sweep["dequant_b4_K5120_N17408"] = measure_dequant(torch, mq, N, K, 50, 3)

    cpu = None if args.no_cpu else cpu_baseline(N, K, args.cpu_seconds)
    cpu_sweep = None if (args.no_cpu or args.no_sweep) else cpu_rows(2.0)

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
            "workload": (f"configs[1] decode qmv: M=1 x K={K} -> N={N}, MLX affine 4-bit g64, "
                         f"bf16 scales/biases/activations, {head['copies']} rotated weight copies "
                         f"({head['copies'] * N * K // 2 / 1e6:.0f} MB > 256 MB MALL), one HIP graph "
                         "of `steps` launches"),
            "M": 1, "K": K, "N": N, "bits": 4, "group_size": 64,
            "bytes_per_call": head["bytes"],
            "pct_peak": round(100 * value / HBM_PEAK_GBS, 1),
            "us_per_call": round(head["us"], 3),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": recorded_traffic(),
            "kernel": "mq::qmv_quad_kernel<bf16,4,64>",
            "avg_launch_us": round(head["us"], 3),
            "measured_read": read,
            "frac_of_measured_read": round(value / read["GBps"], 4),
        },
        "cpu_baseline": cpu,
        "sweep": sweep,
        "cpu_sweep": cpu_sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
