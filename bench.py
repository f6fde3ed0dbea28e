#!/usr/bin/env python3
"""bench.py -- decode throughput of Loom's quantized MoE forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 1,32] [--no-cpu]

Workload (synthetic, seeded): the routed-MoE stack of a Qwen3-30B-A3B-shaped
model -- 48 distinct MoE layers, each hidden 2048, 128 experts top-8, expert
ffn 768, Q4_K gate/up, Q6_K down, f32 router N(0, 1/sqrt(2048)) with a
per-expert Zipf(1.1) logit bias -- all 18.8 GB of experts resident in HBM.
One step = one decode step: every token of the batch through all 48 layers
(router GEMV, softmax top-8, token->expert bucketing, int8 activation
quantization, fused gate/up + SwiGLU, down, gated combine).  Hidden states
are N(0,1) per token and layer; attention and the output head are not part of
this workload (it is named "moe-stack" in the JSON for that reason).

Reported: tok/s at batch 1 (``value``) and batch 32 (``batch32``), the
dominant kernel's HBM roofline fraction measured with HIP events on the
stream the kernels run on, and the CPU restatement of Loom's CPU path timed
on this host's cores over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s + % HBM roofline, Qwen3-30B-A3B-shape Q4_K, batch 1 and 32"
HBM_PEAK_GBS = 8000.0

DIM, FFN, N_EXPERT, TOP_K, N_LAYERS = 2048, 768, 128, 8, 48
Q4_K, Q6_K = 12, 14
GATE_BYTES = 884_736  # one expert's Q4_K [768][2048] plane
DOWN_BYTES = 1_290_240  # one expert's Q6_K [2048][768] plane
ROUTER_BYTES = N_EXPERT * DIM * 4


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", default="1,32")
    ap.add_argument("--layers", type=int, default=N_LAYERS)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0 = the reference's default, host cores - 2 (capped at the box's share)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    return ap.parse_args()


def zipf_bias(rng, n_expert, s=1.1):
    """Per-expert logit bias from a Zipf(s) popularity ranking: a random
    permutation assigns ranks; bias = log(rank^-s), centred."""
    ranks = rng.permutation(n_expert) + 1
    b = np.log(1.0 / ranks.astype(np.float64) ** s)
    return (b - b.mean()).astype(np.float32)


class Stack:
    """48 device-resident MoE layers (device layout) plus, for the first few,
    the GGML bytes on the host for the CPU baseline."""

    def __init__(self, n_layers, host_layers, seed=1234):
        import torch

        from loom_amd import backend as be

        self.layers, self.host = [], []
        rng = np.random.default_rng(seed)
        for li in range(n_layers):
            s = seed + 1000 * li
            gate = be.synth_ggml_dev(Q4_K, FFN, DIM, N_EXPERT, s + 1, 0.02)
            up = be.synth_ggml_dev(Q4_K, FFN, DIM, N_EXPERT, s + 2, 0.02)
            down_g = be.synth_ggml_dev(Q6_K, DIM, FFN, N_EXPERT, s + 3, 0.02)
            down = be.repack_dev(Q6_K, down_g, DIM, FFN, N_EXPERT)  # Q4_K needs no repack
            g = torch.Generator(device="cpu").manual_seed(s + 4)
            router = (torch.randn(N_EXPERT, DIM, generator=g) / np.sqrt(DIM)).float()
            bias = torch.from_numpy(zipf_bias(rng, N_EXPERT))
            layer = be.MoeLayer(DIM, FFN, N_EXPERT, TOP_K, router.cuda(), gate, up, down, Q4_K,
                                Q4_K, Q6_K, router_bias=bias.cuda())
            self.layers.append(layer)
            if li < host_layers:
                torch.cuda.synchronize()
                self.host.append(dict(router=router.numpy(), bias=bias.numpy(),
                                      gate=gate.cpu().numpy(), up=up.cpu().numpy(),
                                      down=down_g.cpu().numpy()))
            del down_g
            if li % 12 == 11:
                log(f"synthesised {li + 1}/{n_layers} layers")
        torch.cuda.synchronize()


def run_step(stack, normed, outs, combine, ids=None):
    for li, layer in enumerate(stack.layers):
        layer(normed, outs[li], combine=combine, ids=None if ids is None else ids[li])


def bench_batch(stack, b, steps, warmup, use_graph):
    """Time `steps` decode steps of batch b; returns (ms_per_step, kernel stats)."""
    import torch

    import loom_amd
    from loom_amd import backend as be

    L = len(stack.layers)
    g = torch.Generator(device="cpu").manual_seed(77 + b)
    n_inputs = 8
    inputs = [torch.randn(b, DIM, generator=g).cuda() for _ in range(n_inputs)]
    normed = torch.empty(b, DIM, device="cuda")
    outs = [torch.zeros(b, DIM, device="cuda") for _ in range(L)]
    combine = be.COMBINE_SELECTION if b == 1 else be.COMBINE_EXPERT_ASC
    ids = [torch.empty(b, TOP_K, dtype=torch.int32, device="cuda") for _ in range(L)]

    # eager warmup (sizes the library's workspace before any capture)
    for i in range(max(1, warmup)):
        normed.copy_(inputs[i % n_inputs])
        run_step(stack, normed, outs, combine)
    torch.cuda.synchronize()

    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_step(stack, normed, outs, combine)
        for i in range(warmup):
            normed.copy_(inputs[i % n_inputs])
            graph.replay()
        torch.cuda.synchronize()

    # timed region: K steps, synchronised on both sides
    st = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(st)
    for i in range(steps):
        normed.copy_(inputs[i % n_inputs])
        if graph is not None:
            graph.replay()
        else:
            run_step(stack, normed, outs, combine)
    ev1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / steps

    # kernel pass: the same steps, eager, with HIP events around every
    # launch of the grouped expert kernels (on the stream they run on)
    be.profileKernels(True)
    n_prof = min(steps, 10)
    distinct = []
    for i in range(n_prof):
        normed.copy_(inputs[i % n_inputs])
        run_step(stack, normed, outs, combine, ids=ids)
        torch.cuda.synchronize()
        for li in range(L):
            distinct.append(len(np.unique(ids[li].cpu().numpy())))
    stats = be.kernelStats()
    be.profileKernels(False)
    return ms, wall / steps * 1e3, stats, distinct


def roofline_for(stats, distinct, which):
    """HBM roofline of one grouped kernel: algorithmic bytes per launch (the
    distinct experts' weight planes) / mean launch time."""
    s = stats[which]
    per_expert = 2 * GATE_BYTES if which == "gate_up" else DOWN_BYTES
    bytes_per_launch = per_expert * float(np.mean(distinct))
    avg_s = s["ms"] / s["count"] / 1e3
    achieved = bytes_per_launch / avg_s / 1e9
    return {"bound": "hbm", "kernel": s["name"], "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None, "avg_launch_us": round(avg_s * 1e6, 2),
            "bytes_per_launch": int(bytes_per_launch)}


def cpu_baseline(stack, seconds, threads):
    """Loom's CPU path (the oracle restatement of llama.moeLayer + moeRun,
    int8-activation kernels, row-parallel pool) on this host's cores, over a
    bounded sample: batch-1 tokens through the host-copied layers."""
    import oracle as o

    o.build()
    ws = [o.MoeWeights(DIM, FFN, N_EXPERT, TOP_K, h["router"], h["gate"], h["up"], h["down"],
                       Q4_K, Q4_K, Q6_K, router_bias=h["bias"]) for h in stack.host]
    rng = np.random.default_rng(5)
    n_layer_calls = 0
    with o.Pool(threads):
        x = rng.standard_normal(DIM).astype(np.float32)
        o.moe_layer_token(ws[0], x)  # warm the pool and the pages
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            x = rng.standard_normal(DIM).astype(np.float32)
            for w in ws:
                o.moe_layer_token(w, x)
                n_layer_calls += 1
        el = time.perf_counter() - t0
    per_layer = el / n_layer_calls
    return {"value": round(1.0 / (per_layer * N_LAYERS), 3), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": f"{n_layer_calls} batch-1 token x layer calls over {len(ws)} host-resident "
                      f"layers in {el:.1f} s ({per_layer * 1e3:.2f} ms/layer), scaled to "
                      f"{N_LAYERS} layers"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU expert split is design only)", file=sys.stderr)
        sys.exit(2)
    import torch

    import loom_amd
    from loom_amd import backend as be

    loom_amd.init(0)
    batches = [int(v) for v in args.batch.split(",") if v]
    host_layers = 0 if args.no_cpu else 2
    stack = Stack(args.layers, host_layers)
    res = {}
    for b in batches:
        ms, wall_ms, stats, distinct = bench_batch(stack, b, args.steps, args.warmup,
                                                   not args.no_graph)
        log(f"batch {b}: {ms:.3f} ms/step, {b * 1e3 / ms:.1f} tok/s")
        dom = max(stats, key=lambda k: stats[k]["ms"])
        res[b] = dict(ms=ms, wall_ms=wall_ms, tok_s=b * 1e3 / ms,
                      roofline=roofline_for(stats, distinct, dom),
                      other=roofline_for(stats, distinct, "down" if dom == "gate_up" else "gate_up"),
                      distinct=float(np.mean(distinct)),
                      layer_bytes=ROUTER_BYTES + float(np.mean(distinct)) * (2 * GATE_BYTES + DOWN_BYTES))
    head = batches[0]
    r = res[head]
    cores = args.cpu_threads or max(1, min(16, os.cpu_count() or 1) - 2)
    line = {
        "metric": METRIC, "value": round(r["tok_s"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"qwen3-30b-a3b-moe-stack: {args.layers} MoE layers (hidden 2048, "
                               "128 experts top-8, ffn 768, Q4_K gate/up, Q6_K down, f32 router + "
                               "Zipf(1.1) bias), no attention/head",
                   "batch": head, "layers": args.layers, "graph": not args.no_graph,
                   "parallelism": "single-gpu"},
        "roofline": r["roofline"],
        "cpu_baseline": None,
        "stack_roofline": {"bytes_per_step": int(r["layer_bytes"] * args.layers),
                           "achieved_GBs": round(r["layer_bytes"] * args.layers / (r["ms"] / 1e3) / 1e9, 1),
                           "frac": round(r["layer_bytes"] * args.layers / (r["ms"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4)},
        "secondary_kernel": r["other"],
    }
    for b in batches[1:]:
        rb = res[b]
        line[f"batch{b}"] = {"value": round(rb["tok_s"], 2), "ms_per_step": round(rb["ms"], 4),
                             "distinct_experts_per_layer": round(rb["distinct"], 2),
                             "roofline": rb["roofline"], "secondary_kernel": rb["other"],
                             "stack_GBs": round(rb["layer_bytes"] * args.layers / (rb["ms"] / 1e3) / 1e9, 1)}
    if not args.no_cpu:
        log(f"cpu baseline: {cores} threads, {args.cpu_seconds} s sample")
        line["cpu_baseline"] = cpu_baseline(stack, args.cpu_seconds, cores)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
