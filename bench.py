#!/usr/bin/env python3
"""bench.py -- decode throughput of a Qwen3-30B-A3B-shaped model on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 1,32] [--ctx 4096]
                    [--numerics both|parity|fast] [--no-cpu]

Workload (config 4, synthetic and seeded; no checkpoint): 48 layers of
GQA attention (32 query / 4 KV heads, head_dim 128, QK-norm, NEOX rope) and
the routed MoE layer (hidden 2048, 128 experts top-8, expert ffn 768, f32
router with a per-expert Zipf(1.1) logit bias), vocab 151936, Q4_K_M mix (Q4_K
with Q6_K for attn_v, ffn_down and output), all weights HBM-resident
(~21 GB), decoding against a 4096-token fp16 K/V context (seeded random rows)
per sequence.  One step = one token of every sequence of the batch through
the whole model, as one device-side frame (loomhip_token_frame_dev: embedding,
48 x (attention + MoE), head, greedy pick), replayed from a HIP graph.

Numerics: the headline runs PARITY -- every kernel in the CPU path's own
evaluation order, so the step is bit-identical to Loom's CPU path (the GPU
tests measure max-rel 0.0 at this 4096-token context); FAST (tree sums and
a split-context attention on the matrix cores) is reported beside it with
its measured error, since it misses north_star's 2e-3 at this context.

Reported: tok/s at batch 1 (``value``) and batch 32 (``batch32``), the
dominant kernel's roofline (HIP events around that kernel's launches on the
stream it runs on), the whole step's bytes against the HBM roofline, and the
CPU restatement of Loom's CPU path timed on this host's cores over a bounded
sample (two layers at the full shapes plus the head, scaled to 48 layers) at
the default thread count and at 1 thread, and at batch 32.
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

N_LAYERS, DIM, VOCAB, N_EXPERT, TOP_K = 48, 2048, 151936, 128, 8
KVD = 4 * 128
GATE_BYTES = 884_736       # one expert's Q4_K [768][2048] plane
DOWN_BYTES = 1_290_240     # one expert's Q6_K [2048][768] plane
ROUTER_BYTES = N_EXPERT * DIM * 4
ATTN_W_BYTES = 4_718_592 + 589_824 + 860_160 + 4_718_592  # wq, wk (Q4_K), wv (Q6_K), wo (Q4_K)
HEAD_BYTES = 151936 * 8 * 210  # Q6_K [151936][2048]
# Latency of a dependent f32 add on gfx950 (in-kernel clock64 over a chain of
# register adds; clock64 against wall_clock64 gave the 2.4 GHz engine clock),
# and the cycles per position measured for the same chain when each addend
# arrives from LDS (a ds_read_b128 per four adds: the read's return into the
# wave's registers costs as much issue time as the adds).
ADD_LATENCY_CYCLES = 4.7
LDS_FED_CYCLES = 8.4
CLOCK_HZ = 2.4e9
# MI355X dense matrix-core peaks (no sparsity) and one v_mfma_i32_16x16x64_i8
# (16 x 16 outputs, 64 deep, a multiply and an add each)
PEAK_BF16_OPS, PEAK_INT8_OPS = 2.5e15, 5.0e15
MFMA_I8_OPS = 2 * 16 * 16 * 64
FFN = 768
# The grouped expert launches at 16+ tokens and the kernels that serve them
# (config 4: Q4_K gate/up over 2048 columns, Q6_K down over 768)
MOE_GEMM_KERNELS = {"gate_up": "lh::mmqs_kernel<true, 8>", "down": "lh::mmq_kernel<14, 1, false, 1>"}
# Largest per-step logit max-rel of FAST numerics against the CPU path at the
# 4096-token context (32 lanes), measured by the GPU parity test named in the
# output line.
FAST_MEASURED_MAXREL = 1.74e-2


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--batch", default="1,32")
    ap.add_argument("--ctx", type=int, default=4096, help="prefilled K/V context per sequence")
    ap.add_argument("--layers", type=int, default=N_LAYERS)
    ap.add_argument("--numerics", default="both", choices=["both", "parity", "fast"],
                    help="both: PARITY (bit-identical to the CPU path) as the headline, FAST beside it")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0 = the reference's default, host cores - 2 (capped at the box's share)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-cache", action="store_true", help="skip the config-5 expert-cache streaming run")
    ap.add_argument("--cache-steps", type=int, default=1024, help="config-5 decode steps at batch 1 and at 64")
    ap.add_argument("--sweep", action="store_true",
                    help="config 2 instead: the dequant-fused matvec alone, GB/s per type x shape x vectors")
    ap.add_argument("--moe-layer", action="store_true",
                    help="config 3 instead: one MoE layer at token batches 1, 8, 32 and 128")
    ap.add_argument("--mla", action="store_true",
                    help="config 5's MLA attention alone: 61 layers at contexts 1024, 2048, 4096")
    ap.add_argument("--mla-ctx", default="1024,2048,4096", help="contexts of the --mla run")
    ap.add_argument("--sweep-rounds", type=int, default=5, help="rounds over each weight ring in --sweep")
    ap.add_argument("--no-mla", action="store_true", help="skip the MLA attention run of the default bench")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="first copy MB megabytes device to device three times: the known-size kernel that "
                         "scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes")
    return ap.parse_args()


def bench_batch(dm, b, args):
    """Time args.steps decode steps of b sequences; returns a result dict."""
    import torch

    import loom_amd
    from loom_amd import backend as be
    from loom_amd.frame import Decoder

    dec = Decoder(dm, b)
    dec.prefill_random(args.ctx, seed=7 + b, scale=0.5)
    g = torch.Generator(device="cpu").manual_seed(11 + b)
    dec.tokens.copy_(torch.randint(0, dm.spec.vocab, (b,), generator=g, dtype=torch.int32))
    for _ in range(max(1, args.warmup)):  # eager: sizes the workspaces before any capture
        dec.step()
    torch.cuda.synchronize()
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            dec.step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
    dec.pos.fill_(args.ctx)  # every timed step attends to ~ctx positions
    st = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(st)
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            dec.step()
    ev1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps

    # kernel pass: eager steps with HIP events around the tagged launches and
    # the routed ids recorded for the distinct-expert count.  A spin kernel
    # ahead of each step holds the stream while the host enqueues the step,
    # so the events time the kernels back to back, as the graph runs them,
    # not the host's launch rate.
    ids = torch.zeros((dm.spec.n_layers, b, TOP_K), dtype=torch.int32, device="cuda")
    dm.desc.ids_out = ids.data_ptr()
    dec.pos.fill_(args.ctx)
    be.profileKernels(True)
    distinct, groups, sets8 = [], [], []
    prof_steps = min(args.steps, 6)
    for _ in range(prof_steps):
        torch.cuda._sleep(50_000_000)
        dec.step()
        torch.cuda.synchronize()
        h = ids.cpu().numpy()
        distinct += [len(np.unique(h[li])) for li in range(dm.spec.n_layers)]
        for li in range(dm.spec.n_layers):  # the expert groups of <= 16 tokens the grouped launches run
            counts = np.bincount(h[li].ravel(), minlength=N_EXPERT)
            sizes = [min(16, c - g) for c in counts if c > 0 for g in range(0, int(c), 16)]
            groups.append(len(sizes))
            sets8.append(sum((n + 7) // 8 for n in sizes))
    stats = be.kernelStats()
    be.profileKernels(False)
    dm.desc.ids_out = None
    del dec, graph
    torch.cuda.empty_cache()
    return dict(ms=ms, wall_ms=wall / args.steps * 1e3, tok_s=b * 1e3 / ms, stats=stats,
                distinct=float(np.mean(distinct)), groups=float(np.mean(groups)), sets8=float(np.mean(sets8)),
                prof_steps=prof_steps)


N_HEADS, HD = 32, 128
WQKV_BYTES = 4_718_592 + 589_824 + 860_160  # wq, wk (Q4_K), wv (Q6_K)
WO_BYTES = 4_718_592


def per_launch_bytes(name, b, ctx, distinct):
    """Algorithmic HBM bytes of one launch of the tagged kernel: every weight,
    K/V row and f32 score / p value the launch must read or write once."""
    P = ctx + 1  # positions attended at a step past a ctx-token context
    if name == "gate_up":
        return distinct * 2 * GATE_BYTES
    if name == "down":
        return distinct * DOWN_BYTES
    if name == "attn":  # FAST split-context attention: K and V rows, fp16
        return b * P * KVD * 2 * 2
    if name == "attn_scores":  # keys (fp16) in, f32 scores out
        return b * P * KVD * 2 + b * N_HEADS * P * 4
    if name == "attn_softmax":  # scores in, p out
        return b * N_HEADS * P * 4 * 2
    if name == "attn_pv":  # values (fp16) and p in (up to 4 lanes: the scores in, the softmax inside)
        return b * P * KVD * 2 + b * N_HEADS * P * 4
    if name == "head":
        return HEAD_BYTES
    if name == "qkv":
        return WQKV_BYTES
    if name == "wo":
        return WO_BYTES
    return 0


# VALU issue ceiling: one wave64 f32 instruction per 4.75 cycles per SIMD
# (measured on this chip with independent add chains), 1024 SIMDs at 2.4 GHz.
VALU_LANE_OPS = 1024 * 64 / 4.75 * 2.4e9


def measured_traffic(b, tag):
    """HBM bytes per launch of a tagged kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_per_launch.json")
    try:
        with open(path) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return None
    return doc.get(f"batch{b}", {}).get(tag)


def rocprof_us(tag, b):
    """The tagged kernel's mean duration at b lanes from the committed
    rocprofv3 trace summary of this same benchmark (profiles/
    kernel_durations.json), for the per-lane kernels whose grid z is the lane
    count; None where the table has no entry."""
    names = {"attn_pv": "lh::attn_pv_split_kernel<128, true>" if b <= 4 else "lh::attn_pv_many_kernel<128, 8>",
             "attn_softmax": "lh::attn_softmax_kernel<512>",
             "attn_scores": "lh::attn_scores_kernel<128>" if b <= 4 else "lh::attn_scores_many_kernel<128>",
             "attn": "lh::attn_partial_kernel<128>" if b <= 4 else "lh::attn_direct_kernel<128, 128>"}
    try:
        with open(os.path.join(ROOT, "profiles", "kernel_durations.json")) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return None
    return doc.get(names.get(tag, ""), {}).get(f"n{b}")


def roofline(r, b, ctx, layers):
    """The dominant kernel (one launch site, one kernel family) by total
    event time: its algorithmic bytes per launch / its mean event-timed
    launch duration, against the HBM peak.  The exact attention's P.V is
    bound by the VALU (one multiply and one dependent add per position and
    column, in order), so its VALU rate against the issue ceiling is given
    beside the HBM figure."""
    stats = r["stats"]
    dom = max(stats, key=lambda k: stats[k]["ms"])
    s = stats[dom]
    avg_s = s["ms"] / s["count"] / 1e3
    byts = per_launch_bytes(dom, b, ctx, r["distinct"])
    achieved = byts / avg_s / 1e9
    per_kernel = {k: {"avg_us": round(v["ms"] / v["count"] * 1e3, 2), "launches": v["count"],
                      "GBs": round(per_launch_bytes(k, b, ctx, r["distinct"]) / (v["ms"] / v["count"] / 1e3) / 1e9, 1)}
                  for k, v in stats.items()}
    roof = {"bound": "hbm", "kernel": s["name"], "tag": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(b, dom),
            "avg_launch_us": round(avg_s * 1e6, 2), "bytes_per_launch": int(byts)}
    prof = rocprof_us(dom, b)
    if prof:  # the same figure from the committed rocprofv3 summary (events include the dispatch gap)
        roof["rocprof_avg_us"] = prof
        roof["frac_rocprof"] = round(byts / (prof / 1e6) / 1e9 / HBM_PEAK_GBS, 4)
    if dom == "attn_pv":
        ops = 2.0 * b * N_HEADS * HD * (ctx + 1)  # multiply + add per (head, column, position)
        roof["valu"] = {"lane_ops_per_launch": int(ops), "achieved_Tops": round(ops / avg_s / 1e12, 2),
                        "issue_ceiling_Tops": round(VALU_LANE_OPS / 1e12, 1),
                        "frac": round(ops / avg_s / VALU_LANE_OPS, 4)}
        if prof:
            roof["valu"]["frac_rocprof"] = round(ops / (prof / 1e6) / VALU_LANE_OPS, 4)
        # every output column is one chain of ctx + 1 dependent f32 adds in
        # position order: its latency floors the launch whatever the bytes
        # (lds_fed_floor_us: the same chain at the cycles per position
        # measured when the addends come through LDS, as they do here)
        floor_s = (ctx + 1) * ADD_LATENCY_CYCLES / CLOCK_HZ
        roof["chain"] = {"adds_in_order": ctx + 1, "add_latency_cycles": ADD_LATENCY_CYCLES,
                         "clock_GHz": CLOCK_HZ / 1e9, "floor_us": round(floor_s * 1e6, 2),
                         "lds_fed_floor_us": round((ctx + 1) * LDS_FED_CYCLES / CLOCK_HZ * 1e6, 2),
                         "frac": round(floor_s / avg_s, 4)}
        if prof:
            roof["chain"]["frac_rocprof"] = round(floor_s / (prof / 1e6), 4)
    return roof, per_kernel


def mfma_issued_measured(kernel):
    """int8 MFMA ops per launch of a kernel as the committed rocprofv3 PMC
    summary counted them (SQ_INSTS_VALU_MFMA_MOPS_I8 x 512), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "mfma_per_launch.json")) as f:
            return json.load(f).get(kernel)
    except (OSError, ValueError):
        return None


def moe_gemm(r, b, ctx):
    """The grouped expert matmuls of one MoE layer at b tokens on the int8
    matrix cores: useful ops (a multiply and an add per weight per routed
    token: 2 x pairs x rows x cols per matrix) per event-timed launch, against
    the bf16 and int8 dense peaks and against the attainable min(int8 peak,
    AI x HBM peak), AI = useful ops / the launch's algorithmic bytes.  Issued
    = the MFMAs the kernels run for this layer's groups (experts' tokens in
    groups of up to 16): gate/up per (group, 16-row tile, super-block) one
    set of 8 MFMAs per matrix per 8 tokens (4 dot + 4 mins, A rows = (token,
    group)), down 16 per (group, 16-row tile, super-block) (one per 16-value
    run); beside it the count rocprofv3 measured, and the same rates over
    the committed rocprof duration."""
    pairs = b * TOP_K
    out = {}
    for tag, kern in MOE_GEMM_KERNELS.items():
        s = r["stats"].get(tag)
        if not s:
            continue
        avg_s = s["ms"] / s["count"] / 1e3
        useful = (2 if tag == "gate_up" else 1) * 2 * pairs * FFN * DIM
        if tag == "gate_up":
            issued = r["sets8"] * 2 * 8 * (FFN // 16) * (DIM // 256) * MFMA_I8_OPS
        else:
            issued = r["groups"] * 16 * (DIM // 16) * (FFN // 256) * MFMA_I8_OPS
        byts = per_launch_bytes(tag, b, ctx, r["distinct"])
        ai = useful / byts
        attain = min(PEAK_INT8_OPS, ai * HBM_PEAK_GBS * 1e9)
        ach = useful / avg_s
        e = {"kernel": kern, "useful_ops": int(useful), "issued_ops_est": int(issued),
             "issued_over_useful": round(issued / useful, 2), "bytes": int(byts), "ai_ops_per_byte": round(ai, 1),
             "avg_launch_us": round(avg_s * 1e6, 2), "achieved_Tops": round(ach / 1e12, 1),
             "frac_bf16_peak": round(ach / PEAK_BF16_OPS, 4), "frac_int8_peak": round(ach / PEAK_INT8_OPS, 4),
             "attainable_Tops": round(attain / 1e12, 1), "frac_attainable": round(ach / attain, 4),
             "hbm_GBs": round(byts / avg_s / 1e9, 1)}
        meas = mfma_issued_measured(kern)
        if meas:
            e["issued_ops_rocprof"] = meas
        try:
            with open(os.path.join(ROOT, "profiles", "kernel_durations.json")) as f:
                prof = json.load(f).get(kern, {}).get("n1")
        except (OSError, ValueError):
            prof = None
        if prof:
            achp = useful / (prof / 1e6)
            e.update({"rocprof_avg_us": prof, "achieved_Tops_rocprof": round(achp / 1e12, 1),
                      "frac_attainable_rocprof": round(achp / attain, 4),
                      "frac_int8_peak_rocprof": round(achp / PEAK_INT8_OPS, 4)})
        out[tag] = e
    return out


def step_bytes(b, ctx, distinct, layers):
    """Algorithmic bytes of one decode step: every dense weight once, the
    distinct experts of each layer once, the head, and each sequence's K/V."""
    per_layer = ATTN_W_BYTES + ROUTER_BYTES + distinct * (2 * GATE_BYTES + DOWN_BYTES)
    return layers * per_layer + HEAD_BYTES + b * layers * (ctx + 1) * KVD * 2 * 2


def cpu_baseline(seconds, threads, ctx):
    """Loom's CPU path -- the oracle's restatement of llama.step (batch 1) and
    decodeBatch (batch 32): int8-activation kernels, the row-parallel pool --
    on this host's cores, over a bounded sample: a two-layer model at the
    config-4 shapes with the full 151936-row head against a ctx-token fp16
    context.  Per token (per step at batch 32) = head + 24 x (two layers),
    the two layers' time being the step's time less the head's.  Timed at
    the reference's default thread count (cores - 2) and at 1 thread (batch
    1), and at the default count for batch 32."""
    import torch

    import oracle as o
    from loom_amd.frame import DeviceModel, qwen3_30b_a3b
    from oracle.model import OracleModel

    o.build()
    spec = qwen3_30b_a3b(ctx_len=ctx + 64, n_layers=2)
    dm = DeviceModel.synth(spec, seed=99, keep_ggml=True)
    om = OracleModel(o, dm)
    del dm
    torch.cuda.empty_cache()
    rng = np.random.default_rng(3)
    x = rng.standard_normal(DIM).astype(np.float32)

    def seqs_at(n):
        seqs, bufs = om.new_seqs(n)
        for buf in bufs:  # a prefilled fp16 context: random rows in [-1, 1)
            buf[:] = (rng.random(buf.size // 2, dtype=np.float32) * 2 - 1).astype(np.float16).view(np.uint8)
        for i in range(n):
            seqs[i].pos = ctx
        return seqs

    def timed(fn, budget):
        fn()  # warm the pool and the pages
        t0 = time.perf_counter()
        k = 0
        while k == 0 or time.perf_counter() - t0 < budget:
            fn()
            k += 1
        return (time.perf_counter() - t0) / k, k

    def b1(seq):
        om.step(seq, int(rng.integers(0, spec.vocab)))
        seq.pos = ctx

    def head(n):
        for _ in range(n):
            o.matvec(spec.output_t, om.host["output"], x, spec.vocab, DIM)

    out = {}
    for nthr, budget in ((threads, seconds * 0.4), (1, seconds * 0.3)):
        s1 = seqs_at(1)
        with o.Pool(nthr):
            t2, n_tok = timed(lambda: b1(s1[0]), budget)
            th, n_head = timed(lambda: head(1), max(1.0, budget / 5))
        out[nthr] = (th + (N_LAYERS / 2) * (t2 - th), t2, th, n_tok)
    s32 = seqs_at(32)
    toks = rng.integers(0, spec.vocab, 32)

    def b32():
        om.decode_batch(s32, toks)
        for i in range(32):
            s32[i].pos = ctx

    with o.Pool(threads):
        t32, n32 = timed(b32, seconds * 0.3)
        th32, _ = timed(lambda: head(32), 1.0)
    step32 = th32 + (N_LAYERS / 2) * (t32 - th32)
    per_token, t2, th, n_tok = out[threads]
    per_token1, t21, th1, n_tok1 = out[1]
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n_tok} tokens of a 2-layer model at the config-4 shapes with the full 151936-row head "
                      f"against a {ctx}-token fp16 context ({t2 * 1e3:.1f} ms/token, head {th * 1e3:.1f} ms), "
                      f"scaled to {N_LAYERS} layers as head + 24 x (step - head)",
            "one_thread": {"value": round(1.0 / per_token1, 4), "unit": "tok/s", "cores": 1,
                           "sample": f"{n_tok1} tokens, {t21 * 1e3:.1f} ms/token, head {th1 * 1e3:.1f} ms"},
            "batch32": {"value": round(32.0 / step32, 4), "unit": "tok/s", "cores": threads,
                        "sample": f"{n32} decodeBatch steps of 32 sequences of the same 2-layer model "
                                  f"({t32 * 1e3:.0f} ms/step, 32 head matvecs {th32 * 1e3:.0f} ms), scaled to "
                                  f"{N_LAYERS} layers"}}


SWEEP_TYPES = (("Q4_0", 2), ("Q8_0", 8), ("Q4_K", 12), ("Q6_K", 14))
SWEEP_SHAPES = ((2048, 2048), (4096, 4096), (768, 2048))  # rows (out) x cols (in)
SWEEP_N = (1, 4, 16)
RING_BYTES = 1 << 30  # distinct weight copies per (type, shape): 4x the 256 MB MALL


def bench_sweep(args):
    """Config 2: the dequant-fused matvec alone.  Per (type, shape) a ring of
    >= 1 GB of distinct weight copies is rotated launch by launch; HIP events
    around each matvec launch (the library's tagged timing) give its mean time
    in each of 5 rounds, the median round is reported; GB/s = weight bytes /
    time.  The CPU leg times the oracle's matvec on the host cores at n = 1."""
    import torch

    from loom_amd import backend as be
    from loom_amd import plane_bytes

    rows_out = []
    for tname, t in SWEEP_TYPES:
        for rows, cols in SWEEP_SHAPES:
            pb = plane_bytes(t, rows, cols)
            copies = max(4, -(-RING_BYTES // pb))
            w = be.repack_dev(t, be.synth_ggml_dev(t, rows, cols, copies, 17 + t, 0.02), rows, cols, copies)
            for n in SWEEP_N:
                x = torch.randn(n, cols, device="cuda")
                out = torch.empty(n, rows, device="cuda")
                planes = [w[i * pb:(i + 1) * pb] for i in range(copies)]
                for pl in planes:  # warm: every copy once
                    be.matvec_dev(t, out, pl, x, n, rows, cols)
                torch.cuda.synchronize()
                rounds = []
                for _ in range(max(1, args.sweep_rounds)):
                    be.profileKernels(True)
                    for pl in planes:
                        be.matvec_dev(t, out, pl, x, n, rows, cols)
                    torch.cuda.synchronize()
                    st = be.kernelStats()["dense"]
                    be.profileKernels(False)
                    rounds.append(st["ms"] / st["count"])
                ms = float(np.median(rounds))
                rows_out.append({"type": tname, "rows": rows, "cols": cols, "n": n, "weight_bytes": pb,
                                 "us": round(ms * 1e3, 2), "GBs": round(pb / (ms / 1e3) / 1e9, 1),
                                 "frac": round(pb / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4), "ring_copies": copies})
                log(f"sweep {tname} {rows}x{cols} n={n}: {ms * 1e3:.2f} us, {rows_out[-1]['GBs']} GB/s")
            del w, planes
            torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        cpu = sweep_cpu(args)
    return {"metric": "dequant-fused matvec GB/s of weight bytes (config 2)", "unit": "GB/s", "n_gpus": 1,
            "peak_GBs": HBM_PEAK_GBS, "data": "synthetic", "dtype": "int8",
            "config": {"workload": "config 2: weights N(0, 0.02) quantized with the GGUF rule, x ~ N(0, 1), "
                                   "each (type, shape) a ring of >= 1 GB of distinct copies rotated per launch"},
            "results": rows_out, "cpu_baseline": cpu}


def sweep_cpu(args):
    """The oracle's matvec (the reference's int8-activation kernels) on the
    host cores at n = 1 for the 4096 x 4096 shape of each type."""
    import oracle as o
    from loom_amd import ggml_bytes

    o.build()
    threads = args.cpu_threads or max(1, min(16, (os.cpu_count() or 2) - 2))
    rng = np.random.default_rng(5)
    out = []
    with o.Pool(threads):
        for tname, t in SWEEP_TYPES:
            rows, cols = 4096, 4096
            nbytes = ggml_bytes(t, rows, cols)
            w = o.quantize(t, o.normal(rows * cols, 91 + t, 0.0, 0.02).reshape(rows, cols))
            x = rng.standard_normal(cols).astype(np.float32)
            o.matvec(t, w, x, rows, cols)
            t0 = time.perf_counter()
            k = 0
            while time.perf_counter() - t0 < max(0.5, args.cpu_seconds / 8):
                o.matvec(t, w, x, rows, cols)
                k += 1
            sec = (time.perf_counter() - t0) / k
            out.append({"type": tname, "rows": rows, "cols": cols, "n": 1, "ms": round(sec * 1e3, 3),
                        "GBs": round(nbytes / sec / 1e9, 2)})
    return {"unit": "GB/s", "cores": threads, "kind": "port", "results": out,
            "sample": "the oracle's matvec, 4096 x 4096 per type at n = 1"}


def bench_moe_layer(args):
    """Config 3: one MoE layer (hidden 2048, 128 experts top-8, ffn 768, Q4_K
    gate/up, Q6_K down, f32 router N(0, 1/sqrt(2048)) with a Zipf(1.1) logit
    bias) at token batches 1, 8, 32, 128; 3 distinct layer copies (~1.2 GB)
    rotated per call.  Bytes = distinct experts x 3,059,712 + the router."""
    import torch

    from loom_amd import COMBINE_EXPERT_ASC, COMBINE_SELECTION, Q4_K, Q6_K
    from loom_amd import backend as be

    E, D, F, K = N_EXPERT, DIM, 768, TOP_K
    layers = []
    for c in range(3):
        gate = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, F, D, E, 300 + 10 * c, 0.02), F, D, E)
        up = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, F, D, E, 301 + 10 * c, 0.02), F, D, E)
        down = be.repack_dev(Q6_K, be.synth_ggml_dev(Q6_K, D, F, E, 302 + 10 * c, 0.02), D, F, E)
        g = torch.Generator(device="cuda").manual_seed(400 + c)
        router = (torch.randn(E, D, generator=g, device="cuda") / np.sqrt(D)).contiguous()
        ranks = torch.randperm(E, generator=g, device="cuda").float() + 1
        z = -1.1 * torch.log(ranks)
        bias = (z - z.mean()).contiguous()
        layers.append((be.MoeLayer(D, F, E, K, router, gate, up, down, Q4_K, Q4_K, Q6_K, router_bias=bias),
                       (gate, up, down, router, bias)))
    res = []
    for b in (1, 8, 32, 128):
        g = torch.Generator(device="cuda").manual_seed(b)
        xs = [torch.randn(b, D, generator=g, device="cuda") for _ in range(3)]
        out = torch.zeros(b, D, device="cuda")
        ids = torch.zeros(b, K, dtype=torch.int32, device="cuda")
        comb = COMBINE_SELECTION if b == 1 else COMBINE_EXPERT_ASC
        for i in range(6):
            layers[i % 3][0](xs[i % 3], out, comb)
        torch.cuda.synchronize()
        n_calls = max(30, args.steps)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for i in range(n_calls):
            layers[i % 3][0](xs[i % 3], out, comb)
        ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / n_calls
        distinct = []
        for c in range(3):
            layers[c][0](xs[c], out, comb, ids=ids)
            torch.cuda.synchronize()
            distinct.append(len(np.unique(ids.cpu().numpy())))
        dist = float(np.mean(distinct))
        byts = dist * (2 * GATE_BYTES + DOWN_BYTES) + ROUTER_BYTES
        gbs = byts / (ms / 1e3) / 1e9
        flops = b * K * 9_437_184 + b * 524_288
        res.append({"batch": b, "us_per_layer": round(ms * 1e3, 2), "tok_s": round(b / (ms / 1e3), 1),
                    "distinct_experts": round(dist, 1), "bytes": int(byts), "GBs": round(gbs, 1),
                    "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "flops": flops,
                    "TFLOPs": round(flops / (ms / 1e3) / 1e12, 2),
                    "path": "decode kernels" if b <= 4 else "grouped matrix-core matmul" if b >= 16 else
                            "grouped matvec"})
        log(f"moe layer batch {b}: {ms * 1e3:.2f} us, {dist:.1f} distinct experts, {gbs:.0f} GB/s")
    return {"metric": "one MoE layer: us per layer and GB/s of distinct expert bytes (config 3)", "n_gpus": 1,
            "peak_GBs": HBM_PEAK_GBS, "data": "synthetic", "dtype": "int8",
            "config": {"workload": "config 3: hidden 2048, 128 experts top-8, ffn 768, Q4_K gate/up, Q6_K "
                                   "down, f32 router with a Zipf(1.1) logit bias; 3 layer copies rotated"},
            "results": res}


# Config 5's attention: DeepSeek-V3 MLA, 128 heads, q/k nope 128, rope 64,
# kv_lora 512, v 128, Q4_K kv_b, 61 layers.
MLA_LAYERS, MLA_H, MLA_NOPE, MLA_ROPE, MLA_KVR, MLA_VD = 61, 128, 128, 64, 512, 128


def mla_launch_bytes(tag, S):
    """Algorithmic bytes of one launch of an MLA kernel at context S: what it
    must read and write once (W_k / W_v as Q4_K planes, the f32 latent and
    rope rows, q, the score rows)."""
    H, nope, rope, kvr, vd = MLA_H, MLA_NOPE, MLA_ROPE, MLA_KVR, MLA_VD
    q4k = lambda rows: rows * kvr // 256 * 144  # noqa: E731
    return {"mla_absorb": q4k(H * nope) + H * nope * 4 + H * kvr * 4,
            "mla_scores": S * (kvr + rope) * 4 + H * (kvr + rope) * 4 + H * S * 4,
            "mla_softmax": 2 * H * S * 4,
            "mla_wsum": S * kvr * 4 + H * S * 4 + H * kvr * 4,
            "mla_wv": q4k(H * vd) + H * kvr * 4 + H * vd * 4}[tag]


def mla_launch_ops(tag, S):
    """VALU lane-ops of the ordered f32 work (one multiply and one add per
    term): the scores' dot products, the weighted sum, the absorb."""
    H = MLA_H
    return {"mla_scores": 2 * H * S * (MLA_KVR + MLA_ROPE), "mla_wsum": 2 * H * S * MLA_KVR,
            "mla_absorb": 2 * H * MLA_NOPE * MLA_KVR}.get(tag)


def bench_mla_layer(args, S, scale, attn_layers):
    """Config 5's whole block at context S, batch 1: loomhip_mla_layer_tail_dev
    = MLA attention, the Q4_K output projection [7168][16384] and residual,
    the exact FFN norm, the routed MoE (256 HBM-resident Q4_K experts of
    24,772,608 B, sigmoid top-8 with renorm, Zipf(1.1) logit bias) plus the
    shared expert and the residual.  Three distinct layers rotated, each with
    its own experts (6.4 GB a layer); one step = the three layers, replayed
    from a HIP graph."""
    import torch

    from loom_amd import GATING_SIGMOID, Q4_K
    from loom_amd import backend as be

    H, vd, D, F, E, K = MLA_H, MLA_VD, C5_DIM, C5_FFN, C5_E, C5_K
    g = torch.Generator(device="cuda").manual_seed(71)
    built = []
    for i, (m, c, r) in enumerate(attn_layers):
        wo = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, D, H * vd, 1, 900 + i, 0.02), D, H * vd, 1)
        ex = [be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, rows, cols, E, 910 + 10 * i + k, 0.02), rows, cols, E)
              for k, (rows, cols) in enumerate(((F, D), (F, D), (D, F)))]
        sh = [be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, rows, cols, 1, 950 + 10 * i + k, 0.02), rows, cols, 1)
              for k, (rows, cols) in enumerate(((C5_SFFN, D), (C5_SFFN, D), (D, C5_SFFN)))]
        router = (torch.randn(E, D, generator=g, device="cuda") / np.sqrt(D)).contiguous()
        ranks = torch.randperm(E, generator=g, device="cuda").float() + 1
        z = -1.1 * torch.log(ranks)
        bias = (z - z.mean()).contiguous()
        moe = be.MoeLayer(D, F, E, K, router, ex[0], ex[1], ex[2], Q4_K, Q4_K, Q4_K, router_bias=bias,
                          gating=GATING_SIGMOID, weights_norm=True, weights_scale=2.5,
                          shexp=(sh[0], sh[1], sh[2], Q4_K, Q4_K, Q4_K, C5_SFFN))
        norm = (1.0 + 0.05 * torch.randn(D, generator=g, device="cuda")).contiguous()
        built.append((m, c, r, wo, norm, moe))
    qn = torch.randn(H * MLA_NOPE, generator=g, device="cuda")
    qr = torch.randn(H * MLA_ROPE, generator=g, device="cuda")
    x = torch.randn(D, generator=g, device="cuda")
    x0 = x.clone()

    def step():
        for m, c, r, wo, norm, moe in built:
            if m.tail(c, r, S, qn, qr, Q4_K, wo, norm, 1e-6, moe, x) != 0:
                from loom_amd import last_error
                raise RuntimeError(f"mla_layer_tail_dev declined: {last_error()}")
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    n = max(5, min(args.steps, 20))
    x.copy_(x0)
    graph.replay()
    st = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(st)
    for _ in range(n):
        x.copy_(x0)  # keep the residual stream at its scale
        graph.replay()
    ev1.record(st)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / n
    per_layer_us = ms * 1e3 / len(built)
    moe_bytes = K * C5_EXPERT_BYTES + 3 * plane_bytes_q4k(C5_SFFN, D) + E * D * 4
    byts = mla_launch_bytes("mla_absorb", S) + mla_launch_bytes("mla_scores", S) + \
        mla_launch_bytes("mla_wsum", S) + mla_launch_bytes("mla_wv", S) + plane_bytes_q4k(D, H * vd) + moe_bytes
    log(f"mla layer (attention + projection + norm + routed MoE + shared expert) ctx {S}: {per_layer_us:.1f} us "
        f"per layer")
    del graph, built
    torch.cuda.empty_cache()
    return {"us_per_layer": round(per_layer_us, 2), "ctx": S, "layers_rotated": len(attn_layers),
            "bytes_per_layer": int(byts), "GBs": round(byts / (per_layer_us / 1e6) / 1e9, 1),
            "entry_point": "loomhip_mla_layer_tail_dev",
            "workload": "config 5 block: MLA attention (128 heads, kv_lora 512, rope 64) + Q4_K wo [7168][16384] "
                        "+ exact rmsnorm + 256 resident Q4_K experts top-8 (sigmoid, renorm, scale 2.5, Zipf(1.1) "
                        "logit bias) + shared expert (ffn 2048)"}


def plane_bytes_q4k(rows, cols):
    return rows * cols // 256 * 144


C5_EXPERT_BYTES = 24_772_608


def bench_mla(args, seqs, cpu=True, tail=True):
    """Config 5's MLA attention (loomhip_mla_attn_dev) over 61 layers, each
    with its own Q4_K kv_b (9.4 MB) and its own f32 latent cache (2,304 B per
    position), replayed from a HIP graph: one step = one token's attention in
    every layer at context S (batch 1).  Per-kernel HIP-event times come from
    an eager pass; the CPU column times the oracle's host head loop on one
    layer."""
    import torch

    from loom_amd import Q4_K
    from loom_amd import backend as be

    H, nope, rope, kvr, vd, L = MLA_H, MLA_NOPE, MLA_ROPE, MLA_KVR, MLA_VD, MLA_LAYERS
    scale = float(1.0 / np.sqrt(nope + rope))
    smax = max(seqs)
    g = torch.Generator(device="cuda").manual_seed(61)
    layers = []
    for li in range(L):
        kvb = be.synth_ggml_dev(Q4_K, H * (nope + vd), kvr, 1, 500 + li, float(1 / np.sqrt(kvr)))
        layers.append((be.MlaAttn(Q4_K, kvb, H, nope, vd, kvr, rope, scale),
                       torch.randn(smax, kvr, generator=g, device="cuda"),
                       torch.randn(smax, rope, generator=g, device="cuda")))
        del kvb
    qn = torch.randn(H * nope, generator=g, device="cuda")
    qr = torch.randn(H * rope, generator=g, device="cuda")
    out = torch.empty(H * vd, device="cuda")
    res = []
    for S in seqs:
        def step():
            for m, c, r in layers:
                m(c, r, S, qn, qr, out)
        step()  # sizes the workspace before the capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(2):
            graph.replay()
        st = torch.cuda.current_stream()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = max(5, min(args.steps, 20))
        torch.cuda.synchronize()
        ev0.record(st)
        for _ in range(n):
            graph.replay()
        ev1.record(st)
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / n
        del graph
        be.profileKernels(True)
        for _ in range(2):
            torch.cuda._sleep(50_000_000)
            step()
            torch.cuda.synchronize()
        stats = be.kernelStats()
        be.profileKernels(False)
        kern = {}
        for k, v in stats.items():
            avg_s = v["ms"] / v["count"] / 1e3
            e = {"avg_us": round(avg_s * 1e6, 2), "launches": v["count"],
                 "GBs": round(mla_launch_bytes(k, S) / avg_s / 1e9, 1)}
            ops = mla_launch_ops(k, S)
            if ops:
                e["valu_Tops"] = round(ops / avg_s / 1e12, 2)
                e["valu_frac"] = round(ops / avg_s / VALU_LANE_OPS, 4)
            kern[k] = e
        dom = max(stats, key=lambda k: stats[k]["ms"])
        avg_s = stats[dom]["ms"] / stats[dom]["count"] / 1e3
        ops = mla_launch_ops(dom, S)
        roof = {"bound": "valu", "kernel": stats[dom]["name"], "tag": dom, "avg_launch_us": round(avg_s * 1e6, 2)}
        if ops:
            roof.update({"achieved": round(ops / avg_s / 1e12, 2), "peak": round(VALU_LANE_OPS / 1e12, 1),
                         "unit": "T lane-ops/s (f32 multiply, add: the order the reference fixes)",
                         "frac": round(ops / avg_s / VALU_LANE_OPS, 4), "lane_ops_per_launch": int(ops)})
        if dom == "mla_wsum":
            floor_s = S * ADD_LATENCY_CYCLES / CLOCK_HZ
            roof["chain"] = {"adds_in_order": S, "floor_us": round(floor_s * 1e6, 2), "frac": round(floor_s / avg_s, 4)}
        r = {"ctx": S, "us_per_layer": round(ms * 1e3 / L, 2), "ms_per_token": round(ms, 3),
             "layers_per_s": round(L / (ms / 1e3), 1), "kernels": kern, "roofline": roof}
        log(f"mla ctx {S}: {ms * 1e3 / L:.2f} us per layer ({ms:.3f} ms per token over {L} layers), kernels {kern}")
        res.append(r)
    if tail:
        res[-1]["layer"] = bench_mla_layer(args, smax, scale, layers[:3])
    if cpu:
        import oracle
        from loom_amd import Q4_K as T

        rng = np.random.default_rng(5)
        S = smax
        w = (rng.standard_normal((H * (nope + vd), kvr)) / np.sqrt(kvr)).astype(np.float32)
        kvb_h = oracle.quantize(T, w)
        c_h = rng.standard_normal((S, kvr)).astype(np.float32)
        r_h = rng.standard_normal((S, rope)).astype(np.float32)
        qn_h = rng.standard_normal(H * nope).astype(np.float32)
        qr_h = rng.standard_normal(H * rope).astype(np.float32)
        t0 = time.perf_counter()
        oracle.mla_attn_heads(c_h, r_h, S, qn_h, qr_h, T, kvb_h, H, nope, vd, scale)
        dt = time.perf_counter() - t0
        res[-1]["cpu_baseline"] = {"value": round(dt * 1e6, 1), "unit": "us per layer", "cores": 1, "kind": "port",
                                   "sample": f"the oracle's host head loop (deepseek.zig:988-1047) on one layer "
                                             f"at context {S}"}
        log(f"mla cpu: {dt * 1e3:.1f} ms per layer at context {S}")
    del layers
    torch.cuda.empty_cache()
    return {"workload": f"config 5 attention: DeepSeek-V3 MLA over {L} layers, {H} heads, nope {nope}, rope {rope}, "
                        f"kv_lora {kvr}, v {vd}, Q4_K kv_b, f32 latent cache, batch 1, seeded random weights and "
                        "cache rows, HIP graph", "numerics": "the reference's order (bit-identical to the CPU path)",
            "results": res}


C5_DIM, C5_FFN, C5_E, C5_K, C5_SLOTS, C5_SFFN = 7168, 2048, 256, 8, 64, 2048


def _c5_layer():
    """Config 5's routed block: 256 experts of Q4_K gate/up [2048][7168] and
    down [7168][2048] (24,772,608 B each) in pinned host memory, the shared
    expert (Q4_K, width 2048) resident in HBM, the f32 router with a
    Zipf(1.1) logit bias, sigmoid top-8 with renorm."""
    import torch

    from loom_amd import GATING_SIGMOID, Q4_K, MoeLayerEcDesc, plane_bytes
    from loom_amd import backend as be
    from loom_amd.expert_cache import HostBuffer

    gb, db = plane_bytes(Q4_K, C5_FFN, C5_DIM), plane_bytes(Q4_K, C5_DIM, C5_FFN)
    slot = 2 * gb + db
    host = HostBuffer(C5_E * slot)
    hv = torch.from_numpy(host.array)
    chunk = 16
    for e0 in range(0, C5_E, chunk):
        for k, (rows, cols, off) in enumerate(((C5_FFN, C5_DIM, 0), (C5_FFN, C5_DIM, gb), (C5_DIM, C5_FFN, 2 * gb))):
            pb = plane_bytes(Q4_K, rows, cols)
            dev = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, rows, cols, chunk, 5000 + 10 * e0 + k, 0.02),
                                rows, cols, chunk)
            d = dev.view(chunk, pb).cpu()
            for i in range(chunk):
                hv[(e0 + i) * slot + off:(e0 + i) * slot + off + pb].copy_(d[i])
            del dev
    g = torch.Generator(device="cuda").manual_seed(55)
    router = (torch.randn(C5_E, C5_DIM, generator=g, device="cuda") / np.sqrt(C5_DIM)).contiguous()
    ranks = torch.randperm(C5_E, generator=g, device="cuda").float() + 1
    z = -1.1 * torch.log(ranks)
    bias = (z - z.mean()).contiguous()
    sh = [be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, r, c, 1, 7000 + i, 0.02), r, c, 1)
          for i, (r, c) in enumerate(((C5_SFFN, C5_DIM), (C5_SFFN, C5_DIM), (C5_DIM, C5_SFFN)))]
    desc = MoeLayerEcDesc(C5_DIM, C5_FFN, C5_E, C5_K, GATING_SIGMOID, 1, 1.0, router.data_ptr(),
                          bias.data_ptr(), None, Q4_K, Q4_K, 0, 0, gb, 2 * gb,
                          Q4_K, Q4_K, Q4_K, sh[0].data_ptr(), sh[1].data_ptr(), sh[2].data_ptr(), C5_SFFN)
    return host, slot, gb, desc, (router, bias, sh)


def _c5_gets(ids, b):
    """The cache accesses of one call in get order: one token, moeFFN's
    selection order; more, each distinct expert once, ascending."""
    return list(ids[0]) if b == 1 else sorted(set(int(v) for v in ids.ravel()))


def bench_cache(args):
    """Config 5: the routed block (and its resident shared expert) decoding
    with its experts streamed from pinned host memory through a 64-slot HBM
    LRU (loomhip_moe_layer_cached); tok/s, hit rate and bytes over each link
    at batch 1 and 64 over args.cache_steps steps each, then the whole block
    with its MLA attention in front (bench_c5_block).  The access trace of
    each run is kept for the oracle's replay (cpu leg)."""
    import torch

    from loom_amd.expert_cache import ExpertCache

    t0 = time.perf_counter()
    host, slot, gb, desc, keep = _c5_layer()
    log(f"config 5: {C5_E} experts x {slot} B in pinned host memory in {time.perf_counter() - t0:.1f} s")
    ec = ExpertCache(C5_SLOTS, slot, C5_E)
    for e in range(C5_E):
        ec.set_source(e, host, e * slot, slot)
    # the fill rate alone: 64 distinct misses
    torch.cuda.synchronize()
    s0 = ec.stats
    t0 = time.perf_counter()
    for e in range(C5_SLOTS):
        ec.get(e)
    ec.release()
    torch.cuda.synchronize()
    fill_s = time.perf_counter() - t0
    fill_gbs = (ec.stats.bytes_read - s0.bytes_read) / fill_s / 1e9
    res = {"fill_GBs": round(fill_gbs, 2)}
    traces = {}
    g = torch.Generator(device="cuda").manual_seed(77)
    for b in (1, 64):
        steps = args.cache_steps
        ec.clear()
        warm = 16
        x = torch.randn(warm + steps, b, C5_DIM, generator=g, device="cuda")
        out = torch.empty(b, C5_DIM, device="cuda")
        warm_trace = []
        for i in range(warm):
            ids, _ = ec.moe_layer(desc, x[i], out, b, want_ids=True)
            warm_trace += _c5_gets(ids, b)
        torch.cuda.synchronize()
        s0 = ec.stats
        trace = []
        t0 = time.perf_counter()
        for i in range(warm, warm + steps):
            ids, _ = ec.moe_layer(desc, x[i], out, b, want_ids=True)
            trace += _c5_gets(ids, b)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        s1 = ec.stats
        hits = (s1.pin_hits - s0.pin_hits) + (s1.lru_hits - s0.lru_hits)
        miss = s1.disk_misses - s0.disk_misses
        key = f"b{b}"
        res[key] = {
            "steps": steps, "tok_s": round(b * steps / dt, 2), "ms_per_step": round(dt / steps * 1e3, 3),
            "hit_rate": round(hits / max(1, hits + miss), 4), "gets_per_step": round((hits + miss) / steps, 2),
            "misses_per_step": round(miss / steps, 2),
            "host_link_GBs": round((s1.bytes_read - s0.bytes_read) / dt / 1e9, 2),
            "hbm_hit_bytes_per_step": int(hits * slot / steps),
        }
        # the state the trace starts from is the warm-up's: replayed with it
        traces[key] = {"warm": warm_trace, "trace": trace,
                       "counts": (s1.pin_hits - s0.pin_hits, s1.lru_hits - s0.lru_hits, miss)}
        log(f"config 5 {key}: {res[key]}")
        del x
    res["block"] = bench_c5_block(args, ec, desc, traces, fill_gbs)
    ec.close()
    return res, host, gb, keep, traces


C5_LINK_PEAK_GBS = 64.0  # PCIe Gen5 x16, one direction: the host link's ceiling


def bench_c5_block(args, ec, desc, traces, fill_gbs):
    """Config 5 as one block (loomhip_mla_layer_cached_dev): deepseek.step's
    MLA layer with its experts streamed -- the MLA attention of each sequence
    over its own compressed cache (128 heads, kv_lora 512, rope 64, Q4_K
    kv_b), x += wo . heads (Q4_K [7168][16384]), the exact FFN rmsnorm, the
    256 routed experts through the 64-slot HBM LRU plus the resident shared
    expert, x += that -- for args.cache_steps sequential decode steps at batch
    1 and 64.  Each sequence's context grows by one position per step from a
    prefill of args.ctx seeded latent rows (the projections that would write
    the new rows are outside the block).  Per-step roofline: the step's HBM
    bytes at 8 TB/s plus its miss bytes over the host link (at the PCIe Gen5
    x16 peak, and at the measured fill rate)."""
    import torch

    from loom_amd import Q4_K
    from loom_amd import backend as be

    H, nope, rope, kvr, vd = MLA_H, MLA_NOPE, MLA_ROPE, MLA_KVR, MLA_VD
    scale = float(1.0 / np.sqrt(nope + rope))
    steps, warm, ctx0 = args.cache_steps, 16, args.ctx
    g = torch.Generator(device="cuda").manual_seed(83)
    kvb = be.synth_ggml_dev(Q4_K, H * (nope + vd), kvr, 1, 800, float(1 / np.sqrt(kvr)))
    attn = be.MlaAttn(Q4_K, kvb, H, nope, vd, kvr, rope, scale)
    wo = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, C5_DIM, H * vd, 1, 801, 0.02), C5_DIM, H * vd, 1)
    norm = (1.0 + 0.05 * torch.randn(C5_DIM, generator=g, device="cuda")).contiguous()
    ring = 16  # distinct queries, cycled (x, fresh every step, drives the routing)
    res = {}
    for b in (1, 64):
        cap = ctx0 + warm + steps
        caches = [(torch.randn(cap, kvr, generator=g, device="cuda"), torch.randn(cap, rope, generator=g, device="cuda"))
                  for _ in range(b)]
        cl, rl = [c for c, _ in caches], [r for _, r in caches]
        qn = torch.randn(ring, b, H * nope, generator=g, device="cuda")
        qr = torch.randn(ring, b, H * rope, generator=g, device="cuda")
        xs = torch.randn(warm + steps, b, C5_DIM, generator=g, device="cuda")
        ec.clear()
        warm_trace, trace = [], []
        for i in range(warm):
            ids = attn.cached_block(cl, rl, ctx0 + i + 1, qn[i % ring], qr[i % ring], Q4_K, wo, norm, 1e-6, desc, ec,
                                    xs[i], want_ids=True)
            warm_trace += _c5_gets(ids, b)
        torch.cuda.synchronize()
        s0 = ec.stats
        t0 = time.perf_counter()
        for i in range(warm, warm + steps):
            ids = attn.cached_block(cl, rl, ctx0 + i + 1, qn[i % ring], qr[i % ring], Q4_K, wo, norm, 1e-6, desc, ec,
                                    xs[i], want_ids=True)
            trace += _c5_gets(ids, b)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        s1 = ec.stats
        hits = (s1.pin_hits - s0.pin_hits) + (s1.lru_hits - s0.lru_hits)
        miss = s1.disk_misses - s0.disk_misses
        # the step's bytes: attention at the mean context (per sequence), wo,
        # the router, the hit experts and the shared expert from HBM; the
        # misses over the host link
        S = ctx0 + warm + (steps + 1) / 2
        attn_b = b * sum(mla_launch_bytes(k, S) for k in ("mla_scores", "mla_softmax", "mla_wsum")) + \
            mla_launch_bytes("mla_absorb", S) + mla_launch_bytes("mla_wv", S)
        hbm = attn_b + plane_bytes_q4k(C5_DIM, H * vd) + C5_E * C5_DIM * 4 + \
            hits / steps * C5_EXPERT_BYTES + 3 * plane_bytes_q4k(C5_SFFN, C5_DIM)
        link = miss / steps * C5_EXPERT_BYTES
        t_step = dt / steps
        floor_pcie = hbm / (HBM_PEAK_GBS * 1e9) + link / (C5_LINK_PEAK_GBS * 1e9)
        floor_fill = hbm / (HBM_PEAK_GBS * 1e9) + link / (fill_gbs * 1e9)
        key = f"block_b{b}"
        res[f"b{b}"] = {
            "steps": steps, "tok_s": round(b * steps / dt, 2), "ms_per_step": round(t_step * 1e3, 3),
            "hit_rate": round(hits / max(1, hits + miss), 4), "misses_per_step": round(miss / steps, 2),
            "ctx": [ctx0 + warm + 1, ctx0 + warm + steps],
            "hbm_bytes_per_step": int(hbm), "host_link_bytes_per_step": int(link),
            "roofline": {"bound": "hbm + host link", "floor_ms": round(floor_pcie * 1e3, 4),
                         "frac": round(floor_pcie / t_step, 4), "link_peak_GBs": C5_LINK_PEAK_GBS,
                         "floor_ms_at_fill_rate": round(floor_fill * 1e3, 4),
                         "frac_at_fill_rate": round(floor_fill / t_step, 4), "fill_GBs": round(fill_gbs, 2)},
        }
        traces[key] = {"warm": warm_trace, "trace": trace,
                       "counts": (s1.pin_hits - s0.pin_hits, s1.lru_hits - s0.lru_hits, miss)}
        log(f"config 5 block b{b}: {res[f'b{b}']}")
        del caches, cl, rl, qn, qr, xs
        torch.cuda.empty_cache()
    res["workload"] = (f"config 5 block (loomhip_mla_layer_cached_dev): MLA attention ({H} heads, kv_lora {kvr}, "
                       f"rope {rope}, Q4_K kv_b) over each sequence's own f32 latent cache, context growing from "
                       f"{ctx0 + warm + 1} by one per step, Q4_K wo [7168][16384] + residual, exact rmsnorm, "
                       f"{C5_E} streamed Q4_K experts top-{C5_K} through the {C5_SLOTS}-slot HBM LRU + the "
                       "resident shared expert + residual")
    del attn, wo, norm
    torch.cuda.empty_cache()
    return res


def cache_replay_check(traces):
    """SURVEY's config-5 bar: the hit/miss counts equal the oracle's replay of
    the same access trace exactly (ExpertCache.get order: pinned, LRU, miss;
    src/engine/expert_cache.zig:230-249).  The runs start from an empty cache
    (cleared before their warm-up), so the replay runs the warm-up's accesses
    and the timed ones; only the timed ones are compared."""
    import oracle as o

    o.build()
    out = {}
    for key, t in traces.items():
        warm, _ = o.cache_replay(C5_SLOTS, np.asarray(t["warm"], np.uint32), n_ids=C5_E)
        full, _ = o.cache_replay(C5_SLOTS, np.asarray(t["warm"] + t["trace"], np.uint32), n_ids=C5_E)
        timed = [int(f - w) for f, w in zip(full, warm)]
        dev = [int(v) for v in t["counts"]]
        out[key] = {"device": dev, "oracle": timed, "accesses": len(t["trace"]), "match": dev == timed}
    return out


def cpu_baseline_c5(host, gb, keep, threads, seconds):
    """Loom's CPU MoE block (the oracle's moeRun restatement and the shared
    expert, row-parallel pool) on the same 256 experts, read from the pinned
    host copy."""
    import oracle as o

    o.build()
    router, bias = (t.cpu().numpy() for t in keep[:2])
    sg, su, sd = (t.cpu().numpy() for t in keep[2])  # Q4_K: the device layout is GGML's
    slot = host.nbytes // C5_E
    db = slot - 2 * gb
    a = host.array.reshape(C5_E, slot)
    gate = np.ascontiguousarray(a[:, :gb])
    up = np.ascontiguousarray(a[:, gb:2 * gb])
    down = np.ascontiguousarray(a[:, 2 * gb:2 * gb + db])
    w = o.MoeWeights(C5_DIM, C5_FFN, C5_E, C5_K, router, gate, up, down, 12, 12, 12, router_bias=bias,
                     gating=o.GATING_SIGMOID, weights_norm=True, shexp=(sg, su, sd, 12, 12, 12, C5_SFFN))
    rng = np.random.default_rng(9)
    with o.Pool(threads):
        o.moe_layer_token(w, rng.standard_normal(C5_DIM).astype(np.float32))
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < seconds:
            o.moe_layer_token(w, rng.standard_normal(C5_DIM).astype(np.float32))
            n += 1
        dt = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} tokens through the config-5 routed block (moeRun order) and its shared expert "
                      f"with all 256 experts in host memory ({dt * 1e3:.1f} ms/token)"}




def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU expert split is design only)", file=sys.stderr)
        sys.exit(2)
    import torch

    import loom_amd
    from loom_amd.frame import DeviceModel, qwen3_30b_a3b

    loom_amd.init(0)
    if args.mla:
        line = {"metric": "MLA attention: us per layer and ms per token (config 5's attention)", "n_gpus": 1,
                "data": "synthetic", "dtype": "f32", **bench_mla(args, tuple(int(v) for v in args.mla_ctx.split(",") if v), cpu=not args.no_cpu)}
        print(json.dumps(line), flush=True)
        return
    if args.copy_probe:
        src = torch.empty(args.copy_probe << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {args.copy_probe} MB device to device")
        del src, dst
    if args.sweep or args.moe_layer:
        line = bench_sweep(args) if args.sweep else bench_moe_layer(args)
        print(json.dumps(line), flush=True)
        return
    batches = [int(v) for v in args.batch.split(",") if v]
    spec = qwen3_30b_a3b(ctx_len=args.ctx + 2 * args.warmup + args.steps + 64, n_layers=args.layers)
    t0 = time.perf_counter()
    dm = DeviceModel.synth(spec, seed=1234)
    torch.cuda.synchronize()
    log(f"model synthesised: {dm.weight_bytes() / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
    modes = ["parity", "fast"] if args.numerics == "both" else [args.numerics]
    res = {}
    for mode in modes:
        dm.set_numerics(loom_amd.NUMERICS_FAST if mode == "fast" else loom_amd.NUMERICS_PARITY)
        for b in batches:
            r = bench_batch(dm, b, args)
            r["roofline"], r["per_kernel"] = roofline(r, b, args.ctx, args.layers)
            r["bytes"] = step_bytes(b, args.ctx, r["distinct"], args.layers)
            res[mode, b] = r
            log(f"{mode} batch {b}: {r['ms']:.3f} ms/step, {r['tok_s']:.1f} tok/s, "
                f"{r['distinct']:.1f} distinct experts/layer, kernels {r['per_kernel']}")
    head, hmode = batches[0], modes[0]
    r = res[hmode, head]

    def step_roof(rr):
        gbs = rr["bytes"] / (rr["ms"] / 1e3) / 1e9
        return {"bytes_per_step": int(rr["bytes"]), "achieved_GBs": round(gbs, 1),
                "frac": round(gbs / HBM_PEAK_GBS, 4)}

    line = {
        "metric": METRIC, "value": round(r["tok_s"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"qwen3-30b-a3b shape (config 4): {args.layers} layers, GQA 32/4 x 128 "
                               "with QK-norm and NEOX rope, MoE 128 experts top-8 ffn 768 with a Zipf(1.1) "
                               "router bias, vocab 151936, Q4_K_M mix (Q4_K; Q6_K attn_v/ffn_down/output), "
                               f"fp16 K/V context {args.ctx} per sequence, seeded random weights",
                   "batch": head, "ctx": args.ctx, "layers": args.layers, "graph": not args.no_graph,
                   "numerics": hmode, "parallelism": "single-gpu"},
        "roofline": r["roofline"],
        "cpu_baseline": None,
        "step_roofline": step_roof(r),
        "kernels": r["per_kernel"],
        "distinct_experts_per_layer": round(r["distinct"], 2),
    }
    for b in batches[1:]:
        rb = res[hmode, b]
        line[f"batch{b}"] = {"value": round(rb["tok_s"], 2), "ms_per_step": round(rb["ms"], 4),
                             "distinct_experts_per_layer": round(rb["distinct"], 2),
                             "roofline": rb["roofline"], "step_roofline": step_roof(rb),
                             "kernels": rb["per_kernel"]}
        if b >= 16:  # the grouped expert matmuls run on the matrix cores
            line[f"batch{b}"]["moe_gemm"] = moe_gemm(rb, b, args.ctx)
    if "fast" in modes and hmode != "fast":
        # FAST numerics do not hold north_star's 2e-3 at this context: reported
        # beside the headline with the bound the tests measure for them
        line["fast"] = {
            "numerics": "fast (tree-summed rmsnorm, split-context attention on the matrix cores)",
            "measured_max_rel": FAST_MEASURED_MAXREL,
            "max_rel_source": "tests/test_gpu_frame.py::test_qwen3moe_frame_4096_context[32-fast] (2 layers, "
                              "4096-token context; PARITY measures 0.0 there)",
            **{f"batch{b}": {"value": round(res["fast", b]["tok_s"], 2), "ms_per_step": round(res["fast", b]["ms"], 4),
                             "step_roofline": step_roof(res["fast", b]), "roofline": res["fast", b]["roofline"],
                             "kernels": res["fast", b]["per_kernel"]} for b in batches}}
    cores = args.cpu_threads or max(1, min(16, os.cpu_count() or 1) - 2)
    del dm
    torch.cuda.empty_cache()
    if not args.no_cpu:
        log(f"cpu baseline: {cores} threads, {args.cpu_seconds} s sample")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds, cores, args.ctx)
    if not args.no_cache:
        c5, host, gb, keep, traces = bench_cache(args)
        line["expert_cache"] = {
            "workload": f"config 5: DeepSeek-V3-class routed block, hidden {C5_DIM}, {C5_E} experts top-{C5_K} "
                        "(sigmoid, renorm, Zipf(1.1) logit bias) plus 1 shared expert (ffn 2048, resident), "
                        "expert ffn 2048, Q4_K gate/up/down (24,772,608 B per expert), 6.34 GB pinned host "
                        f"backing store, {C5_SLOTS}-slot HBM LRU (1.59 GB); synthetic hidden states; b1/b64: the "
                        "routed block alone; block: the whole block with its MLA attention",
            **c5}
        if not args.no_cpu:
            line["expert_cache"]["cpu_baseline"] = cpu_baseline_c5(host, gb, keep, cores, args.cpu_seconds / 3)
            line["expert_cache"]["oracle_replay"] = cache_replay_check(traces)
        host.free()
    if not args.no_mla:
        line["mla"] = bench_mla(args, (args.ctx,), cpu=not args.no_cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
