"""Pins the CPU oracle's routing, MoE layer and expert-cache bookkeeping
(oracle/model_ref.c, oracle/cache_ref.c) against the reference's own
known-answer tests, independent numpy restatements, float64 forwards and an
OrderedDict LRU replay.  CPU only."""
import collections
import json
import math
import os

import numpy as np
import pytest

import npref

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
Q4_K, Q6_K, Q8_0, F32 = 12, 14, 8, 0


def _sig(x):
    return 1.0 / (1.0 + math.exp(-x))


# ---- routing ---------------------------------------------------------------------


def test_route_reference_kats(oracle):
    gat = {"sigmoid": oracle.GATING_SIGMOID, "softmax": oracle.GATING_SOFTMAX,
           "softmax_topk": oracle.GATING_SOFTMAX_TOPK}
    expect_gates = {  # the literals the reference tests assert, evaluated
        "src/gguf/moe.zig:210-223": [_sig(0.0), _sig(3.0)],
        "src/gguf/moe.zig:225-242": [math.exp(3) / (math.exp(3) + math.exp(2)),
                                     math.exp(2) / (math.exp(3) + math.exp(2))],
    }
    for case in GOLD["route"]:
        ids, gates = oracle.route(np.array(case["logits"], np.float32), case["n_used"],
                                  gat[case["gating"]], case["weights_norm"], case["weights_scale"],
                                  None if case["bias"] is None else np.array(case["bias"], np.float32))
        if "expect_ids" in case:
            assert list(ids) == case["expect_ids"], case["source"]
        if case["source"] in expect_gates:
            assert np.allclose(gates, expect_gates[case["source"]], atol=case["gate_tol"]), case["source"]
        if "expect_gate_sum" in case:
            assert abs(float(gates.sum()) - case["expect_gate_sum"]) < 1e-5, case["source"]


def _route_numpy(logits, k, gating, norm, scale, bias):
    """Independent restatement: float32 scores, a stable sort on
    (-choice, index) for the k strict-'>' argmax rounds, float32 gate tail."""
    l = logits.astype(np.float32)
    if gating == 2:
        sc = (np.float32(1) / (np.float32(1) + np.exp(-l))).astype(np.float32)
    elif gating == 3:
        sc = l.copy()
    else:
        e = np.exp(l - l.max()).astype(np.float32)
        s = np.float32(0)
        for v in e:  # the reference's sequential sum
            s = np.float32(s + v)
        sc = (e * (np.float32(1) / s)).astype(np.float32)
    ch = sc if bias is None else (sc + bias).astype(np.float32)
    order = sorted(range(len(ch)), key=lambda i: (-float(ch[i]), i))
    ids = np.array(order[:k], np.uint32)
    g = sc[ids].astype(np.float32)
    if gating == 3:
        ge = np.exp(g - g.max()).astype(np.float32)
        s = np.float32(0)
        for v in ge:
            s = np.float32(s + v)
        g = (ge * (np.float32(1) / s)).astype(np.float32)
    if norm:
        s = np.float32(0)
        for v in g:
            s = np.float32(s + v)
        g = (g / max(s, np.float32(6.103515625e-5))).astype(np.float32)
    if scale != 1.0:
        g = (g * np.float32(scale)).astype(np.float32)
    return ids, g


@pytest.mark.parametrize("gating", [1, 2, 3])
@pytest.mark.parametrize("with_bias", [False, True])
def test_route_matches_numpy_restatement(oracle, gating, with_bias):
    rng = np.random.default_rng(gating * 10 + with_bias)
    for trial in range(40):
        E = int(rng.choice([8, 64, 128, 256]))
        k = int(rng.integers(1, min(E, 16) + 1))
        logits = rng.normal(0, 2, E).astype(np.float32)
        if trial % 3 == 0:  # exact ties: the lowest index must win
            logits[E // 2] = logits[E // 3]
        bias = rng.normal(0, 0.3, E).astype(np.float32) if with_bias else None
        norm, scale = bool(trial % 2), [1.0, 2.5][trial % 2]
        ids, gates = oracle.route(logits, k, gating, norm, scale, bias)
        wid, wg = _route_numpy(logits, k, gating, norm, scale, bias)
        assert np.array_equal(ids, wid), (E, k, trial)
        assert np.allclose(gates, wg, rtol=2e-6, atol=1e-7), (E, k, trial)


def test_route_picks_expert_zero_when_nothing_beats_minus_inf(oracle):
    # every selection value -inf: each round keeps best = 0 (moe.zig:128-140)
    logits = np.full(8, -np.inf, np.float32)
    ids, _ = oracle.route(logits, 3, oracle.GATING_SOFTMAX_TOPK, False, 1.0)
    assert list(ids) == [0, 0, 0]
    logits = np.array([1.0, -np.inf, 2.0, -np.inf], np.float32)
    ids, _ = oracle.route(logits, 3, oracle.GATING_SOFTMAX_TOPK, False, 1.0)
    assert list(ids) == [2, 0, 0]


# ---- MoE layer ---------------------------------------------------------------------


def _layer(oracle, dim, ffn, E, k, seed, gate_t=Q4_K, down_t=Q6_K):
    rng = np.random.default_rng(seed)
    gate = npref.pinned_scale_blocks(gate_t, ffn, dim, rng, planes=E)
    up = npref.pinned_scale_blocks(gate_t, ffn, dim, rng, planes=E)
    down = npref.pinned_scale_blocks(down_t, dim, ffn, rng, planes=E)
    router = oracle.normal(E * dim, seed + 1, 0.0, 1.0 / np.sqrt(dim)).reshape(E, dim)
    rb = rng.normal(0, 0.5, E).astype(np.float32)
    return oracle.MoeWeights(dim, ffn, E, k, router, gate, up, down, gate_t, gate_t, down_t,
                             router_bias=rb)


def _plane(t, raw, e, rows, cols):
    from oracle import row_bytes

    pb = rows * row_bytes(t, cols)
    return npref.dequant(t, raw[e * pb:(e + 1) * pb], rows, cols).astype(np.float64)


def _q256(v):
    """The reference's int8 activation for K-quant weights (quantizeX256,
    ggml.zig:776-800, pinned by test_oracle_ggml), dequantized."""
    import oracle as o

    d, q, _ = o.quantize_x256(np.ascontiguousarray(v, np.float32))
    return (q.astype(np.float64) * d.astype(np.float64)[:, None]).ravel()


def test_moe_layer_token_against_float64_forward(oracle):
    """llama.moeLayer + moeRun (llama.zig:1262-1419): router matvec + logit
    bias -> route -> per selected expert silu(gate x) * (up x) -> down ->
    gate-weighted sum.  The float64 forward sees the same int8-quantized
    activations the reference's kernels see, so only f32 accumulation
    separates it from the oracle."""
    dim, ffn, E, k = 256, 256, 8, 2
    w = _layer(oracle, dim, ffn, E, k, seed=5)
    for s in range(6):
        x = oracle.normal(dim, 100 + s, 0.0, 1.0)
        got, ids, gates = oracle.moe_layer_token(w, x)
        logits = (w.router.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
        logits = (logits + w.router_bias).astype(np.float32)
        wid, wg = oracle.route(logits, k, oracle.GATING_SOFTMAX, True, 1.0)
        assert np.array_equal(ids, wid)
        xq = _q256(x)
        want = np.zeros(dim)
        for e, g in zip(ids, gates):
            gt = _plane(w.gate_t, w.gate, e, ffn, dim) @ xq
            ut = _plane(w.up_t, w.up, e, ffn, dim) @ xq
            h = gt / (1.0 + np.exp(-gt)) * ut
            want += float(g) * (_plane(w.down_t, w.down, e, dim, ffn) @ _q256(h))
        rel = np.abs(got - want).max() / np.abs(want).max()
        assert rel < 2e-3, rel


def test_moe_layer_planted_mistakes_exceed_the_bound(oracle):
    """The float64 forward's 2e-3 bound separates a correct layer from
    plausible slips: slots' planes swapped, SwiGLU's silu dropped, gates
    unnormalised.  Each slip must miss by more than 10x the bound."""
    dim, ffn, E, k = 256, 256, 8, 4
    w = _layer(oracle, dim, ffn, E, k, seed=6)
    w.router_bias = None
    x = oracle.normal(dim, 1007, 0.0, 1.0)  # a stream unrelated to the router's
    got, ids, gates = oracle.moe_layer_token(w, x)
    xq = _q256(x)

    def forward(plane_of, act, gate_of):
        out = np.zeros(dim)
        for s_, (e, g) in enumerate(zip(ids, gates)):
            pe = plane_of(s_, e)
            gt = _plane(w.gate_t, w.gate, pe, ffn, dim) @ xq
            ut = _plane(w.up_t, w.up, pe, ffn, dim) @ xq
            out += gate_of(s_, g) * (_plane(w.down_t, w.down, pe, dim, ffn) @ _q256(act(gt, ut)))
        return out

    def rel(v):
        return np.abs(got - v).max() / np.abs(v).max()

    silu = lambda gt, ut: gt / (1.0 + np.exp(-gt)) * ut
    right = forward(lambda s_, e: e, silu, lambda s_, g: float(g))
    assert rel(right) < 2e-3
    swapped = forward(lambda s_, e: ids[(s_ + 1) % k], silu, lambda s_, g: float(g))
    no_silu = forward(lambda s_, e: e, lambda gt, ut: gt * ut, lambda s_, g: float(g))
    raw = (w.router.astype(np.float64) @ x.astype(np.float64))
    p = np.exp(raw - raw.max()) / np.exp(raw - raw.max()).sum()
    unnorm = forward(lambda s_, e: e, silu, lambda s_, g: float(p[ids[s_]]))
    for bad in (swapped, no_silu, unnorm):
        assert rel(bad) > 2e-2, rel(bad)


@pytest.mark.parametrize("n", [1, 3, 8, 11])
def test_moe_batch_union_matches_per_token(oracle, n):
    """llama.moeBatchUnion (llama.zig:1828-1924) == per-token moeRun up to the
    combine order: the reference's own bound, 1e-3*max + 1e-3
    (llama.zig:2323-2389)."""
    dim, ffn, E, k = 256, 256, 16, 4
    w = _layer(oracle, dim, ffn, E, k, seed=9 + n)
    xs = np.stack([oracle.normal(dim, 300 + i, 0.0, 1.0) for i in range(n)])
    resid = np.stack([oracle.normal(dim, 400 + i, 0.0, 1.0) for i in range(n)])
    got, ids, gates = oracle.moe_batch_union(w, xs, resid)
    for i in range(n):
        acc, tid, tg = oracle.moe_layer_token(w, xs[i])
        assert np.array_equal(ids[i], tid)
        assert np.array_equal(gates[i].view(np.uint32), tg.view(np.uint32))
        want = resid[i] + acc
        assert np.all(np.abs(got[i] - want) <= 1e-3 * np.abs(want).max() + 1e-3)


# ---- expert cache bookkeeping ------------------------------------------------------


def test_lru_reference_kat(oracle):
    kat = GOLD["lru_eviction"]
    lru = oracle.Lru(kat["capacity"])
    for op in kat["ops"]:
        if op[0] == "reserve":
            lru.reserve(op[1])
        else:
            assert (lru.find(op[1]) >= 0) == op[2], op


def _replay_numpy(capacity, trace, pinned):
    lru = collections.OrderedDict()
    counts = [0, 0, 0]
    mask = []
    for t in trace:
        if pinned is not None and pinned[t]:
            counts[0] += 1
            mask.append(1)
        elif t in lru:
            lru.move_to_end(t)
            counts[1] += 1
            mask.append(2)
        else:
            if len(lru) >= capacity:
                lru.popitem(last=False)
            lru[t] = True
            counts[2] += 1
            mask.append(0)
    return counts, mask


@pytest.mark.parametrize("capacity,n_ids", [(1, 4), (4, 16), (64, 256), (100, 128)])
def test_cache_replay_matches_ordereddict(oracle, capacity, n_ids):
    """ExpertCache.get order (expert_cache.zig:230-249): pinned -> LRU (touch
    to front) -> miss (fill free slots first, else evict the tail); the same
    replay as scripts/expert-replay-sim.py:53-113."""
    rng = np.random.default_rng(capacity * 7 + n_ids)
    ranks = np.arange(1, n_ids + 1, dtype=np.float64)
    p = ranks ** -1.1
    p /= p.sum()
    trace = rng.choice(n_ids, size=5000, p=p).astype(np.uint32)
    for pinned in (None, (rng.random(n_ids) < 0.1).astype(np.uint8)):
        counts, mask = oracle.cache_replay(capacity, trace, pinned=pinned, n_ids=n_ids)
        wc, wm = _replay_numpy(capacity, trace, pinned)
        assert list(counts) == wc
        assert list(mask) == wm


def test_hottest_within_budget_kat(oracle):
    kat = GOLD["hottest_within_budget"]
    got = oracle.hottest_within_budget(np.array(kat["counts"], np.uint64), kat["expert_bytes"],
                                       kat["budget"])
    assert sorted(got) == sorted(kat["expect_ids_set"])


# ---- shared expert and moeFfnBlock -------------------------------------------------


def _shexp(oracle, dim, sffn, seed, t=Q4_K, down_t=Q6_K):
    rng = np.random.default_rng(seed)
    g = npref.pinned_scale_blocks(t, sffn, dim, rng)
    u = npref.pinned_scale_blocks(t, sffn, dim, rng)
    d = npref.pinned_scale_blocks(down_t, dim, sffn, rng)
    return g, u, d, t, t, down_t, sffn


def _ffn64(gate_t, g, u, down_t, d, x, dim, f, plane=0):
    xq = _q256(x)
    gt = _plane(gate_t, g, plane, f, dim) @ xq
    ut = _plane(gate_t, u, plane, f, dim) @ xq
    return _plane(down_t, d, plane, dim, f) @ _q256(gt / (1.0 + np.exp(-gt)) * ut)


@pytest.mark.parametrize("slip", [None, "no_shared", "shared_weighted", "shared_before_norm"])
def test_moe_layer_with_shared_expert_against_float64(oracle, slip):
    """deepseek.zig:1485-1502: acc = sum over the selected experts of gate *
    FFN_e(x), then acc += FFN_shared(x) (unweighted, wider).  Against a
    float64 forward within 2e-3; the planted slips (shared expert dropped,
    scaled by the last gate, fed a scaled input) miss by far
    more."""
    dim, ffn, sffn, E, k = 256, 256, 512, 8, 2
    w = _layer(oracle, dim, ffn, E, k, seed=15)
    w.shexp = _shexp(oracle, dim, sffn, seed=16)
    g, u, d, gt_, _, dt_, _ = w.shexp
    worst = 0.0
    for s in range(4):
        x = oracle.normal(dim, 500 + s, 0.0, 1.0)
        got, ids, gates = oracle.moe_layer_token(w, x)
        want = np.zeros(dim)
        for e, gg in zip(ids, gates):
            want += float(gg) * _ffn64(w.gate_t, w.gate, w.up, w.down_t, w.down, x, dim, ffn, plane=e)
        sh = _ffn64(gt_, g, u, dt_, d, x, dim, sffn)
        if slip is None:
            want += sh
        elif slip == "shared_weighted":
            want += float(gates[-1]) * sh
        elif slip == "shared_before_norm":
            want += _ffn64(gt_, g, u, dt_, d, 3.0 * x, dim, sffn)
        worst = max(worst, float(np.abs(got - want).max() / np.abs(want).max()))
    if slip is None:
        assert worst < 2e-3, worst
    else:
        assert worst > 2e-2, (slip, worst)


def test_moe_batch_union_shared_expert_matches_per_token(oracle):
    """The batched layer adds each lane's shared expert after its routed
    experts: per lane within the reference's batch bound of moeRun + shared."""
    dim, ffn, sffn, E, k, n = 256, 256, 512, 16, 4, 5
    w = _layer(oracle, dim, ffn, E, k, seed=17)
    w.shexp = _shexp(oracle, dim, sffn, seed=18)
    xs = np.stack([oracle.normal(dim, 600 + i, 0.0, 1.0) for i in range(n)])
    resid = np.zeros((n, dim), np.float32)
    got, _, _ = oracle.moe_batch_union(w, xs, resid)
    for i in range(n):
        acc, _, _ = oracle.moe_layer_token(w, xs[i])
        assert np.all(np.abs(got[i] - acc) <= 1e-3 * np.abs(acc).max() + 1e-3)


def test_moe_ffn_block_against_float64(oracle):
    """backend.moeFfnBlock (compute/cpu.zig:23-30; metal/backend.zig:2322-2410):
    out = sum over the refs in order of weight * FFN_ref(x), the shared expert
    as a ref of weight 1 and its own width.  Float64 forward within 2e-3;
    weights applied to the wrong refs miss."""
    dim, ffn, sffn, E = 256, 256, 512, 6
    w = _layer(oracle, dim, ffn, E, 2, seed=19)
    from oracle import row_bytes

    gb, db = ffn * row_bytes(w.gate_t, dim), dim * row_bytes(w.down_t, ffn)
    g_, u_, d_, gt_, ut_, dt_, _ = _shexp(oracle, dim, sffn, seed=20)
    weights = [0.4, 0.25, 0.2, 0.15]
    refs = [(w.gate[e * gb:(e + 1) * gb], w.up[e * gb:(e + 1) * gb], w.down[e * db:(e + 1) * db],
             w.gate_t, w.up_t, w.down_t, ffn, wt) for e, wt in zip([3, 0, 5, 1], weights)]
    refs.append((g_, u_, d_, gt_, ut_, dt_, sffn, 1.0))
    x = oracle.normal(dim, 700, 0.0, 1.0)
    got = oracle.moe_ffn_block(x, refs)
    parts = [_ffn64(w.gate_t, w.gate, w.up, w.down_t, w.down, x, dim, ffn, plane=e) for e in [3, 0, 5, 1]]
    sh = _ffn64(gt_, g_, u_, dt_, d_, x, dim, sffn)
    want = sum(wt * p for wt, p in zip(weights, parts)) + sh
    assert np.abs(got - want).max() / np.abs(want).max() < 2e-3
    wrong = sum(wt * p for wt, p in zip(weights[::-1], parts)) + sh
    assert np.abs(got - wrong).max() / np.abs(wrong).max() > 2e-2
