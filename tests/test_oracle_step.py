"""Pins the oracle's whole-token step (oracle/model_ref.c lo_step, the
restatement of src/gguf/llama.zig step 1111-1227 with headNorm 938-949, rope
821-855 and the attention loop 1162-1192) against an independent float64
forward written from the reference's text, on CPU.

The float64 forward sees the same int8-quantized activations the reference's
matvecs see (quantizeX / quantizeX256, pinned in test_oracle_ggml) and the
same fp16 K/V rounding the oracle's config-4 cache applies, so only f32
accumulation separates the two (an int8 rounding flip it could cause would
show here as a ~1e-2 miss; the seeds are fixed and show none).
Planted mistakes (NORM/NEOX pairing swapped, rope rotation reversed, GQA
head mapping, keys rotated one position off the queries, q/k norm weights
dropped, attention scale) must each miss by far more than the bound.
"""
import ctypes as C

import numpy as np
import pytest

import npref

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


def _q(t, v):
    """The reference's int8 activation for weight type t, dequantized."""
    import oracle as o

    v = np.ascontiguousarray(v, np.float32)
    if t in (Q4_K, Q6_K):
        d, q, _ = o.quantize_x256(v)
    else:
        d, _, q = o.quantize_x(v)
    return (q.astype(np.float64) * d.astype(np.float64)[:, None]).ravel()


class TinyModel:
    """Host GGML tensors of a small model plus its lo_model."""

    def __init__(self, oracle, arch, seed):
        o = oracle
        rng = np.random.default_rng(seed)
        if arch == "qwen3moe":
            self.c = dict(dim=256, hd=32, nh=8, nkv=2, vocab=512, ctx=16, rope_dim=32, base=10000.0,
                          eps=1e-6, neox=True, qk_norm=True, moe=True, E=8, k=2, ffn=256,
                          wt=Q4_K, vt=Q6_K, et=Q4_K, ot=Q6_K, gt=Q4_K, dt=Q6_K, layers=2)
        else:
            self.c = dict(dim=128, hd=32, nh=4, nkv=4, vocab=256, ctx=16, rope_dim=32, base=10000.0,
                          eps=1e-5, neox=False, qk_norm=False, moe=False, ffn=256,
                          wt=Q4_0, vt=Q4_0, et=Q4_0, ot=Q4_0, gt=Q4_0, dt=Q4_0, layers=2)
        c = self.c
        self.keep = []
        qd, kvd = c["nh"] * c["hd"], c["nkv"] * c["hd"]

        def blocks(t, rows, cols, planes=1):
            raw = npref.pinned_scale_blocks(t, rows, cols, rng, planes=planes)
            self.keep.append(raw)
            return raw

        def f32(a):
            a = np.ascontiguousarray(a, np.float32)
            self.keep.append(a)
            return a

        def tensor(t, raw, rows, cols, planes=1):
            return o.Tensor(t, raw.ctypes.data, cols, rows, planes)

        self.embed = blocks(c["et"], c["vocab"], c["dim"])
        self.output = blocks(c["ot"], c["vocab"], c["dim"])
        self.out_norm = f32(rng.uniform(0.5, 1.5, c["dim"]))
        self.L = []
        layers = (o.Layer * c["layers"])()
        for li in range(c["layers"]):
            d = {}
            d["attn_norm"] = f32(rng.uniform(0.5, 1.5, c["dim"]))
            d["ffn_norm"] = f32(rng.uniform(0.5, 1.5, c["dim"]))
            d["wq"] = blocks(c["wt"], qd, c["dim"])
            d["wk"] = blocks(c["wt"], kvd, c["dim"])
            d["wv"] = blocks(c["vt"], kvd, c["dim"])
            d["wo"] = blocks(c["wt"], c["dim"], qd)
            L = layers[li]
            L.attn_norm, L.ffn_norm = d["attn_norm"].ctypes.data, d["ffn_norm"].ctypes.data
            L.wq = tensor(c["wt"], d["wq"], qd, c["dim"])
            L.wk = tensor(c["wt"], d["wk"], kvd, c["dim"])
            L.wv = tensor(c["vt"], d["wv"], kvd, c["dim"])
            L.wo = tensor(c["wt"], d["wo"], c["dim"], qd)
            if c["qk_norm"]:
                d["q_norm"] = f32(rng.uniform(0.5, 1.5, c["hd"]))
                d["k_norm"] = f32(rng.uniform(0.5, 1.5, c["hd"]))
                L.q_norm, L.k_norm = d["q_norm"].ctypes.data, d["k_norm"].ctypes.data
            if c["moe"]:
                d["router"] = f32(rng.normal(0, 1 / np.sqrt(c["dim"]), (c["E"], c["dim"])))
                d["gate"] = blocks(c["gt"], c["ffn"], c["dim"], c["E"])
                d["up"] = blocks(c["gt"], c["ffn"], c["dim"], c["E"])
                d["down"] = blocks(c["dt"], c["dim"], c["ffn"], c["E"])
                L.is_moe = 1
                L.moe = o.MoeLayer(c["dim"], c["ffn"], o.RouteCfg(c["E"], c["k"], o.GATING_SOFTMAX, 1, 1.0),
                                   o.Tensor(0, d["router"].ctypes.data, c["dim"], c["E"], 1), None, None,
                                   tensor(c["gt"], d["gate"], c["ffn"], c["dim"], c["E"]),
                                   tensor(c["gt"], d["up"], c["ffn"], c["dim"], c["E"]),
                                   tensor(c["dt"], d["down"], c["dim"], c["ffn"], c["E"]))
            else:
                d["ffn_gate"] = blocks(c["gt"], c["ffn"], c["dim"])
                d["ffn_up"] = blocks(c["gt"], c["ffn"], c["dim"])
                d["ffn_down"] = blocks(c["dt"], c["dim"], c["ffn"])
                L.is_moe = 0
                L.ffn_gate = tensor(c["gt"], d["ffn_gate"], c["ffn"], c["dim"])
                L.ffn_up = tensor(c["gt"], d["ffn_up"], c["ffn"], c["dim"])
                L.ffn_down = tensor(c["dt"], d["ffn_down"], c["dim"], c["ffn"])
            self.L.append(d)
        self.layers = layers
        self.model = o.Model(c["dim"], c["hd"], c["layers"], c["nh"], c["nkv"], c["vocab"], c["ctx"],
                             c["rope_dim"], c["base"], c["eps"], int(c["neox"]), 1,
                             tensor(c["et"], self.embed, c["vocab"], c["dim"]), self.out_norm.ctypes.data,
                             tensor(c["ot"], self.output, c["vocab"], c["dim"]), C.cast(layers, C.c_void_p))

    def oracle_logits(self, oracle, tokens):
        cb = int(oracle.lib().lo_seq_cache_bytes(C.byref(self.model)))
        k = np.zeros(cb, np.uint8)
        v = np.zeros(cb, np.uint8)
        seq = oracle.Seq(k.ctypes.data, v.ctypes.data, 0)
        out = []
        for tok in tokens:
            lg = np.empty(self.c["vocab"], np.float32)
            assert oracle.lib().lo_step(C.byref(self.model), C.byref(seq), int(tok), lg.ctypes.data) == 0
            out.append(lg)
        return np.array(out)


def _deq(t, raw, rows, cols, plane=0):
    from oracle import row_bytes

    pb = rows * row_bytes(t, cols)
    return npref.dequant(t, raw[plane * pb:(plane + 1) * pb], rows, cols).astype(np.float64)


def _rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def forward64(oracle, m, tokens, slip=None):
    """llama.step in float64 (src/gguf/llama.zig:1111-1227); `slip` plants
    one mistake."""
    c = m.c
    hd, nh, nkv, dim = c["hd"], c["nh"], c["nkv"], c["dim"]
    G, kvd = nh // nkv, nkv * c["hd"]
    W = [{k: _deq(*v) for k, v in (
        ("wq", (c["wt"], L["wq"], nh * hd, dim)), ("wk", (c["wt"], L["wk"], kvd, dim)),
        ("wv", (c["vt"], L["wv"], kvd, dim)), ("wo", (c["wt"], L["wo"], dim, nh * hd)))} for L in m.L]
    E = _deq(c["et"], m.embed, c["vocab"], dim)
    O = _deq(c["ot"], m.output, c["vocab"], dim)
    kc = np.zeros((c["layers"], c["ctx"], kvd))
    vc = np.zeros((c["layers"], c["ctx"], kvd))
    scale = 1.0 / np.sqrt(dim if slip == "scale" else hd)

    def rope(vec, pos):
        rd = c["rope_dim"]
        out = vec.copy()
        neox = c["neox"] if slip != "pairing" else not c["neox"]
        sgn = -1.0 if slip == "rotation" else 1.0
        for i in range(rd // 2):
            ang = pos * c["base"] ** (-(2 * i) / rd)
            cs, sn = np.cos(ang), sgn * np.sin(ang)
            ia, ib = (i, i + rd // 2) if neox else (2 * i, 2 * i + 1)
            a, b = vec[ia], vec[ib]
            out[ia] = a * cs - b * sn
            out[ib] = a * sn + b * cs
        return out

    logits = []
    for pos, tok in enumerate(tokens):
        x = E[tok].copy()
        for li, L in enumerate(m.L):
            w = W[li]
            h = _rms(x, L["attn_norm"], c["eps"])
            hq = _q(c["wt"], h)
            q = w["wq"] @ hq
            k = w["wk"] @ hq
            v = w["wv"] @ _q(c["vt"], h)
            if c["qk_norm"] and slip != "qk_norm":
                q = np.concatenate([_rms(q[i * hd:(i + 1) * hd], L["q_norm"], c["eps"]) for i in range(nh)])
                k = np.concatenate([_rms(k[i * hd:(i + 1) * hd], L["k_norm"], c["eps"]) for i in range(nkv)])
            q = np.concatenate([rope(q[i * hd:(i + 1) * hd], pos) for i in range(nh)])
            k = np.concatenate([rope(k[i * hd:(i + 1) * hd], pos + (slip == "pos")) for i in range(nkv)])
            kc[li, pos] = k.astype(np.float16).astype(np.float64)  # the fp16 cache
            vc[li, pos] = v.astype(np.float16).astype(np.float64)
            att = np.zeros(nh * hd)
            for hh in range(nh):
                kvh = hh % nkv if slip == "gqa" else hh // G
                qh = q[hh * hd:(hh + 1) * hd]
                s = kc[li, :pos + 1, kvh * hd:(kvh + 1) * hd] @ qh * scale
                p = np.exp(s - s.max())
                p /= p.sum()
                att[hh * hd:(hh + 1) * hd] = p @ vc[li, :pos + 1, kvh * hd:(kvh + 1) * hd]
            x = x + w["wo"] @ _q(c["wt"], att)
            h2 = _rms(x, L["ffn_norm"], c["eps"])
            if c["moe"]:
                lg = (L["router"].astype(np.float64) @ h2).astype(np.float32)
                ids, gates = oracle.route(lg, c["k"], oracle.GATING_SOFTMAX, True, 1.0)
                hq2 = _q(c["gt"], h2)
                acc = np.zeros(dim)
                for e, g in zip(ids, gates):
                    gt = _deq(c["gt"], L["gate"], c["ffn"], dim, e) @ hq2
                    ut = _deq(c["gt"], L["up"], c["ffn"], dim, e) @ hq2
                    a = gt / (1.0 + np.exp(-gt)) * ut
                    acc += float(g) * (_deq(c["dt"], L["down"], dim, c["ffn"], e) @ _q(c["dt"], a))
                x = x + acc
            else:
                hq2 = _q(c["gt"], h2)
                gt = _deq(c["gt"], L["ffn_gate"], c["ffn"], dim) @ hq2
                ut = _deq(c["gt"], L["ffn_up"], c["ffn"], dim) @ hq2
                a = gt / (1.0 + np.exp(-gt)) * ut
                x = x + _deq(c["dt"], L["ffn_down"], dim, c["ffn"]) @ _q(c["dt"], a)
        logits.append(O @ _q(c["ot"], _rms(x, m.out_norm, c["eps"])))
    return np.array(logits)


def _rel(a, b):
    return np.abs(a - b).max(axis=1) / np.abs(b).max(axis=1)


# observed: ~3e-7 (f32 vs f64 accumulation; no int8 rounding flip at these
# seeds, which are fixed); the slips miss by 2e-2 .. 1.6
BOUND = 1e-4


@pytest.mark.parametrize("arch", ["qwen3moe", "llama"])
def test_step_matches_float64_forward(oracle, arch):
    m = TinyModel(oracle, arch, seed=21)
    tokens = np.random.default_rng(5).integers(0, m.c["vocab"], 8)
    got = m.oracle_logits(oracle, tokens)
    want = forward64(oracle, m, tokens)
    rel = _rel(got, want)
    assert rel.max() < BOUND, rel
    assert np.array_equal(np.argmax(got, axis=1), np.argmax(want, axis=1))


@pytest.mark.parametrize("arch,slips", [
    ("qwen3moe", ["pairing", "rotation", "gqa", "pos", "qk_norm", "scale"]),
    ("llama", ["pairing", "rotation", "pos", "scale"]),
])
def test_step_planted_mistakes_exceed_the_bound(oracle, arch, slips):
    m = TinyModel(oracle, arch, seed=22)
    tokens = np.random.default_rng(6).integers(0, m.c["vocab"], 8)
    got = m.oracle_logits(oracle, tokens)
    assert _rel(got, forward64(oracle, m, tokens)).max() < BOUND
    for slip in slips:
        bad = _rel(got, forward64(oracle, m, tokens, slip)).max()
        assert bad > 10 * BOUND, (slip, bad)


# ---- decodeBatch == independent single streams (llama.zig:2323-2389) -------


def _batch_vs_single(oracle, m, n, seed, n_steps=4):
    """Lane k first runs its own prompt of (k % 5) + 1 tokens through lo_step,
    so the lanes sit at different positions over different contexts; its
    cache is then copied to a batch lane.  n_steps of lo_decode_batch over all
    lanes are compared with lo_step on each lane's single stream, fed the
    same (greedy) tokens.  Returns (worst tolerance ratio, tokens equal)."""
    o = oracle
    L = o.lib()
    vocab = m.c["vocab"]
    cb = int(L.lo_seq_cache_bytes(C.byref(m.model)))
    rng = np.random.default_rng(seed)
    single, bufs = [], []
    for k in range(n):
        kb, vb = np.zeros(cb, np.uint8), np.zeros(cb, np.uint8)
        s = o.Seq(kb.ctypes.data, vb.ctypes.data, 0)
        lg = np.empty(vocab, np.float32)
        for tok in rng.integers(0, vocab, (k % 5) + 1):
            assert L.lo_step(C.byref(m.model), C.byref(s), int(tok), lg.ctypes.data) == 0
        single.append((s, lg))
        bufs += [kb, vb]
    seqs = (o.Seq * n)()
    copies = []
    for k in range(n):
        kb, vb = bufs[2 * k].copy(), bufs[2 * k + 1].copy()
        copies += [kb, vb]
        seqs[k].k_cache, seqs[k].v_cache, seqs[k].pos = kb.ctypes.data, vb.ctypes.data, single[k][0].pos
    assert len({int(seqs[k].pos) for k in range(n)}) == min(n, 5)
    worst, same = 0.0, True
    toks = np.array([int(np.argmax(single[k][1])) for k in range(n)], np.uint32)
    for _ in range(n_steps):
        got = np.empty((n, vocab), np.float32)
        assert L.lo_decode_batch(C.byref(m.model), C.cast(seqs, C.c_void_p), toks.ctypes.data, n,
                                 got.ctypes.data) == 0
        want = np.empty((n, vocab), np.float32)
        for k in range(n):
            assert L.lo_step(C.byref(m.model), C.byref(single[k][0]), int(toks[k]), want[k].ctypes.data) == 0
        tol = np.maximum(np.abs(want), np.abs(got)) * 1e-3 + 1e-3  # the reference test's bound
        worst = max(worst, float((np.abs(got - want) / tol).max()))
        same &= bool(np.array_equal(np.argmax(got, axis=1), np.argmax(want, axis=1)))
        toks = np.argmax(want, axis=1).astype(np.uint32)
    return worst, same


@pytest.mark.parametrize("arch", ["qwen3moe", "llama"])
@pytest.mark.parametrize("n", [2, 3, 8, 11])
def test_decode_batch_equals_single_streams(oracle, arch, n):
    """lo_decode_batch over n lanes at different positions and contexts
    equals n independent lo_step streams: every logit within the reference
    test's max(|w|, |g|)*1e-3 + 1e-3, identical greedy tokens."""
    m = TinyModel(oracle, arch, seed=40 + n)
    worst, same = _batch_vs_single(oracle, m, n, seed=n)
    assert worst <= 1.0, worst
    assert same


@pytest.mark.parametrize("slip,name", [(1, "cross-lane cache read"), (2, "K/V row at the batch index"),
                                       (3, "rope at lane 0's position")])
def test_decode_batch_planted_mistakes_break_the_invariant(oracle, slip, name):
    """Each silent failure mode the reference's test names (llama.zig:
    2324-2328), planted in the oracle's lo_decode_batch, breaks the
    batch == single-streams comparison above."""
    m = TinyModel(oracle, "qwen3moe", seed=48)
    assert _batch_vs_single(oracle, m, 8, seed=8)[0] <= 1.0
    oracle.lib().lo_set_batch_slip(slip)
    try:
        worst, _ = _batch_vs_single(oracle, m, 8, seed=8)
    finally:
        oracle.lib().lo_set_batch_slip(0)
    assert worst > 10.0, (name, worst)


@pytest.mark.parametrize("heads", [(4, 1, 64), (8, 4, 48), (6, 6, 32)])
def test_attn_heads_against_float64(oracle, heads):
    """lo_attn_heads (backend.attnHeads' contract, llama.zig:1162-1192; the
    loop lo_step itself runs) against float64 attention over the same fp16
    cache: softmax(scale * q_h . K^T) V with head h reading KV head h / G,
    within 1e-5 of the output's scale.  Planted in the oracle's inputs: the
    scale off by 2x, or the query heads permuted (another KV head mapping),
    each miss by far more than the bound."""
    n_heads, n_kv, hd = heads
    layers, ctx, li, pos = 3, 40, 1, 33
    kvd = n_kv * hd
    rng = np.random.default_rng(n_heads * 100 + hd)
    kc = rng.standard_normal((layers, ctx, kvd)).astype(np.float16)
    vc = rng.standard_normal((layers, ctx, kvd)).astype(np.float16)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    m = oracle.Model()
    m.head_dim, m.n_layers, m.n_heads, m.n_kv_heads, m.ctx_len, m.kv_f16 = hd, layers, n_heads, n_kv, ctx, 1

    def run(qv, sc):
        out = np.empty(n_heads * hd, np.float32)
        oracle.lib().lo_attn_heads(C.byref(m), kc.ctypes.data, vc.ctypes.data, li, pos, qv.ctypes.data,
                                   out.ctypes.data, sc)
        return out

    G = n_heads // n_kv
    K = kc[li, :pos + 1].astype(np.float64).reshape(pos + 1, n_kv, hd)
    V = vc[li, :pos + 1].astype(np.float64).reshape(pos + 1, n_kv, hd)
    want = np.empty((n_heads, hd))
    for h in range(n_heads):
        s = K[:, h // G] @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        p = np.exp(s - s.max())
        want[h] = (p / p.sum()) @ V[:, h // G]
    want = want.ravel()
    bound = 1e-5 * np.abs(want).max()
    assert np.abs(run(q, scale) - want).max() <= bound
    assert np.abs(run(q, 2 * scale) - want).max() > 100 * bound
    perm = np.roll(q.reshape(n_heads, hd), G, axis=0).ravel().copy()
    if n_kv > 1:
        assert np.abs(run(perm, scale) - want).max() > 100 * bound
