"""The oracle's MLA attention (oracle/mla_ref.c, deepseek.zig:988-1047)
against a float64 forward that never absorbs: it decompresses every cached
position's key and value per head (K_t = W_k c_t, V_t = W_v c_t, the form
the reference's comment at deepseek.zig:896-914 says the absorption is
equal to) from the independent numpy decoder's weights.  A mistake in the
absorption (head stride, W_k/W_v rows, the rope term, the scale, the
context length) makes the float64 forward miss by far more than the bound;
each is planted in the float64 forward and must miss the oracle."""
import numpy as np
import pytest

import npref
from mla_case import make_case

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


def mla64(case, seq, slip=None):
    """(out, o_lat) in float64 by decompression; `slip` plants one mistake."""
    H, nope, vd, kvr = case.n_heads, case.nope, case.vd, case.kvr
    W = npref.dequant(case.t, case.kv_b, H * (nope + vd), kvr).astype(np.float64)
    c = case.c_kv[:seq - 1 if slip == "seq" else seq].astype(np.float64)
    kr = case.k_rope[:c.shape[0]].astype(np.float64)
    scale = 1.0 if slip == "scale" else case.scale
    out, olat = [], []
    for h in range(H):
        base = h * (nope if slip == "stride" else nope + vd)
        Wk, Wv = W[base:base + nope], W[base + nope:base + nope + vd]
        if slip == "kv_swap":
            Wk = W[base + nope:base + nope + nope] if vd >= nope else Wk[::-1]
        K, V = c @ Wk.T, c @ Wv.T
        hr = 0 if slip == "rope_head" else h
        qr = case.q_rope[hr * case.rope:(hr + 1) * case.rope].astype(np.float64)
        s = K @ case.q_nope[h * nope:(h + 1) * nope].astype(np.float64)
        if slip != "no_rope":
            s = s + kr @ qr
        s = s * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out.append(p @ V)
        olat.append(p @ c)
    return np.concatenate(out), np.concatenate(olat), W


CASES = [
    # the reference's own device test shape (vulkan/backend.zig:1432-1450): Q8_0, 4 heads
    ("vulkan_test", Q8_0, 4, 32, 16, 64, 16, 64, 5),
    ("q4_0", Q4_0, 4, 32, 16, 64, 16, 64, 9),
    # config 5's per-head shape (DeepSeek-V3: nope 128, rope 64, kv_lora 512, v 128), fewer heads
    ("q4_k", Q4_K, 8, 128, 128, 512, 64, 80, 77),
    ("q6_k", Q6_K, 8, 128, 128, 512, 64, 80, 33),
]
# observed: o_lat 1.2e-7 .. 5.5e-7 relative; the slips miss by 0.3 .. 0.9
OLAT_BOUND = 2e-6


@pytest.mark.parametrize("name,t,H,nope,vd,kvr,rope,ctx,seq", CASES, ids=[c[0] for c in CASES])
def test_mla_attention_matches_decompressed_float64(oracle, name, t, H, nope, vd, kvr, rope, ctx, seq):
    case = make_case(oracle, t, H, nope, vd, kvr, rope, ctx, seed=sum(map(ord, name)))
    out, olat = oracle.mla_attn_heads(case.c_kv, case.k_rope, seq, case.q_nope, case.q_rope, t, case.kv_b,
                                      H, nope, vd, case.scale)
    want, want_lat, W = mla64(case, seq)
    rel = np.abs(olat - want_lat).max() / np.abs(want_lat).max()
    assert rel < OLAT_BOUND, rel
    # W_v is a matvec with int8 activations: the reference's matvec bound
    # |y - w.x| <= 0.01 * sum |w * x| per row (ggml.zig tests)
    for h in range(H):
        Wv = W[h * (nope + vd) + nope:(h + 1) * (nope + vd)]
        x = want_lat[h * kvr:(h + 1) * kvr]
        bound = 0.01 * np.abs(Wv * x).sum(axis=1)
        assert np.all(np.abs(out[h * vd:(h + 1) * vd] - want[h * vd:(h + 1) * vd]) <= bound), h


@pytest.mark.parametrize("slip", ["stride", "kv_swap", "no_rope", "rope_head", "scale", "seq"])
def test_mla_planted_mistakes_exceed_the_bound(oracle, slip):
    t, H, nope, vd, kvr, rope, ctx, seq = Q8_0, 4, 32, 16, 64, 16, 64, 7
    case = make_case(oracle, t, H, nope, vd, kvr, rope, ctx, seed=5)
    _, olat = oracle.mla_attn_heads(case.c_kv, case.k_rope, seq, case.q_nope, case.q_rope, t, case.kv_b,
                                    H, nope, vd, case.scale)
    _, good, _ = mla64(case, seq)
    assert np.abs(olat - good).max() / np.abs(good).max() < OLAT_BOUND
    _, bad, _ = mla64(case, seq, slip)
    assert np.abs(olat - bad).max() / np.abs(bad).max() > 100 * OLAT_BOUND, slip


def test_mla_single_position_is_the_value_row(oracle):
    """At seq 1 softmax is exactly 1, so o_lat is the cached row bit for bit
    (c_acc = 0 + 1 * c_0) whatever the query."""
    case = make_case(oracle, Q8_0, 4, 32, 16, 64, 16, 8, seed=9)
    _, olat = oracle.mla_attn_heads(case.c_kv, case.k_rope, 1, case.q_nope, case.q_rope, Q8_0, case.kv_b,
                                    4, 32, 16, case.scale)
    assert np.array_equal(olat.reshape(4, 64), np.tile(case.c_kv[0], (4, 1)))


def test_rope_yarn_regimes(oracle):
    """deepseek.zig:581-613: factor <= 1 is the plain NORM rope (the same
    expressions as llama.zig's ropeNorm, bit for bit); position 0 is the
    identity; pairs below the ramp's low end rotate by pos * base^(-2i/d)
    (extrapolated), pairs above its high end by that angle / factor
    (interpolated), each pair keeps its length; with DeepSeek-V3's rope
    (64 dims, base 10000, factor 40, original context 4096) the ramp runs
    over pairs 10 .. 23."""
    rng = np.random.default_rng(3)
    v = rng.standard_normal(64).astype(np.float32)
    for pos in (0, 1, 17, 4095):
        assert np.array_equal(oracle.rope_yarn(v, pos, 10000.0, 1.0, 4096.0), oracle.rope(v, 64, pos, 10000.0, False))
    assert np.array_equal(oracle.rope_yarn(v, 0, 10000.0, 40.0, 4096.0), v)
    d, base, factor, orig = 64, 10000.0, 40.0, 4096.0
    corr = lambda beta: d * np.log(orig / (beta * 2 * np.pi)) / (2 * np.log(base))  # noqa: E731
    low, high = max(0.0, np.floor(corr(32.0))), min(d - 1.0, np.ceil(corr(1.0)))
    assert (low, high) == (10.0, 23.0)
    for pos in (1, 300, 4095):
        got = oracle.rope_yarn(v, pos, base, factor, orig).astype(np.float64)
        for i in range(d // 2):
            a, b = float(v[2 * i]), float(v[2 * i + 1])
            assert abs(np.hypot(got[2 * i], got[2 * i + 1]) - np.hypot(a, b)) < 1e-5 * (1 + np.hypot(a, b))
            theta = pos * base ** (-2 * i / d)
            if i <= low:
                ang = theta
            elif i >= high:
                ang = theta / factor
            else:
                continue
            want = (a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang))
            assert abs(got[2 * i] - want[0]) < 2e-3 and abs(got[2 * i + 1] - want[1]) < 2e-3, (pos, i)


def _q(t, v):
    """The reference's int8 activation for weight type t, dequantized."""
    import oracle as o

    v = np.ascontiguousarray(v, np.float32)
    if t in (Q4_K, Q6_K):
        d, q, _ = o.quantize_x256(v)
    else:
        d, _, q = o.quantize_x(v)
    return (q.astype(np.float64) * d.astype(np.float64)[:, None]).ravel()


def _yarn64(v, pos, base, factor, orig):
    """deepseek.zig:581-613 in float64."""
    d = len(v)
    corr = lambda beta: d * np.log(orig / (beta * 2 * np.pi)) / (2 * np.log(base))  # noqa: E731
    low, high = max(0.0, np.floor(corr(32.0))), min(d - 1.0, np.ceil(corr(1.0)))
    out = v.copy()
    for i in range(d // 2):
        te = pos * base ** (-2 * i / d)
        ramp = 1.0 - min(max((i - low) / max(0.001, high - low), 0.0), 1.0)
        th = te / factor * (1.0 - ramp) + te * ramp
        a, b = v[2 * i], v[2 * i + 1]
        out[2 * i], out[2 * i + 1] = a * np.cos(th) - b * np.sin(th), a * np.sin(th) + b * np.cos(th)
    return out


class _Step64:
    """The MLA token in float64 from the independent decoder's weights: norms,
    projections (int8 activations as the reference's matvecs quantize them),
    YaRN, attention with the keys decompressed (K = W_k c per position and
    head) and W_v applied to the softmax-weighted latent sum, residuals; the routed MoE layer through the oracle's moeRun +
    shared expert (pinned in test_oracle_moe) on the float64 stream rounded
    to f32."""

    def __init__(self, oracle, mc, stepper):
        self.o, self.mc, self.st = oracle, mc, stepper
        self.c = [[] for _ in mc.layers]
        self.r = [[] for _ in mc.layers]
        deq = lambda t, a, rows, cols: npref.dequant(t, a, rows, cols).astype(np.float64)  # noqa: E731
        H, kd = mc.n_heads, mc.nope + mc.rope
        self.W = []
        for L in mc.layers:
            w = {"wq": deq(Q4_K, L["wq"], H * kd, mc.dim), "kv_a": deq(Q4_K, L["kv_a"], mc.kvr + mc.rope, mc.dim),
                 "kv_b": deq(Q4_K, L["kv_b"], H * (mc.nope + mc.vd), mc.kvr),
                 "attn_out": deq(Q4_K, L["attn_out"], mc.dim, H * mc.vd)}
            if not L["is_moe"]:
                w["dgate"] = deq(Q4_K, L["dgate"], mc.dffn, mc.dim)
                w["dup"] = deq(Q4_K, L["dup"], mc.dffn, mc.dim)
                w["ddown"] = deq(Q6_K, L["ddown"], mc.dim, mc.dffn)
            self.W.append(w)
        self.out = deq(Q6_K, mc.output, mc.vocab, mc.dim)

    def norm(self, x, w):
        x = np.asarray(x, np.float64)
        return x / np.sqrt(np.mean(x * x) + self.mc.eps) * w.astype(np.float64)

    def step(self, x, pos):
        mc, H, nope, rope, kvr, vd = self.mc, self.mc.n_heads, self.mc.nope, self.mc.rope, self.mc.kvr, self.mc.vd
        kd = nope + rope
        x = np.asarray(x, np.float64).copy()
        for li, (L, W) in enumerate(zip(mc.layers, self.W)):
            n = self.norm(x, L["attn_norm"])
            q = W["wq"] @ _q(Q4_K, n)
            kv = W["kv_a"] @ _q(Q4_K, n)
            self.c[li].append(self.norm(kv[:kvr], L["kv_a_norm"]))
            self.r[li].append(_yarn64(kv[kvr:], pos, mc.rope_base, mc.yarn_factor, mc.yarn_orig_ctx))
            C_, R_ = np.array(self.c[li]), np.array(self.r[li])
            heads = []
            for h in range(H):
                qn = q[h * kd:h * kd + nope]
                qr = _yarn64(q[h * kd + nope:(h + 1) * kd], pos, mc.rope_base, mc.yarn_factor, mc.yarn_orig_ctx)
                Wk = W["kv_b"][h * (nope + vd):h * (nope + vd) + nope]
                Wv = W["kv_b"][h * (nope + vd) + nope:(h + 1) * (nope + vd)]
                s = ((C_ @ Wk.T) @ qn + R_ @ qr) * mc.scale
                p = np.exp(s - s.max())
                p /= p.sum()
                # o = W_v (sum_t p_t c_t): W_v is a matvec, whose input the
                # reference quantizes to int8 like every matvec's
                heads.append(Wv @ _q(Q4_K, p @ C_))
            x = x + W["attn_out"] @ _q(Q4_K, np.concatenate(heads))
            n = self.norm(x, L["ffn_norm"])
            if L["is_moe"]:
                acc, _, _ = self.o.moe_layer_token(self.st.keep[0], n.astype(np.float32))
                x = x + acc
            else:
                g, u = W["dgate"] @ _q(Q4_K, n), W["dup"] @ _q(Q4_K, n)
                x = x + W["ddown"] @ _q(Q6_K, g / (1.0 + np.exp(-g)) * u)
        return self.out @ _q(Q6_K, self.norm(x, mc.out_norm)), x


# observed without a slip: 3.9e-7 relative; the slips miss by 3.4e-2, 0.18 and 0.55.  The float64
# forward quantizes its own values at every matvec input, so a value on an int8 rounding boundary
# could round the other way than the oracle's f32 value (a ~1e-2 miss); the seed is fixed and
# shows none (seed 11 does, at position 2's W_v input of head 1)
STEP_BOUND = 1e-4


@pytest.mark.parametrize("slip", [0, 1, 2, 3], ids=["none", "k_rope_unrotated", "rope_on_nope", "no_kv_a_norm"])
def test_mla_step_against_float64(oracle, slip):
    """lo_mla_step (the MLA token mlaTokenFrame records: deepseek.zig:
    851-1048, 1275-1440) over 5 positions of a dense layer then a MoE layer
    with a shared expert, DeepSeek-V3's per-head shape and YaRN (factor 40,
    original context 4096) at position offsets where the ramp matters,
    against the float64 forward: logits and the residual stream within
    1e-4.  Each planted slip (k_rope cached before its rope, q's rope on the
    nope slice, kv_a's norm skipped) misses by far more."""
    from mla_case import MlaOracleStepper, make_mla_model

    mc = make_mla_model(oracle, 12, moe=(False, True), dim=512, n_heads=4, ctx=16, vocab=256, n_expert=8,
                        n_used=2, ffn=256, sffn=256, dffn=256)
    st = MlaOracleStepper(oracle, mc)
    ref = _Step64(oracle, mc, st)
    oracle.lib().lo_set_mla_slip(slip)
    try:
        worst = 0.0
        for pos, tok in enumerate(np.random.default_rng(4).integers(0, mc.vocab, 5)):
            x = st.embed(tok)
            x0 = x.astype(np.float64)
            logits = st.step(x, pos)
            want, x64 = ref.step(x0, pos)
            worst = max(worst, np.abs(logits - want).max() / np.abs(want).max(),
                        np.abs(x - x64).max() / np.abs(x64).max())
        if slip == 0:
            assert worst < STEP_BOUND, worst
        else:
            assert worst > 100 * STEP_BOUND, (slip, worst)
    finally:
        oracle.lib().lo_set_mla_slip(0)
