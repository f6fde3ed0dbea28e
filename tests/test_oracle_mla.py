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
