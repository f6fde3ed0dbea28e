"""MLA attention on the device (loom_amd/csrc/mla.hip) against the oracle's
host head loop (oracle/mla_ref.c, deepseek.zig:988-1047): the compressed
output o and the head outputs bit-identical, through the seam (mlaInit /
mlaAppend / mlaAttnHeads, the reference's own device-test layout of
vulkan/backend.zig:1432-1546: layer 1 of 2 with decoy rows in layer 0) and
through the device-resident entry point at config 5's per-head shape
(DeepSeek-V3: 128 heads, nope 128, rope 64, kv_lora 512, v 128) up to a
4096-position context."""
import numpy as np
import pytest

from mla_case import make_case

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K, F32 = 2, 8, 12, 14, 0


@pytest.fixture(scope="module")
def lh():
    import loom_amd
    from loom_amd import backend

    loom_amd.init(0)
    return backend


def _vulkan_kvb(rng, n_heads, stride, kvr):
    """The reference test's kv_b: random Q8_0 bytes with every block's d set
    to 0x2C00 (0.0625), vulkan/backend.zig:1459-1463."""
    from oracle import row_bytes

    kvb = rng.integers(0, 256, n_heads * stride * row_bytes(Q8_0, kvr), dtype=np.uint8)
    kvb.reshape(-1, 34)[:, 0] = 0x00
    kvb.reshape(-1, 34)[:, 1] = 0x2C
    return kvb


def test_seam_mla_attn_heads_matches_the_host_loop(lh, oracle):
    """mlaInit(2 layers) / mlaAppend (decoys in layer 0) / mlaAttnHeads at
    layer 1: out bit-identical to the oracle; mlaReadCache returns the rows;
    mlaSetWk in order only; one launch count moved."""
    import loom_amd

    n_heads, nope, vd, kvr, rope, ctx, seq, li, scale = 4, 32, 16, 64, 16, 64, 5, 1, 0.25
    rng = np.random.default_rng(0x1207A)
    kvb = _vulkan_kvb(rng, n_heads, nope + vd, kvr)
    assert lh.mlaInit(2, ctx, kvr, rope)
    assert lh.hasMlaCache()
    assert lh.mlaSetWk(0, np.zeros(8, np.float32)) and lh.mlaSetWk(1, np.zeros(8, np.float32))
    assert not lh.mlaSetWk(3, np.zeros(8, np.float32))  # out of order: declined
    c_rows = ((rng.random((seq, kvr)) - 0.5) * 2).astype(np.float32)
    r_rows = ((rng.random((seq, rope)) - 0.5) * 2).astype(np.float32)
    for t in range(seq):
        assert lh.mlaAppend(0, t, ((rng.random(kvr) - 0.5) * 2).astype(np.float32),
                            ((rng.random(rope) - 0.5) * 2).astype(np.float32))
        assert lh.mlaAppend(li, t, c_rows[t], r_rows[t])
    assert not lh.mlaAppend(li, 0, c_rows[0][:-1], r_rows[0])  # wrong length: declined
    back_c, back_r = np.empty(kvr, np.float32), np.empty(rope, np.float32)
    assert lh.mlaReadCache(li, 3, back_c, back_r)
    assert np.array_equal(back_c, c_rows[3]) and np.array_equal(back_r, r_rows[3])
    q_nope = ((rng.random(n_heads * nope) - 0.5) * 2).astype(np.float32)
    q_rope = ((rng.random(n_heads * rope) - 0.5) * 2).astype(np.float32)
    got = np.full(n_heads * vd, np.nan, np.float32)
    loom_amd.take_launch_count()
    assert lh.mlaAttnHeads(li, seq - 1, q_nope, q_rope, lh.WeightRef(Q8_0, kvb), got, n_heads, nope, vd, scale)
    assert loom_amd.take_launch_count() > 0
    want, _ = oracle.mla_attn_heads(c_rows, r_rows, seq, q_nope, q_rope, Q8_0, kvb, n_heads, nope, vd, scale)
    assert np.array_equal(got, want), np.abs(got - want).max()
    # the same call again (kv_b split cached) and past the cache: declined
    assert lh.mlaAttnHeads(li, seq - 1, q_nope, q_rope, lh.WeightRef(Q8_0, kvb), got, n_heads, nope, vd, scale)
    assert np.array_equal(got, want)
    assert not lh.mlaAttnHeads(li, ctx, q_nope, q_rope, lh.WeightRef(Q8_0, kvb), got, n_heads, nope, vd, scale)
    assert not lh.mlaAttnHeads(li, 2, q_nope[:-1], q_rope, lh.WeightRef(Q8_0, kvb), got, n_heads, nope, vd, scale)
    f32 = lh.WeightRef(F32, np.zeros(n_heads * (nope + vd) * kvr * 4, np.uint8))
    assert not lh.mlaAttnHeads(li, 2, q_nope, q_rope, f32, got, n_heads, nope, vd, scale)
    assert not lh.mlaInit(2, 8192, kvr, rope)  # past the exact softmax's context: declined


CASES = [
    # (type, heads, nope, vd, kvr, rope, seqs)
    (Q4_K, 128, 128, 128, 512, 64, (1, 17, 300, 4096)),  # config 5's MLA shape
    (Q6_K, 128, 128, 128, 512, 64, (301,)),
    (Q8_0, 20, 32, 16, 96, 20, (1, 7, 65)),  # heads past a 32-tile, a 3-step kvr, a rope tail of 4
    (Q4_0, 36, 16, 24, 64, 16, (33, 130)),
]


@pytest.mark.parametrize("t,H,nope,vd,kvr,rope,seqs", CASES, ids=["q4_k_cfg5", "q6_k_cfg5", "q8_0_ragged", "q4_0"])
def test_device_mla_attention_is_bit_identical(lh, oracle, t, H, nope, vd, kvr, rope, seqs):
    import torch

    ctx = max(seqs)
    case = make_case(oracle, t, H, nope, vd, kvr, rope, ctx, seed=H * 7 + kvr + t)
    kvb_dev = torch.from_numpy(case.kv_b).cuda()
    mla = lh.MlaAttn(t, kvb_dev, H, nope, vd, kvr, rope, case.scale)
    c = torch.from_numpy(case.c_kv).cuda()
    r = torch.from_numpy(case.k_rope).cuda()
    qn = torch.from_numpy(case.q_nope).cuda()
    qr = torch.from_numpy(case.q_rope).cuda()
    out = torch.full((H * vd,), float("nan"), device="cuda")
    olat = torch.full((H * kvr,), float("nan"), device="cuda")
    for seq in seqs:
        print(f"mla t={t} H={H} kvr={kvr} rope={rope} seq={seq}", flush=True)
        mla(c, r, seq, qn, qr, out, olat)
        want, want_lat = oracle.mla_attn_heads(case.c_kv, case.k_rope, seq, case.q_nope, case.q_rope, t, case.kv_b,
                                               H, nope, vd, case.scale)
        torch.cuda.synchronize()
        got_lat = olat.cpu().numpy()
        assert np.array_equal(got_lat, want_lat), (seq, np.abs(got_lat - want_lat).max())
        got = out.cpu().numpy()
        assert np.array_equal(got, want), (seq, np.abs(got - want).max())


def test_seam_mla_layer_tail_matches_the_engine_sequence(lh, oracle):
    """mlaLayerTail (src/compute/cpu.zig:63) on a DeepSeek-V3-shaped layer at
    reduced width (dim 1024, 16 heads of nope 128 / rope 64 / v 128, kv_lora
    512; 16 experts top-4 of ffn 256 with sigmoid gating, exp_probs_b as the
    selection bias, renormalised gates scaled by 2.5, a shared expert of ffn
    512; Q4_K, Q6_K down): x after the layer is bit-identical to the engine's
    own sequence run by the oracle -- the head loop, matvec(attn_output) and
    the residual add, rmsnorm, moeLayer with the shared expert, the second
    residual add (deepseek.zig:1044-1046, 1325-1387) -- and a second call
    with the kv_b split cached matches again."""
    import loom_amd
    from recipes import planes

    dim, H, nope, vd, kvr, rope, ctx, seq = 1024, 16, 128, 128, 512, 64, 64, 37
    E, k, ffn, sffn = 16, 4, 256, 512
    case = make_case(oracle, Q4_K, H, nope, vd, kvr, rope, ctx, seed=41)
    rng = np.random.default_rng(42)
    attn_out = planes(Q4_K, dim, H * vd, 1, 51)
    gate, up, down = planes(Q4_K, ffn, dim, E, 52), planes(Q4_K, ffn, dim, E, 53), planes(Q6_K, dim, ffn, E, 54)
    sg, su, sd = planes(Q4_K, sffn, dim, 1, 55), planes(Q4_K, sffn, dim, 1, 56), planes(Q6_K, dim, sffn, 1, 57)
    router = (rng.standard_normal((E, dim)) / np.sqrt(dim)).astype(np.float32)
    sel_bias = (0.1 * rng.standard_normal(E)).astype(np.float32)
    ffn_norm = (1.0 + 0.05 * rng.standard_normal(dim)).astype(np.float32)
    x0 = rng.standard_normal(dim).astype(np.float32)
    eps = 1e-6
    assert lh.mlaInit(1, ctx, kvr, rope)
    for t in range(seq):
        assert lh.mlaAppend(0, t, case.c_kv[t], case.k_rope[t])
    cfg = lh.RoutedCfg(E, k, True, True, 2.5)
    WR = lh.WeightRef
    args = (case.q_nope, case.q_rope, WR(Q4_K, case.kv_b), WR(Q4_K, attn_out), ffn_norm, eps,
            WR(F32, router.view(np.uint8).ravel()), sel_bias, WR(Q4_K, gate), WR(Q4_K, up), WR(Q6_K, down),
            (WR(Q4_K, sg), WR(Q4_K, su), WR(Q6_K, sd)), ffn, sffn, cfg, H, nope, vd, case.scale)
    # the engine's sequence on the oracle
    heads, _ = oracle.mla_attn_heads(case.c_kv, case.k_rope, seq, case.q_nope, case.q_rope, Q4_K, case.kv_b, H,
                                     nope, vd, case.scale)
    x1 = x0 + oracle.matvec(Q4_K, attn_out, heads, dim, H * vd)
    normed = oracle.rmsnorm(x1, ffn_norm, eps)
    w = oracle.MoeWeights(dim, ffn, E, k, router, gate, up, down, Q4_K, Q4_K, Q6_K, sel_bias=sel_bias,
                          gating=oracle.GATING_SIGMOID, weights_norm=True, weights_scale=2.5,
                          shexp=(sg, su, sd, Q4_K, Q4_K, Q6_K, sffn))
    acc, _, _ = oracle.moe_layer_token(w, normed)
    want = x1 + acc
    for _ in range(2):
        x = x0.copy()
        loom_amd.take_launch_count()
        assert lh.mlaLayerTail(0, seq - 1, x, *args), loom_amd.last_error()
        assert loom_amd.take_launch_count() > 0
        assert np.array_equal(x, want), np.abs(x - want).max()
    # declines: a quantized router, a position past the cache
    x = x0.copy()
    bad = list(args)
    bad[6] = WR(Q4_K, planes(Q4_K, E, dim, 1, 58))
    assert not lh.mlaLayerTail(0, seq - 1, x, *bad)
    assert not lh.mlaLayerTail(0, ctx, x, *args)
    assert np.array_equal(x, x0)


def _mla_descs(lh, mc):
    """MlaLayerDesc per layer over the model case's host arrays."""
    WR = lh.WeightRef
    ty = lambda k: mc.types.get(k, Q4_K)  # noqa: E731
    descs = []
    for L in mc.layers:
        d = lh.MlaLayerDesc(L["attn_norm"], WR(Q4_K, L["wq"]), WR(Q4_K, L["kv_a"]), L["kv_a_norm"], WR(Q4_K, L["kv_b"]),
                            WR(Q4_K, L["attn_out"]), L["ffn_norm"], bool(L["is_moe"]))
        if L["is_moe"]:
            d.router = WR(F32, L["router"].view(np.uint8).ravel())
            d.gate, d.up, d.down = WR(Q4_K, L["gate"]), WR(Q4_K, L["up"]), WR(ty("down"), L["down"])
            d.shexp = (WR(Q4_K, L["sg"]), WR(Q4_K, L["su"]), WR(ty("sd"), L["sd"]))
            d.ffn, d.shexp_ffn = mc.ffn, mc.sffn
        else:
            d.dgate, d.dup, d.ddown = WR(Q4_K, L["dgate"]), WR(Q4_K, L["dup"]), WR(ty("ddown"), L["ddown"])
            d.dffn = mc.dffn
        descs.append(d)
    cfg = lh.MlaFrameCfg(mc.dim, mc.n_heads, mc.nope, mc.rope, mc.kvr, mc.vd, mc.eps, mc.scale, mc.rope_base,
                         mc.yarn_factor, mc.yarn_orig_ctx, lh.RoutedCfg(mc.n_expert, mc.n_used, True, True, mc.wscale))
    return descs, cfg


def test_mla_token_frame_matches_the_engine_step(lh, oracle):
    """mlaTokenFrame (src/compute/backend.zig:186-191) on a DeepSeek-V3-style
    model at reduced width (dim 1024, 8 heads of nope 128 / rope 64 / v 128,
    kv_lora 512, YaRN factor 40 over an original 4096 context; a dense layer,
    then a MoE layer of 8 experts top-2 with sigmoid gating, renorm, scale
    2.5 and a shared expert; Q4_K with Q6_K downs and head): over 10 tokens,
    the 5th and 6th through the engine's host path (the oracle's step, its
    cache rows mirrored in by mlaAppend), every frame's logits and residual
    stream bit-identical to the engine's own step (lo_mla_step, pinned by a
    float64 forward), and mlaReadCache's rows equal to the rows the step
    wrote -- the device YaRN rope and head projections included."""
    import loom_amd
    from mla_case import MlaOracleStepper, make_mla_model

    mc = make_mla_model(oracle, 21, moe=(False, True), ctx=32)
    st = MlaOracleStepper(oracle, mc)
    descs, cfg = _mla_descs(lh, mc)
    lh.clearWeightCache()
    assert lh.mlaInit(len(mc.layers), mc.ctx, mc.kvr, mc.rope)
    logits = np.empty(mc.vocab, np.float32)
    c_row, r_row = np.empty(mc.kvr, np.float32), np.empty(mc.rope, np.float32)
    head = lh.WeightRef(Q6_K, mc.output)
    for pos, tok in enumerate(np.random.default_rng(5).integers(0, mc.vocab, 10)):
        x_ref = st.embed(tok)
        x = x_ref.copy()
        want = st.step(x_ref, pos)
        if pos in (4, 5):  # the engine's host path, its rows mirrored onto the device
            for li in range(len(mc.layers)):
                assert lh.mlaAppend(li, pos, st.c_kv[li, pos], st.k_rope[li, pos])
            continue
        loom_amd.take_launch_count()
        assert lh.mlaTokenFrame(descs, cfg, x, pos, mc.out_norm, head, logits), loom_amd.last_error()
        assert loom_amd.take_launch_count() > 0
        print(f"pos {pos}: max |diff| logits {float(np.abs(logits - want).max()):.2e}, "
              f"x {float(np.abs(x - x_ref).max()):.2e}", flush=True)
        assert np.array_equal(logits.view(np.uint32), want.view(np.uint32)), pos
        assert np.array_equal(x.view(np.uint32), x_ref.view(np.uint32)), pos
        for li in range(len(mc.layers)):
            assert lh.mlaReadCache(li, pos, c_row, r_row)
            assert np.array_equal(c_row, st.c_kv[li, pos]) and np.array_equal(r_row, st.k_rope[li, pos]), (li, pos)
    # declines before anything runs: a weight of the wrong length, a position past the cache
    import dataclasses
    bad = [dataclasses.replace(descs[0], wq=lh.WeightRef(Q4_K, mc.layers[0]["wq"][:-144]))] + descs[1:]
    loom_amd.take_launch_count()
    assert not lh.mlaTokenFrame(bad, cfg, st.embed(1), 10, mc.out_norm, head, logits)
    assert not lh.mlaTokenFrame(descs, cfg, st.embed(1), mc.ctx, mc.out_norm, head, logits)
    assert loom_amd.take_launch_count() == 0
    lh.clearWeightCache()
