"""GPU parity of the whole-token decode frame against the oracle's restated
llama.step / decodeBatch (src/gguf/llama.zig:1111-1227, 1939-2043).

Two kinds of check:
  * per step, with the oracle's K/V cache and position reset to the device's
    before the step, so that each step compares one token's arithmetic on
    identical state: in PARITY numerics the logits are bit-identical
    (max-relative 0.0: every reduction runs in the reference's order, and
    exp is the once-rounded double exponential on both sides); FAST is
    bounded, not held to north_star's 2e-3;
  * free-running greedy decode on both sides: identical tokens (north_star:
    64 tokens at config 1).
"""
import numpy as np
import pytest

from oracle.model import OracleModel, maxrel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    import loom_amd

    loom_amd.init(0)
    from loom_amd import frame

    return frame


def _sync_oracle(dec, seqs, bufs, lane_idx=None):
    import torch

    torch.cuda.synchronize()
    lanes = range(dec.n) if lane_idx is None else lane_idx
    for i in lanes:
        bufs[2 * i][:] = dec.k_cache[i].cpu().numpy().view(np.uint8).ravel()
        bufs[2 * i + 1][:] = dec.v_cache[i].cpu().numpy().view(np.uint8).ravel()
        seqs[i].pos = int(dec.pos[i].item())


def _synced_steps(lh, om, dm, tokens, prefill=0):
    """Per-step max-rel of device vs oracle logits on identical state."""
    import torch

    dec = lh.Decoder(dm, 1)
    if prefill:
        dec.prefill_random(prefill, seed=11, scale=0.5)
    seqs, bufs = om.new_seqs(1)
    rels = []
    for tok in tokens:
        _sync_oracle(dec, seqs, bufs)
        dec.tokens.fill_(int(tok))
        dec.step()
        want = om.step(seqs[0], int(tok))
        torch.cuda.synchronize()
        rels.append(maxrel(dec.logits[0].cpu().numpy(), want))
        assert int(dec.tokens[0].item()) == int(np.argmax(want))  # sampler.argmax: first maximum
    return np.array(rels)


def _greedy(lh, om, dm, prompt, n_gen):
    """Feed `prompt`, then greedy-decode n_gen tokens on both sides, each side
    on its own state; returns (device tokens, oracle tokens)."""
    import torch

    dec = lh.Decoder(dm, 1)
    seqs, _ = om.new_seqs(1)
    dev_toks, ref_toks = [], []
    tok_ref = None
    for i in range(len(prompt) + n_gen - 1):
        if i < len(prompt):
            dec.tokens.fill_(int(prompt[i]))
            tok_ref = int(prompt[i])
        dec.step()
        want = om.step(seqs[0], tok_ref)
        tok_ref = int(np.argmax(want))
        if i >= len(prompt) - 1:
            torch.cuda.synchronize()
            dev_toks.append(int(dec.tokens[0].item()))
            ref_toks.append(tok_ref)
    return dev_toks, ref_toks


def test_stories15m_greedy_64(lh, oracle, tmp_path):
    """Config 1 at full size and by its input recipe: the stories15M shape
    (llama architecture, NORM rope, dense SwiGLU) with every matrix N(0,
    0.02) through the reference's Q4_0 rule (ggml.zig:1861), written as a
    GGUF file and loaded from it; a seeded 16-token prompt, then 64 greedy
    tokens identical to the oracle's."""
    from loom_amd import gguf
    from recipes import stories15m_gguf

    path = str(tmp_path / "stories15m.gguf")
    stories15m_gguf(path, seed=3)
    with gguf.GgufFile(path) as g:
        dm = lh.DeviceModel.from_gguf(g, ctx_len=96, keep_ggml=True)
    spec = dm.spec
    assert (spec.dim, spec.n_layers, spec.n_heads, spec.head_dim, spec.vocab) == (288, 6, 6, 48, 32000)
    om = OracleModel(oracle, dm)
    prompt = np.random.default_rng(16).integers(0, spec.vocab, 16)
    dev, ref = _greedy(lh, om, dm, prompt, 64)
    assert dev == ref


def test_stories15m_steps_parity(lh, oracle):
    spec = lh.stories15m(ctx_len=64)
    dm = lh.DeviceModel.synth(spec, seed=4, keep_ggml=True)
    om = OracleModel(oracle, dm)
    rels = _synced_steps(lh, om, dm, np.random.default_rng(2).integers(0, spec.vocab, 40))
    _check(rels, "parity")


def _qwen_small(lh, n_layers=2, vocab=4096, n_expert=16, ctx_len=80):
    return lh.qwen3_30b_a3b(ctx_len=ctx_len, n_layers=n_layers, vocab=vocab, n_expert=n_expert)


def test_qwen3moe_frame_steps_parity(lh, oracle):
    """qwen3moe architecture at the Qwen3-30B-A3B layer shapes (hidden 2048,
    GQA 32/4 x 128, QK-norm, NEOX rope, Q4_K/Q6_K mix, MoE top-8 with the
    Zipf logit bias), 2 layers, 16 experts, vocab 4096: 40 steps against
    llama.step on identical state."""
    spec = _qwen_small(lh)
    dm = lh.DeviceModel.synth(spec, seed=5, keep_ggml=True)
    om = OracleModel(oracle, dm)
    rels = _synced_steps(lh, om, dm, np.random.default_rng(4).integers(0, spec.vocab, 40))
    _check(rels, "parity")


def test_qwen3moe_frame_greedy(lh, oracle):
    spec = _qwen_small(lh)
    dm = lh.DeviceModel.synth(spec, seed=8, keep_ggml=True)
    om = OracleModel(oracle, dm)
    prompt = np.random.default_rng(9).integers(0, spec.vocab, 8)
    dev, ref = _greedy(lh, om, dm, prompt, 32)
    assert dev == ref


def _set_numerics(dm, numerics):
    from loom_amd import NUMERICS_FAST, NUMERICS_PARITY

    dm.set_numerics(NUMERICS_PARITY if numerics == "parity" else NUMERICS_FAST)


# FAST numerics (tree-summed rmsnorm, split-context attention on the matrix
# cores, hardware exp) are not the reference's order: a last-bit difference
# can move one int8 step of a quantized matvec input, which moves logits by up
# to ~1.5e-2 relative at these shapes (measured).  They are bounded here, not
# held to north_star's 2e-3; PARITY is, and is what the benchmark reports.
FAST_BOUND = 5e-2


def _check(rels, numerics):
    """PARITY: every lane-step bit-identical to the oracle.  FAST: bounded."""
    rels = np.asarray(rels)
    if numerics == "parity":
        assert rels.max() == 0.0, rels
    else:
        assert rels.max() <= FAST_BOUND, rels


@pytest.mark.parametrize("numerics", ["parity", "fast"])
def test_qwen3moe_frame_prefilled_context(lh, oracle, numerics):
    """A prefilled fp16 context (random K/V rows 0..99), then 12 steps on
    identical state: PARITY runs the reference-order attention over the whole
    context (bit-identical), FAST the split-context
    merge.  Every step's greedy token matches."""
    spec = _qwen_small(lh, ctx_len=128)
    dm = lh.DeviceModel.synth(spec, seed=6, keep_ggml=True)
    _set_numerics(dm, numerics)
    om = OracleModel(oracle, dm)
    rels = _synced_steps(lh, om, dm, np.random.default_rng(1).integers(0, spec.vocab, 12),
                         prefill=100)
    _check(rels, numerics)


def _batch_steps(lh, om, dm, n, steps, prefill, seed):
    """n lanes over a prefilled context with staggered positions (lane i at
    prefill - i % 7): per-lane logits against lo_decode_batch on identical
    state for `steps` steps, the device fed the oracle's greedy tokens.
    Returns (per lane-step max-rel, greedy tokens identical)."""
    import torch

    dec = lh.Decoder(dm, n)
    if prefill:
        dec.prefill_random(prefill, seed=seed, scale=0.5)
        dec.pos.copy_(torch.tensor([prefill - (i % 7) for i in range(n)], dtype=torch.int32))
    seqs, bufs = om.new_seqs(n)
    toks = np.random.default_rng(seed).integers(0, dm.spec.vocab, n)
    rels, same = [], True
    for _ in range(steps):
        _sync_oracle(dec, seqs, bufs)
        dec.tokens.copy_(torch.from_numpy(toks.astype(np.int32)))
        dec.step()
        want = om.step(seqs[0], int(toks[0]))[None] if n == 1 else om.decode_batch(seqs, toks)
        torch.cuda.synchronize()
        got = dec.logits.cpu().numpy()
        rels += [maxrel(got[i], want[i]) for i in range(n)]
        toks = np.argmax(want, axis=1)
        same &= bool(np.array_equal(dec.tokens.cpu().numpy(), toks.astype(np.int32)))
    return np.array(rels), same


@pytest.mark.parametrize("numerics", ["parity", "fast"])
@pytest.mark.parametrize("n", [3, 6, 16, 32])
def test_qwen3moe_frame_batch(lh, oracle, n, numerics):
    """decodeBatch semantics at n lanes (moeBatchUnion; n = 3 the few-token
    MoE path and the fused rope, n = 6 the grouped MoE and the separate rope
    launch, n >= 16 the matrix-core matmuls; FAST from 5 lanes the direct
    attention over 128-position records) over a 300-position prefilled context
    (several merge records, a partly filled last one): per-lane logits against
    lo_decode_batch over 4 steps on identical state."""
    spec = _qwen_small(lh, ctx_len=320)
    dm = lh.DeviceModel.synth(spec, seed=7, keep_ggml=True)
    _set_numerics(dm, numerics)
    om = OracleModel(oracle, dm)
    rels, same = _batch_steps(lh, om, dm, n, 4, 300, seed=n)
    _check(rels, numerics)
    if numerics == "parity":
        assert same


@pytest.mark.parametrize("heads", [(6, 6, 48), (8, 4, 64), (16, 4, 64)])
def test_llama_frame_batch_head_layouts(lh, oracle, heads):
    """PARITY at 5 lanes over a 200-position prefilled context (a whole
    128-position value tile and a partial one) for head layouts the Qwen3
    tests do not reach: 1, 2 and 4 query heads per KV head, head sizes 48
    and 64 -- the many-lane scores and P.V kernels at each work-group shape
    they take.  Per-lane logits against lo_decode_batch on identical state,
    identical greedy tokens."""
    import dataclasses

    n_heads, n_kv, hd = heads
    spec = dataclasses.replace(lh.stories15m(ctx_len=224), n_layers=2, vocab=4096, n_heads=n_heads,
                               n_kv_heads=n_kv, head_dim=hd, rope_dim=hd)
    dm = lh.DeviceModel.synth(spec, seed=21, keep_ggml=True)
    om = OracleModel(oracle, dm)
    rels, same = _batch_steps(lh, om, dm, 5, 3, 200, seed=hd + n_heads)
    print(f"heads {heads}: max-rel {rels.max():.2e}")
    _check(rels, "parity")
    assert same


@pytest.mark.parametrize("wt", [2, 8])  # Q4_0, Q8_0
@pytest.mark.parametrize("n", [16, 32])
def test_llama_frame_batch_32_block_matrix_cores(lh, oracle, wt, n):
    """A llama-architecture model 512 wide in Q4_0 or Q8_0 throughout (q, k,
    v, wo, the FFN and the head): from 16 lanes every one of its matmuls runs
    on mmq32_kernel (whole 64-value spans, 512 to 4096 columns) through the
    frame.  PARITY per-lane logits against lo_decode_batch over 3 steps on
    identical state, identical greedy tokens."""
    import dataclasses

    spec = dataclasses.replace(lh.stories15m(ctx_len=160), dim=512, n_layers=2, vocab=2048, n_heads=8,
                               n_kv_heads=4, head_dim=64, rope_dim=64, ffn=1024, embed_t=wt, output_t=wt,
                               wq_t=wt, wk_t=wt, wv_t=wt, wo_t=wt, ffn_gate_t=wt, ffn_down_t=wt)
    dm = lh.DeviceModel.synth(spec, seed=31 + wt, keep_ggml=True)
    om = OracleModel(oracle, dm)
    rels, same = _batch_steps(lh, om, dm, n, 3, 140, seed=wt + n)
    _check(rels, "parity")
    assert same


@pytest.mark.parametrize("numerics", ["parity", "fast"])
@pytest.mark.parametrize("n", [1, 32])
def test_qwen3moe_frame_4096_context(lh, oracle, n, numerics):
    """The benchmark's shape: two layers at the full Qwen3-30B-A3B layer
    shapes (128 experts top-8, vocab 4096) over a 4096-token prefilled fp16
    context, 1 lane (llama.step) and 32 lanes (decodeBatch), 3 steps on
    identical state.  PARITY: every logit bit-identical (north_star asks for
    2e-3) and identical greedy tokens -- the reference's sequential
    softmax sum and position-ordered P.V over all 4096 positions, the merge
    tail of long contexts included."""
    spec = lh.qwen3_30b_a3b(ctx_len=4096 + 16, n_layers=2, vocab=4096, n_expert=128)
    dm = lh.DeviceModel.synth(spec, seed=6, keep_ggml=True)
    _set_numerics(dm, numerics)
    om = OracleModel(oracle, dm)
    rels, same = _batch_steps(lh, om, dm, n, 3, 4096, seed=11 + n)
    print(f"{numerics} n={n}: max-rel {rels.max():.2e}, steps > 2e-3: {(rels > 2e-3).sum()}/{rels.size}")
    _check(rels, numerics)
    if numerics == "parity":
        assert same


def test_frame_declines_unserved_dims(lh):
    """Shapes outside the frame's limits decline before launching anything."""
    import loom_amd

    spec = lh.stories15m(ctx_len=8)
    dm = lh.DeviceModel.synth(spec, seed=1)
    assert dm.frame_check(1) and dm.frame_check(32)
    dm.desc.head_dim = 300  # > 256
    dec = lh.Decoder(dm, 1)
    loom_amd.take_launch_count()
    assert not dm.frame_check(1)  # gpuLayersSupported's answer at load
    assert dec.step() == loom_amd.DECLINED
    assert loom_amd.take_launch_count() == 0


@pytest.mark.parametrize("bad", ["top17", "gate_up_types", "no_router"])
def test_frame_declines_unserved_moe_layer(lh, bad):
    """A MoE layer the routed path would refuse (top-k above 16, gate and up
    of different types, no router) is caught before the frame launches
    anything: DECLINED (ERR_ARG for a missing router), no launch, no K/V row
    written."""
    import loom_amd

    spec = _qwen_small(lh, ctx_len=8)
    dm = lh.DeviceModel.synth(spec, seed=1)
    L = dm.layers[1].moe
    if bad == "top17":
        L.n_used = 17
    elif bad == "gate_up_types":
        L.up_t = loom_amd.Q6_K
    else:
        L.router = None
    dec = lh.Decoder(dm, 1)
    loom_amd.take_launch_count()
    assert not dm.frame_check(1)
    if bad == "no_router":
        with pytest.raises(loom_amd.LoomHipError):
            dec.step()
    else:
        assert dec.step() == loom_amd.DECLINED
    assert loom_amd.take_launch_count() == 0
    assert int(dec.k_cache.abs().sum().item()) == 0


@pytest.mark.parametrize("numerics", ["parity", "fast"])
@pytest.mark.parametrize("n", [1, 3, 4, 6])
def test_frame_lane_at_negative_position(lh, oracle, n, numerics):
    """A lane at position -1 (no context) among n lanes over a 200-position
    prefilled context.  Its attention is +0: no K/V row read or written, no
    softmax over an empty row, and with wo's quantization fused into the
    few-lane P.V (n <= 4) its arrival still counts, so its neighbours'
    quantized inputs complete.  The other lanes' logits are those
    lo_decode_batch gives them on their own (PARITY: bit-identical); the
    empty lane's are finite and it leaves at position 0.  n = 6 runs the
    many-lane kernels."""
    import torch

    spec = _qwen_small(lh, ctx_len=224)
    dm = lh.DeviceModel.synth(spec, seed=13, keep_ggml=True)
    _set_numerics(dm, numerics)
    om = OracleModel(oracle, dm)
    dec = lh.Decoder(dm, n)
    dec.prefill_random(200, seed=5, scale=0.5)
    neg = n // 2
    pos0 = [200 - (i % 7) for i in range(n)]
    pos0[neg] = -1
    dec.pos.copy_(torch.tensor(pos0, dtype=torch.int32))
    toks = np.random.default_rng(n).integers(0, spec.vocab, n).astype(np.int32)
    dec.tokens.copy_(torch.from_numpy(toks))
    others = [i for i in range(n) if i != neg]
    seqs, bufs = om.new_seqs(max(1, len(others)))
    torch.cuda.synchronize()
    for j, i in enumerate(others):
        bufs[2 * j][:] = dec.k_cache[i].cpu().numpy().view(np.uint8).ravel()
        bufs[2 * j + 1][:] = dec.v_cache[i].cpu().numpy().view(np.uint8).ravel()
        seqs[j].pos = pos0[i]
    k_before, v_before = dec.k_cache[neg].clone(), dec.v_cache[neg].clone()
    print(f"n={n} {numerics}: lane {neg} at position -1", flush=True)
    dec.step()
    torch.cuda.synchronize()
    got = dec.logits.cpu().numpy()
    assert torch.equal(dec.k_cache[neg], k_before) and torch.equal(dec.v_cache[neg], v_before)
    assert np.isfinite(got[neg]).all()
    assert int(dec.pos[neg].item()) == 0
    if others:
        want = om.decode_batch(seqs, toks[others])
        rels = [maxrel(got[i], want[j]) for j, i in enumerate(others)]
        if numerics == "parity":
            assert max(rels) == 0.0, rels
        else:
            assert max(rels) <= FAST_BOUND, rels


def test_parity_frame_declines_past_its_context_limit(lh):
    """PARITY attention serves contexts up to 7,936 positions (its softmax
    row and sequential sum live in LDS): a model with a longer context is
    refused at load (frame_check, gpuLayersSupported's question) and on the
    step itself before anything is launched -- no K/V row written, the
    position unchanged.  FAST numerics serve the same model."""
    import dataclasses

    import loom_amd

    spec = dataclasses.replace(lh.stories15m(ctx_len=7937), n_layers=1, vocab=512)
    dm = lh.DeviceModel.synth(spec, seed=2)
    dec = lh.Decoder(dm, 1)
    loom_amd.take_launch_count()
    assert not dm.frame_check(1)
    assert dec.step() == loom_amd.DECLINED
    assert loom_amd.take_launch_count() == 0
    assert int(dec.k_cache.abs().sum().item()) == 0 and int(dec.pos[0].item()) == 0
    _set_numerics(dm, "fast")
    assert dm.frame_check(1)
    assert dec.step() == loom_amd.OK
    assert int(dec.pos[0].item()) == 1
