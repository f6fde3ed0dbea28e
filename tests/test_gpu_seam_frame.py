"""The seam's frame calls over host buffers, as Loom's engine would make them
(src/compute/backend.zig:121-160,186-191), against the oracle's llama.step
(src/gguf/llama.zig:1111-1227) on the same host GGML bytes:

  * gqaTokenFrame (the qwen3moe form of mlaTokenFrame): the embedding row in,
    every layer and the head on the device, logits out -- bit-identical to
    llama.step -- and readKvCache's rows equal to the rows llama.step wrote
    into its cache (fp16, as the device keeps them);
  * a host-path step in between (the engine's fallback: its own cache, then
    kvAppend of the rows it wrote), after which the frame still matches bit
    for bit, so the two caches never disagree;
  * attnHeads against the host loop over the same cache;
  * the recorded dense frame of stepRecorded (beginFrame, frameLoadX,
    layerBlock per layer, endFrame, frameStoreX) on a llama model, the head
    then on the host as llama.step does it;
  * every decline happens before anything is launched.
Everything goes through the C ABI with host buffers."""
import numpy as np
import pytest

from oracle.model import OracleModel, attn_heads

pytestmark = pytest.mark.gpu

F32 = 0


@pytest.fixture(scope="module")
def lh():
    import loom_amd

    loom_amd.init(0)
    from loom_amd import backend, frame

    backend.clearWeightCache()
    yield frame, backend
    backend.releaseKvCache()
    backend.clearWeightCache()


class HostModel:
    """A device model's weights as an engine holds them: host GGML bytes and
    f32 norms, plus the oracle over the very same arrays."""

    def __init__(self, oracle, dm):
        self.dm, self.spec = dm, dm.spec
        self.om = OracleModel(oracle, dm)
        self.f = {k: np.ascontiguousarray(v.cpu().numpy(), np.float32) for k, v in dm.f32.items()}

    def w(self, be, name):
        return be.WeightRef(self.dm.tensors[name].t, self.om.host[name])

    def norm(self, name, ones):
        return self.f.get(name, self.f[ones])

    def embed_row(self, oracle, tok):
        # llama.zig:1122: the engine dequantizes the embedding row itself
        return np.ascontiguousarray(oracle.dequant_row(self.dm.tensors["embed"].t, self.om.host["embed"], int(tok),
                                                       self.spec.dim), np.float32)

    def scale(self):
        return float(np.float32(1.0) / np.sqrt(np.float32(self.spec.head_dim)))


def _gqa_descs(be, hm):
    s = hm.spec
    descs = []
    for li in range(s.n_layers):
        p = f"l{li}."
        d = be.GqaLayerDesc(attn_norm=hm.norm(p + "attn_norm", "ones_dim"), ffn_norm=hm.norm(p + "ffn_norm", "ones_dim"),
                            wq=hm.w(be, p + "wq"), wk=hm.w(be, p + "wk"), wv=hm.w(be, p + "wv"),
                            wo=hm.w(be, p + "wo"), is_moe=bool(s.n_expert))
        if s.qk_norm:
            d.q_norm, d.k_norm = hm.norm(p + "q_norm", "ones_hd"), hm.norm(p + "k_norm", "ones_hd")
        if s.n_expert:
            d.router = be.WeightRef(F32, hm.f[p + "router"].view(np.uint8).ravel())
            d.router_bias = hm.f.get(p + "router_bias")
            d.gate, d.up, d.down = (hm.w(be, p + n) for n in ("gate", "up", "down"))
            d.ffn = s.moe_ffn
        else:
            d.dgate, d.dup, d.ddown = (hm.w(be, p + n) for n in ("ffn_gate", "ffn_up", "ffn_down"))
            d.dffn = s.ffn
        descs.append(d)
    cfg = be.GqaFrameCfg(s.dim, s.n_heads, s.n_kv_heads, s.head_dim, s.rope_dim, s.eps, hm.scale(), s.rope_base,
                         s.rope_neox, be.RoutedCfg(s.n_expert, s.n_used, False, s.weights_norm, s.weights_scale)
                         if s.n_expert else None, gating=s.gating)
    return descs, cfg


def _oracle_rows(hm, bufs, li, pos):
    """Layer li's cache rows at pos in the oracle's fp16 cache, widened."""
    s = hm.spec
    kvd, i = s.kvd, (li * s.ctx_len + pos) * s.kvd
    return (bufs[0].view(np.float16)[i:i + kvd].astype(np.float32),
            bufs[1].view(np.float16)[i:i + kvd].astype(np.float32))


def _same(got, want, what):
    assert np.array_equal(np.asarray(got, np.float32).view(np.uint32), np.asarray(want, np.float32).view(np.uint32)), (
        what, float(np.abs(got - want).max()))


def test_gqa_token_frame_matches_step_with_host_steps_between(lh, oracle):
    """qwen3moe at the Qwen3-30B-A3B layer shapes (hidden 2048, GQA 32/4 x
    128, QK-norm, NEOX rope, Q4_K/Q6_K mix, 16 experts top-8 with the Zipf
    logit bias), 2 layers: 10 tokens, the 5th and 6th through the engine's
    host path (the oracle's step on the host cache, then kvAppend of every
    layer's new row).  Each frame's logits equal llama.step's bit for bit,
    each read-back row equals the row llama.step wrote, and attnHeads over
    the device cache equals the host loop over the host cache."""
    import loom_amd

    frame, be = lh
    spec = frame.qwen3_30b_a3b(ctx_len=64, n_layers=2, vocab=4096, n_expert=16)
    dm = frame.DeviceModel.synth(spec, seed=31, keep_ggml=True)
    hm = HostModel(oracle, dm)
    descs, cfg = _gqa_descs(be, hm)
    out_norm = hm.norm("out_norm", "ones_dim")
    assert be.attnInit(spec.n_layers, spec.ctx_len, spec.kvd) and be.hasKvCache()
    seqs, bufs = hm.om.new_seqs(1)
    toks = np.random.default_rng(3).integers(0, spec.vocab, 10)
    logits = np.empty(spec.vocab, np.float32)
    k, v = np.empty(spec.kvd, np.float32), np.empty(spec.kvd, np.float32)
    for pos, tok in enumerate(toks):
        x = hm.embed_row(oracle, tok)
        want = hm.om.step(seqs[0], int(tok))  # advances the oracle's cache and position
        if pos in (4, 5):  # the engine's host path: its cache, then the rows mirrored
            for li in range(spec.n_layers):
                kr, vr = _oracle_rows(hm, bufs, li, pos)
                assert be.kvAppend(li, pos, kr, vr)
            continue
        loom_amd.take_launch_count()
        assert be.gqaTokenFrame(descs, cfg, x, pos, out_norm, hm.w(be, "output"), logits)
        assert loom_amd.take_launch_count() > 0
        print(f"pos {pos}: max |diff| {float(np.abs(logits - want).max()):.2e}", flush=True)
        _same(logits, want, f"logits at {pos}")
        for li in range(spec.n_layers):
            assert be.readKvCache(li, pos, k, v)
            kr, vr = _oracle_rows(hm, bufs, li, pos)
            _same(k, kr, f"k row {li}/{pos}")
            _same(v, vr, f"v row {li}/{pos}")
    # rows of an earlier position come from the device, not the mirror
    assert be.readKvCache(1, 2, k, v)
    _same(k, _oracle_rows(hm, bufs, 1, 2)[0], "k row 1/2")
    # attnHeads (llama.zig:1162-1192) over every cached position of layer 1
    q = np.random.default_rng(8).standard_normal(spec.qd).astype(np.float32)
    out = np.empty(spec.qd, np.float32)
    pos = len(toks) - 1
    assert be.attnHeads(1, pos, q, out, spec.n_heads, spec.n_kv_heads, spec.head_dim, hm.scale())
    _same(out, attn_heads(hm.om, bufs[0], bufs[1], 1, pos, q, hm.scale()), "attnHeads")


def test_recorded_dense_frame_matches_step(lh, oracle):
    """stepRecorded (llama.zig:1067-1108) on a llama model (NORM rope, dense
    SwiGLU, Q4_0, the stories15M attention shape): beginFrame, frameLoadX of
    the embedding row, layerBlock per layer, endFrame, frameStoreX, then the
    output norm and head on the host as llama.step does them.  Logits equal
    llama.step's bit for bit over 8 tokens, and the read-back rows equal the
    rows it wrote."""
    import dataclasses

    frame, be = lh
    spec = dataclasses.replace(frame.stories15m(ctx_len=32), n_layers=3, vocab=2048)
    dm = frame.DeviceModel.synth(spec, seed=32, keep_ggml=True)
    hm = HostModel(oracle, dm)
    assert be.attnInit(spec.n_layers, spec.ctx_len, spec.kvd)
    seqs, bufs = hm.om.new_seqs(1)
    out_norm = hm.norm("out_norm", "ones_dim")
    k, v = np.empty(spec.kvd, np.float32), np.empty(spec.kvd, np.float32)
    for pos, tok in enumerate(np.random.default_rng(4).integers(0, spec.vocab, 8)):
        x = hm.embed_row(oracle, tok)
        assert be.beginFrame() and be.frameOpen()
        assert be.frameLoadX(x)
        for li in range(spec.n_layers):
            p = f"l{li}."
            s = be.LayerSpec(li, pos, hm.norm(p + "attn_norm", "ones_dim"), hm.norm(p + "ffn_norm", "ones_dim"),
                             spec.eps, *(hm.w(be, p + n) for n in ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up",
                                                                   "ffn_down")),
                             spec.dim, spec.ffn, spec.n_heads, spec.n_kv_heads, spec.head_dim, spec.rope_dim,
                             spec.rope_base, spec.rope_neox, hm.scale())
            assert be.layerBlock(s)
        be.endFrame()
        assert not be.frameOpen()
        assert be.frameStoreX(x)
        normed = oracle.rmsnorm(x, out_norm, spec.eps)
        logits = oracle.matvec(hm.dm.tensors["output"].t, hm.om.host["output"], normed, spec.vocab, spec.dim)
        want = hm.om.step(seqs[0], int(tok))
        _same(logits, want, f"logits at {pos}")
        for li in range(spec.n_layers):
            assert be.readKvCache(li, pos, k, v)
            kr, vr = _oracle_rows(hm, bufs, li, pos)
            _same(k, kr, f"k row {li}/{pos}")
            _same(v, vr, f"v row {li}/{pos}")


def test_seam_frame_declines_before_launching(lh, oracle):
    """The decline rules, each before anything is launched: a context past
    the PARITY attention's 7,936 positions, a layer whose weight length does
    not match its shape, a frame call without an open frame, a token frame
    whose head does not match the vocabulary, a device cache of other dims."""
    import dataclasses

    import loom_amd

    frame, be = lh
    spec = dataclasses.replace(frame.stories15m(ctx_len=16), n_layers=2, vocab=512)
    dm = frame.DeviceModel.synth(spec, seed=33, keep_ggml=True)
    hm = HostModel(oracle, dm)
    loom_amd.take_launch_count()
    assert not be.attnInit(spec.n_layers, 7937, spec.kvd)
    assert be.attnInit(spec.n_layers, spec.ctx_len, spec.kvd)
    p = "l0."
    good = be.LayerSpec(0, 0, hm.norm(p + "attn_norm", "ones_dim"), hm.norm(p + "ffn_norm", "ones_dim"), spec.eps,
                        *(hm.w(be, p + n) for n in ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down")),
                        spec.dim, spec.ffn, spec.n_heads, spec.n_kv_heads, spec.head_dim, spec.rope_dim,
                        spec.rope_base, spec.rope_neox, hm.scale())
    x = hm.embed_row(oracle, 1)
    assert not be.layerBlock(good)  # no open frame
    assert be.beginFrame() and be.frameLoadX(x)
    short = dataclasses.replace(good, wq=be.WeightRef(good.wq.ty, good.wq.data[:-18]))
    assert not be.layerBlock(short)
    assert not be.layerBlock(dataclasses.replace(good, li=spec.n_layers))  # past the cache
    assert not be.layerBlock(dataclasses.replace(good, n_kv_heads=2))      # another kv width
    be.endFrame()
    descs, cfg = _gqa_descs(be, hm)
    logits = np.empty(spec.vocab + 1, np.float32)
    assert not be.gqaTokenFrame(descs, cfg, x, 0, hm.norm("out_norm", "ones_dim"), hm.w(be, "output"), logits)
    logits = np.empty(spec.vocab, np.float32)
    assert not be.gqaTokenFrame(descs[:1], cfg, x, 0, hm.norm("out_norm", "ones_dim"), hm.w(be, "output"), logits)
    assert loom_amd.take_launch_count() == 0
    assert be.gqaTokenFrame(descs, cfg, x, 0, hm.norm("out_norm", "ones_dim"), hm.w(be, "output"), logits)
    assert loom_amd.take_launch_count() > 0
