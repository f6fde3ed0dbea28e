"""A GGUF file through the device and the oracle side by side: a fixture in
writeMoeFixture's layout (src/gguf/gguf.zig:643-912) carrying quantized
weights, written by libloomhip's writer, parsed by its reader, loaded by
DeviceModel.from_gguf (the frame's llama.zig:335-420 load) and stepped by
the frame, against the oracle's llama.step over the very bytes the file
holds.  The weights follow the configs' input recipe: N(0, 0.02) values
through the oracle's quantizers (GGUF's Q4_K/Q6_K rules for the Q4_K_M mix,
the reference's Q4_0 rule of ggml.zig:1861 for the all-Q4_0 model); norms
near 1 and the router N(0, 1/sqrt(dim)) as f32."""
import numpy as np
import pytest

from loom_amd import gguf
from oracle.model import OracleModel, maxrel

pytestmark = pytest.mark.gpu

Q4_0, Q4_K, Q6_K = 2, 12, 14


@pytest.fixture(scope="module")
def lh():
    import loom_amd

    loom_amd.init(0)
    from loom_amd import frame

    return frame


def _fill(oracle, seed, types, dim):
    """Each tensor's bytes: matrices N(0, 0.02) quantized row by row (experts
    plane by plane), norms 1 + N(0, 0.05), routers N(0, 1/sqrt(dim))."""
    rng = np.random.default_rng(seed)

    def fill(name, dims):
        n = int(np.prod(dims))
        if len(dims) == 1:
            return 0, (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)
        if name.endswith("ffn_gate_inp.weight"):
            return 0, (rng.standard_normal(n) / np.sqrt(dim)).astype(np.float32)
        t = types(name)
        cols, rows = dims[0], dims[1]
        planes = dims[2] if len(dims) == 3 else 1
        w = (0.02 * rng.standard_normal((planes * rows, cols))).astype(np.float32)
        return t, np.concatenate([oracle.quantize(t, w[p * rows:(p + 1) * rows]) for p in range(planes)])

    return fill


def _q4km(name):  # the Q4_K_M mix of config 4: Q6_K for attn_v, ffn_down and the output
    return Q6_K if any(k in name for k in ("attn_v.", "ffn_down", "output.weight")) else Q4_K


CASES = {
    # qwen3moe at frame-served shapes: GQA 4/2 x 64, QK-norm, NEOX rope, 8 experts top-2, Q4_K_M
    "qwen3moe": (gguf.FixtureShape(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, n_expert=8,
                                   n_used=2, moe_ffn=256, n_layers=2, vocab_bytes=False, vocab=512,
                                   context_length=96), _q4km),
    # llama (the fixture's MoE llama) at the stories15M attention shape, all Q4_0 (config 1's type)
    "llama": (gguf.FixtureShape(dim=288, n_heads=6, n_kv_heads=6, head_dim=48, ffn=768, n_expert=8,
                                n_used=2, moe_ffn=96, n_layers=2, vocab_bytes=False, vocab=512,
                                context_length=96), lambda name: Q4_0),
}


@pytest.mark.parametrize("arch", sorted(CASES))
def test_gguf_file_decodes_as_the_oracle(lh, oracle, tmp_path, arch):
    """The file's tensors reach the device bit for bit (the oracle reads the
    same bytes back from the device copies), the frame serves the model
    (frame_check), and 24 PARITY decode steps on identical state give the
    oracle's logits bit-identically, with its greedy token each step."""
    import torch

    shape, types = CASES[arch]
    path = tmp_path / f"{arch}.gguf"
    gguf.write_moe_fixture(str(path), 11, arch, shape=shape, fill=_fill(oracle, 5, types, shape.dim))
    with gguf.GgufFile(str(path)) as g:
        dm = lh.DeviceModel.from_gguf(g, keep_ggml=True)
        s = dm.spec
        assert (s.dim, s.head_dim, s.n_layers, s.n_expert, s.n_used) == (shape.dim, shape.head_dim, 2, 8, 2)
        assert s.rope_neox == (arch == "qwen3moe") and s.qk_norm == (arch == "qwen3moe")
        # the device's GGML copies are the file's bytes
        for key, name in (("embed", "token_embd.weight"), ("l1.down", "blk.1.ffn_down_exps.weight"),
                          ("l0.wv", "blk.0.attn_v.weight")):
            assert np.array_equal(dm.tensors[key].ggml.cpu().numpy(), g.find_tensor(name).data)
        assert np.array_equal(dm.f32["l1.attn_norm"].cpu().numpy(), g.find_tensor("blk.1.attn_norm.weight").data.view(np.float32))
    assert dm.frame_check(1)
    om = OracleModel(oracle, dm)
    dec = lh.Decoder(dm, 1)
    seqs, bufs = om.new_seqs(1)
    rels = []
    for tok in np.random.default_rng(3).integers(0, s.vocab, 24):
        torch.cuda.synchronize()
        bufs[0][:] = dec.k_cache[0].cpu().numpy().view(np.uint8).ravel()
        bufs[1][:] = dec.v_cache[0].cpu().numpy().view(np.uint8).ravel()
        seqs[0].pos = int(dec.pos[0].item())
        dec.tokens.fill_(int(tok))
        dec.step()
        want = om.step(seqs[0], int(tok))
        torch.cuda.synchronize()
        rels.append(maxrel(dec.logits[0].cpu().numpy(), want))
        assert int(dec.tokens[0].item()) == int(np.argmax(want))
    assert max(rels) == 0.0, rels
