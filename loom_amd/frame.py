"""Whole-token decode on the device: the model held in HBM and the frame
call (``loomhip_token_frame_dev``) that runs one decode step for n lanes.

This is the host mirror of the reference's model/frame seam
(src/gguf/llama.zig step 1111-1227 and decodeBatch 1939-2043 behind
src/compute/backend.zig:141-191): ``ModelSpec`` names the shapes and GGML
types of a llama- or qwen3moe-architecture model, ``DeviceModel`` holds its
tensors in the device layout, and ``Decoder`` owns the per-lane state (fp16
K/V caches, positions, tokens, logits) and steps it.  Synthetic weights are
generated on the device (seeded, GGML block layout, then repacked), which is
how the benchmark builds the 17 GB Qwen3-30B-A3B-shaped model without a
checkpoint.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import (GATING_SIGMOID, GATING_SOFTMAX, NUMERICS_PARITY, Q4_0, Q4_K, Q6_K, Q8_0, LayerDesc,
               ModelDesc, MoeLayerDesc, check, ggml_bytes, lib, OK)
from .backend import _ptr, _stream, repack_dev, synth_ggml_dev


@dataclass
class ModelSpec:
    dim: int
    head_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    ctx_len: int
    rope_dim: int
    rope_base: float
    eps: float
    rope_neox: bool
    qk_norm: bool
    embed_t: int
    output_t: int
    wq_t: int
    wk_t: int
    wv_t: int
    wo_t: int
    # dense SwiGLU FFN (n_expert == 0)
    ffn: int = 0
    ffn_gate_t: int = Q4_0
    ffn_down_t: int = Q4_0
    # routed MoE (n_expert > 0)
    n_expert: int = 0
    n_used: int = 0
    moe_ffn: int = 0
    moe_gate_t: int = Q4_K
    moe_down_t: int = Q6_K
    router_bias: bool = False
    gating: int = GATING_SOFTMAX
    weights_norm: bool = True
    weights_scale: float = 1.0
    std: float = 0.02

    @property
    def qd(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kvd(self) -> int:
        return self.n_kv_heads * self.head_dim


def stories15m(ctx_len: int = 256) -> ModelSpec:
    """Config 1: the stories15M shape, llama architecture, Q4_0 throughout."""
    return ModelSpec(dim=288, head_dim=48, n_layers=6, n_heads=6, n_kv_heads=6, vocab=32000,
                     ctx_len=ctx_len, rope_dim=48, rope_base=10000.0, eps=1e-5, rope_neox=False,
                     qk_norm=False, embed_t=Q4_0, output_t=Q4_0, wq_t=Q4_0, wk_t=Q4_0, wv_t=Q4_0,
                     wo_t=Q4_0, ffn=768, ffn_gate_t=Q4_0, ffn_down_t=Q4_0)


def qwen3_30b_a3b(ctx_len: int = 4160, n_layers: int = 48, vocab: int = 151936,
                  n_expert: int = 128) -> ModelSpec:
    """Config 4: the Qwen3-30B-A3B shape (GQA 32/4, head_dim 128, QK-norm,
    NEOX rope, 128 experts top-8 of ffn 768), Q4_K_M mix: Q4_K with Q6_K for
    attn_v, ffn_down and output."""
    return ModelSpec(dim=2048, head_dim=128, n_layers=n_layers, n_heads=32, n_kv_heads=4,
                     vocab=vocab, ctx_len=ctx_len, rope_dim=128, rope_base=1000000.0, eps=1e-6,
                     rope_neox=True, qk_norm=True, embed_t=Q4_K, output_t=Q6_K, wq_t=Q4_K,
                     wk_t=Q4_K, wv_t=Q6_K, wo_t=Q4_K, n_expert=n_expert, n_used=8, moe_ffn=768,
                     moe_gate_t=Q4_K, moe_down_t=Q6_K, router_bias=True)


@dataclass
class _Tensor:
    t: int
    rows: int
    cols: int
    planes: int
    dev: object               # device layout (torch uint8)
    ggml: object = None       # GGML bytes on the device, when kept


class DeviceModel:
    """A model's tensors in HBM plus its ``loomhip_model`` descriptor."""

    def __init__(self, spec: ModelSpec):
        self.spec = spec
        self.tensors: dict[str, _Tensor] = {}
        self.f32: dict[str, object] = {}
        self.numerics = NUMERICS_PARITY

    def set_numerics(self, mode: int) -> None:
        """NUMERICS_PARITY (sequential rmsnorm sums, bit-identical steps) or
        NUMERICS_FAST (tree sums)."""
        self.numerics = mode
        self.desc.numerics = mode

    def frame_check(self, n: int = 1) -> bool:
        """gpuLayersSupported (src/gguf/llama.zig:985-1009) for the HIP arm:
        True when the frame serves this model at n lanes -- the checks the
        frame call makes before launching anything, asked once at load."""
        rc = lib().loomhip_frame_check(C.byref(self.desc), n)
        return rc == OK

    # ---- construction ----------------------------------------------------
    @classmethod
    def synth(cls, spec: ModelSpec, seed: int = 1, keep_ggml: bool = False) -> "DeviceModel":
        """Seeded synthetic weights: GGML blocks from the device generator,
        norms = 1, router N(0, 1/sqrt(dim)) plus a Zipf(1.1) logit bias."""
        import torch

        m = cls(spec)
        s = spec
        counter = [seed * 1000]

        def q(name, t, rows, cols, planes=1):
            counter[0] += 1
            g = synth_ggml_dev(t, rows, cols, planes, counter[0], s.std)
            dev = repack_dev(t, g, rows, cols, planes)
            m.tensors[name] = _Tensor(t, rows, cols, planes, dev, g if keep_ggml else None)
            if not keep_ggml:
                del g

        ones = torch.ones(s.dim, dtype=torch.float32, device="cuda")
        m.f32["ones_dim"] = ones
        m.f32["ones_hd"] = torch.ones(s.head_dim, dtype=torch.float32, device="cuda")
        q("embed", s.embed_t, s.vocab, s.dim)
        q("output", s.output_t, s.vocab, s.dim)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        for li in range(s.n_layers):
            p = f"l{li}."
            q(p + "wq", s.wq_t, s.qd, s.dim)
            q(p + "wk", s.wk_t, s.kvd, s.dim)
            q(p + "wv", s.wv_t, s.kvd, s.dim)
            q(p + "wo", s.wo_t, s.dim, s.qd)
            if s.n_expert:
                q(p + "gate", s.moe_gate_t, s.moe_ffn, s.dim, s.n_expert)
                q(p + "up", s.moe_gate_t, s.moe_ffn, s.dim, s.n_expert)
                q(p + "down", s.moe_down_t, s.dim, s.moe_ffn, s.n_expert)
                m.f32[p + "router"] = (torch.randn(s.n_expert, s.dim, generator=gen, device="cuda")
                                       / np.sqrt(s.dim)).contiguous()
                if s.router_bias:
                    ranks = torch.randperm(s.n_expert, generator=gen, device="cuda").float() + 1
                    z = -1.1 * torch.log(ranks)
                    m.f32[p + "router_bias"] = (z - z.mean()).contiguous()
            else:
                q(p + "ffn_gate", s.ffn_gate_t, s.ffn, s.dim)
                q(p + "ffn_up", s.ffn_gate_t, s.ffn, s.dim)
                q(p + "ffn_down", s.ffn_down_t, s.dim, s.ffn)
        m._build_desc()
        return m

    @classmethod
    def from_gguf(cls, g, ctx_len: int | None = None, keep_ggml: bool = False) -> "DeviceModel":
        """llama.zig:335-420 load, for the architectures the frame serves
        (llama: NORM rope; qwen3moe: NEOX rope and per-head q/k RMSNorm),
        from a loom_amd.gguf.GgufFile: the configuration from the metadata
        with load's defaults, every matrix's GGML bytes uploaded and
        repacked to the device layout (each layer keeps its own types), the
        norms, routers and selection bias as f32 (routeCfgFromMeta,
        src/gguf/moe.zig:63-97, for the gating)."""
        import torch

        arch = g.get_string("general.architecture")
        if arch not in ("llama", "qwen3moe"):
            raise ValueError(f"UnsupportedArchitecture: {arch} (the frame serves llama and qwen3moe)")

        def u(key, default=None):
            v = g.get_uint(f"{arch}.{key}")
            return default if v is None else int(v)

        def fl(key, default):
            v = g.get_float(f"{arch}.{key}")
            return default if v is None else float(v)

        dim, n_heads = u("embedding_length"), u("attention.head_count")
        if not dim or not n_heads:
            raise ValueError("BadConfig: embedding_length / attention.head_count")
        head_dim = u("attention.key_length", dim // n_heads)
        n_layers = u("block_count") - u("nextn_predict_layers", 0)
        n_expert, n_used = u("expert_count", 0), u("expert_used_count", 0)
        ffn = u("feed_forward_length", 0)
        moe_ffn = u("expert_feed_forward_length", 0) or (ffn // n_used if n_expert and n_used else 0)
        norm = g.get_bool(f"{arch}.expert_weights_norm")

        def tensor(name):
            t = g.find_tensor(name)
            if t is None:
                raise ValueError(f"missing tensor {name}")
            return t

        # llama.zig:316-334 validateConfig: metadata that would divide by zero
        # or break an index bound is rejected before any tensor is read
        n_kv = u("attention.head_count_kv", n_heads)
        ctx = ctx_len or u("context_length", 2048)
        rope_dim = u("rope.dimension_count", head_dim)
        if (not head_dim or not n_layers or n_layers < 0 or not ctx or not n_kv or n_heads % n_kv
                or rope_dim > head_dim or n_used > 16 or n_expert > 256 or (n_expert and n_used > n_expert)
                or (n_expert and (not n_used or not moe_ffn)) or (not n_expert and not ffn)):
            raise ValueError("BadConfig: the model's metadata is inconsistent")

        embd = tensor("token_embd.weight")
        if len(embd.dims) < 2:
            raise ValueError(f"BadTensorShape: tensor {embd.name} has shape {list(embd.dims)}")
        out = g.find_tensor("output.weight") or embd  # tied embeddings
        first_moe = tensor("blk.0.ffn_gate_exps.weight") if n_expert else None
        spec = ModelSpec(dim=dim, head_dim=head_dim, n_layers=n_layers, n_heads=n_heads,
                         n_kv_heads=n_kv, vocab=embd.dims[1], ctx_len=ctx, rope_dim=rope_dim,
                         rope_base=fl("rope.freq_base", 10000.0), eps=fl("attention.layer_norm_rms_epsilon", 1e-5),
                         rope_neox=arch == "qwen3moe", qk_norm=g.find_tensor("blk.0.attn_q_norm.weight") is not None,
                         embed_t=embd.ggml_type, output_t=out.ggml_type,
                         wq_t=tensor("blk.0.attn_q.weight").ggml_type, wk_t=tensor("blk.0.attn_k.weight").ggml_type,
                         wv_t=tensor("blk.0.attn_v.weight").ggml_type,
                         wo_t=tensor("blk.0.attn_output.weight").ggml_type, ffn=ffn, n_expert=n_expert,
                         n_used=n_used, moe_ffn=moe_ffn,
                         moe_gate_t=first_moe.ggml_type if first_moe else Q4_K,
                         router_bias=g.find_tensor("blk.0.exp_probs_b.bias") is not None,
                         gating=GATING_SIGMOID if u("expert_gating_func", 1) == 2 else GATING_SOFTMAX,
                         weights_norm=True if norm is None else norm,
                         weights_scale=fl("expert_weights_scale", 1.0))
        m = cls(spec)

        def expect_shape(t, want):
            # llama.zig:293-309 expectShape / expectExpertShape: the file's dims
            # must be exactly what the configuration implies (trailing unit
            # dims read as absent, as resolve reads a missing ne1/ne2 as 1)
            dims = tuple(int(d) for d in t.dims)
            while len(dims) > len(want) and dims[-1] == 1:
                dims = dims[:-1]
            if dims != tuple(want):
                raise ValueError(f"BadTensorShape: tensor {t.name} has shape {list(dims)}, "
                                 f"config implies {list(want)}")

        # every tensor is resolved and checked first; nothing reaches the
        # device before all of them pass
        plan = []

        def quant(key, t, rows, cols, planes=1):
            if t.ggml_type not in (Q4_0, Q8_0, Q4_K, Q6_K):
                raise ValueError(f"UnsupportedTensorType: {t.name}: GGML type {t.ggml_type} is not served")
            expect_shape(t, (cols, rows) if planes == 1 else (cols, rows, planes))
            # llama.zig:258-272 resolve: the bytes the shape implies, inside the file
            want = ggml_bytes(t.ggml_type, rows, cols) * planes
            if t.nbytes != want:
                raise ValueError(f"BadTensorShape: tensor {t.name} holds {t.nbytes} bytes, its shape {want}")
            if t.data is None or t.data.size != want:
                raise ValueError(f"TruncatedGguf: tensor {t.name} lies outside the file")
            plan.append((key, t, (rows, cols, planes)))

        def f32(key, t, n, shape=None):
            # llama.zig:281-291 expectF32, then the configured shape
            if t.ggml_type != 0:
                raise ValueError(f"BadTensorType: tensor {t.name} must be f32, got type {t.ggml_type}")
            expect_shape(t, shape or (n,))
            if t.nbytes != 4 * n or t.data is None or t.data.size != 4 * n:
                raise ValueError(f"TruncatedGguf: tensor {t.name}: expected {n} f32 values inside the file")
            plan.append((key, t, None))

        quant("embed", embd, spec.vocab, dim)
        quant("output", out, spec.vocab, dim)
        f32("out_norm", tensor("output_norm.weight"), dim)
        for li in range(n_layers):
            b, p = f"blk.{li}.", f"l{li}."
            f32(p + "attn_norm", tensor(b + "attn_norm.weight"), dim)
            f32(p + "ffn_norm", tensor(b + "ffn_norm.weight"), dim)
            if spec.qk_norm:
                f32(p + "q_norm", tensor(b + "attn_q_norm.weight"), head_dim)
                f32(p + "k_norm", tensor(b + "attn_k_norm.weight"), head_dim)
            quant(p + "wq", tensor(b + "attn_q.weight"), spec.qd, dim)
            quant(p + "wk", tensor(b + "attn_k.weight"), spec.kvd, dim)
            quant(p + "wv", tensor(b + "attn_v.weight"), spec.kvd, dim)
            quant(p + "wo", tensor(b + "attn_output.weight"), dim, spec.qd)
            if n_expert:
                f32(p + "router", tensor(b + "ffn_gate_inp.weight"), n_expert * dim, (dim, n_expert))
                if spec.router_bias:
                    f32(p + "router_bias", tensor(b + "exp_probs_b.bias"), n_expert)
                quant(p + "gate", tensor(b + "ffn_gate_exps.weight"), moe_ffn, dim, n_expert)
                quant(p + "up", tensor(b + "ffn_up_exps.weight"), moe_ffn, dim, n_expert)
                quant(p + "down", tensor(b + "ffn_down_exps.weight"), dim, moe_ffn, n_expert)
            else:
                quant(p + "ffn_gate", tensor(b + "ffn_gate.weight"), ffn, dim)
                quant(p + "ffn_up", tensor(b + "ffn_up.weight"), ffn, dim)
                quant(p + "ffn_down", tensor(b + "ffn_down.weight"), dim, ffn)

        m.f32["ones_dim"] = torch.ones(dim, dtype=torch.float32, device="cuda")
        m.f32["ones_hd"] = torch.ones(head_dim, dtype=torch.float32, device="cuda")
        for key, t, shp in plan:
            if shp is None:
                m.f32[key] = torch.from_numpy(np.array(t.data.view(np.float32), copy=True)).cuda()
            else:
                rows, cols, planes = shp
                gb = torch.from_numpy(np.array(t.data, copy=True)).cuda()
                m.tensors[key] = _Tensor(t.ggml_type, rows, cols, planes,
                                         repack_dev(t.ggml_type, gb, rows, cols, planes), gb if keep_ggml else None)
        m._build_desc()
        return m

    def _ptr(self, name):
        t = self.tensors.get(name)
        return None if t is None else t.dev.data_ptr()

    def _f(self, name):
        t = self.f32.get(name)
        return None if t is None else t.data_ptr()

    def _build_desc(self):
        s = self.spec
        layers = (LayerDesc * s.n_layers)()
        ty = lambda name: self.tensors[name].t  # noqa: E731
        for li in range(s.n_layers):
            p = f"l{li}."
            L = layers[li]
            L.attn_norm = self._f(p + "attn_norm") or self._f("ones_dim")
            L.ffn_norm = self._f(p + "ffn_norm") or self._f("ones_dim")
            L.q_norm = (self._f(p + "q_norm") or self._f("ones_hd")) if s.qk_norm else None
            L.k_norm = (self._f(p + "k_norm") or self._f("ones_hd")) if s.qk_norm else None
            L.wq_t, L.wk_t, L.wv_t, L.wo_t = (ty(p + n) for n in ("wq", "wk", "wv", "wo"))
            L.wq, L.wk, L.wv, L.wo = (self._ptr(p + n) for n in ("wq", "wk", "wv", "wo"))
            if s.n_expert:
                L.is_moe = 1
                L.moe = MoeLayerDesc(s.dim, s.moe_ffn, s.n_expert, s.n_used, s.gating,
                                     int(s.weights_norm), s.weights_scale, self._f(p + "router"),
                                     self._f(p + "router_bias"), None, ty(p + "gate"), ty(p + "up"),
                                     ty(p + "down"), self._ptr(p + "gate"), self._ptr(p + "up"),
                                     self._ptr(p + "down"))
            else:
                L.is_moe = 0
                L.ffn_gate_t, L.ffn_up_t, L.ffn_down_t = (ty(p + n) for n in ("ffn_gate", "ffn_up", "ffn_down"))
                L.ffn_gate, L.ffn_up, L.ffn_down = (self._ptr(p + n)
                                                    for n in ("ffn_gate", "ffn_up", "ffn_down"))
                L.ffn = s.ffn
        self.layers = layers
        self.desc = ModelDesc(s.dim, s.head_dim, s.n_layers, s.n_heads, s.n_kv_heads, s.vocab,
                              s.ctx_len, s.rope_dim, s.rope_base, s.eps, int(s.rope_neox),
                              ty("embed"), self._ptr("embed"), self._f("out_norm") or self._f("ones_dim"),
                              ty("output"), self._ptr("output"), C.cast(layers, C.POINTER(LayerDesc)), None,
                              self.numerics, None)

    def weight_bytes(self) -> int:
        """Bytes of every quantized tensor plus the f32 ones (routers, norms)."""
        n = sum(t.dev.numel() for t in self.tensors.values())
        return n + sum(v.numel() * 4 for v in self.f32.values())


class Decoder:
    """Per-lane decode state on the device: fp16 K/V caches
    [n][n_layers][ctx_len][kvd], positions, tokens and logits."""

    def __init__(self, model: DeviceModel, n: int):
        import torch

        s = model.spec
        self.model, self.n = model, n
        shape = (n, s.n_layers, s.ctx_len, s.kvd)
        self.k_cache = torch.zeros(shape, dtype=torch.int16, device="cuda")
        self.v_cache = torch.zeros(shape, dtype=torch.int16, device="cuda")
        self.pos = torch.zeros(n, dtype=torch.int32, device="cuda")
        self.tokens = torch.zeros(n, dtype=torch.int32, device="cuda")
        self.logits = torch.empty((n, s.vocab), dtype=torch.float32, device="cuda")

    def prefill_random(self, n_pos: int, seed: int = 7, scale: float = 1.0):
        """Fill cache rows [0, n_pos) of every lane and layer with seeded
        random fp16 K/V and set pos = n_pos (the benchmark's prefilled
        context)."""
        import torch

        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        for c in (self.k_cache, self.v_cache):
            for lane in range(self.n):
                r = torch.randn((c.shape[1], n_pos, c.shape[3]), generator=g, device="cuda") * scale
                c[lane, :, :n_pos, :] = r.to(torch.float16).view(torch.int16)
        self.pos.fill_(n_pos)

    def step(self, tokens=None, next_out=True) -> int:
        """One decode step of every lane: tokens (device int32 [n]) default to
        ``self.tokens``; the greedy pick is written back into ``self.tokens``
        when ``next_out``."""
        tok = self.tokens if tokens is None else tokens
        nxt = self.tokens if next_out else None
        return check(lib().loomhip_token_frame_dev(
            C.byref(self.model.desc), _ptr(tok), _ptr(self.pos), self.n, _ptr(self.k_cache),
            _ptr(self.v_cache), _ptr(self.logits), _ptr(nxt), _stream()), "token_frame_dev")


__all__ = ["DeviceModel", "Decoder", "ModelSpec", "qwen3_30b_a3b", "stories15m"]
