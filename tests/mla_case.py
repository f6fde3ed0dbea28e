"""Seeded MLA attention inputs (test helper): one layer's compressed cache
rows, the absorbed-query inputs and a quantized fused kv_b, shaped as
deepseek.zig's attnLayer hands them to mlaAttnHeads (deepseek.zig:977-988):
c_kv [ctx][kvr] (rmsnorm outputs, ~N(0, 1)), k_rope [ctx][rope], q_nope
[n_heads][nope], q_rope [n_heads][rope], kv_b rows h*(nope+vd) .. +nope =
head h's W_k and the next vd its W_v, N(0, 1/sqrt(kvr)) quantized by the
oracle's quantizers."""
from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np


@dataclasses.dataclass
class MlaCase:
    n_heads: int
    nope: int
    vd: int
    kvr: int
    rope: int
    ctx: int
    t: int
    c_kv: np.ndarray
    k_rope: np.ndarray
    q_nope: np.ndarray
    q_rope: np.ndarray
    kv_b: np.ndarray
    scale: float


def make_case(oracle, t, n_heads, nope, vd, kvr, rope, ctx, seed) -> MlaCase:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n_heads * (nope + vd), kvr)) / np.sqrt(kvr)).astype(np.float32)
    return MlaCase(
        n_heads, nope, vd, kvr, rope, ctx, t,
        c_kv=rng.standard_normal((ctx, kvr)).astype(np.float32),
        k_rope=rng.standard_normal((ctx, rope)).astype(np.float32),
        q_nope=rng.standard_normal(n_heads * nope).astype(np.float32),
        q_rope=rng.standard_normal(n_heads * rope).astype(np.float32),
        kv_b=oracle.quantize(t, w),
        scale=float(1.0 / np.sqrt(nope + rope)),
    )


@dataclasses.dataclass
class MlaModelCase:
    """A DeepSeek-V3-style MLA model at reduced width (test helper): host
    GGML bytes and f32 norms, in the shape mlaTokenFrame records (direct q,
    fused kv_b; layer kinds from `moe`, each MoE layer with sigmoid gating,
    renormalised gates scaled by `wscale`, and a shared expert)."""
    dim: int
    n_heads: int
    nope: int
    rope: int
    kvr: int
    vd: int
    ctx: int
    vocab: int
    eps: float
    scale: float
    rope_base: float
    yarn_factor: float
    yarn_orig_ctx: float
    n_expert: int
    n_used: int
    ffn: int
    sffn: int
    dffn: int
    wscale: float
    layers: list
    embed: np.ndarray
    out_norm: np.ndarray
    output: np.ndarray
    types: dict


def make_mla_model(oracle, seed, moe=(False, True), dim=1024, n_heads=8, nope=128, rope=64, kvr=512, vd=128,
                   ctx=48, vocab=512, n_expert=8, n_used=2, ffn=256, sffn=512, dffn=512) -> MlaModelCase:
    from recipes import planes

    Q4_K, Q6_K = 12, 14
    rng = np.random.default_rng(seed)
    s = seed * 100

    def norm(n):
        return (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)

    layers = []
    for li, is_moe in enumerate(moe):
        b = s + 20 * li
        L = {"attn_norm": norm(dim), "kv_a_norm": norm(kvr), "ffn_norm": norm(dim), "is_moe": is_moe,
             "wq": planes(Q4_K, n_heads * (nope + rope), dim, 1, b + 1),
             "kv_a": planes(Q4_K, kvr + rope, dim, 1, b + 2),
             "attn_out": planes(Q4_K, dim, n_heads * vd, 1, b + 4)}
        w = (rng.standard_normal((n_heads * (nope + vd), kvr)) / np.sqrt(kvr)).astype(np.float32)
        L["kv_b"] = oracle.quantize(Q4_K, w)
        if is_moe:
            L["router"] = (rng.standard_normal((n_expert, dim)) / np.sqrt(dim)).astype(np.float32)
            L["gate"], L["up"] = planes(Q4_K, ffn, dim, n_expert, b + 5), planes(Q4_K, ffn, dim, n_expert, b + 6)
            L["down"] = planes(Q6_K, dim, ffn, n_expert, b + 7)
            L["sg"], L["su"] = planes(Q4_K, sffn, dim, 1, b + 8), planes(Q4_K, sffn, dim, 1, b + 9)
            L["sd"] = planes(Q6_K, dim, sffn, 1, b + 10)
        else:
            L["dgate"], L["dup"] = planes(Q4_K, dffn, dim, 1, b + 11), planes(Q4_K, dffn, dim, 1, b + 12)
            L["ddown"] = planes(Q6_K, dim, dffn, 1, b + 13)
        layers.append(L)
    return MlaModelCase(dim, n_heads, nope, rope, kvr, vd, ctx, vocab, 1e-6, float(1.0 / np.sqrt(nope + rope)),
                        10000.0, 40.0, 4096.0, n_expert, n_used, ffn, sffn, dffn, 2.5, layers,
                        planes(Q4_K, vocab, dim, 1, s + 90), norm(dim), planes(Q6_K, vocab, dim, 1, s + 91),
                        {"down": Q6_K, "sd": Q6_K, "ddown": Q6_K, "output": Q6_K})


class MlaOracleStepper:
    """lo_mla_step over an MlaModelCase, with its own f32 latent caches."""

    def __init__(self, oracle, mc: MlaModelCase):
        o = oracle
        self.o, self.mc = o, mc
        ty = lambda k: mc.types.get(k, 12)  # noqa: E731
        T = lambda k, a, rows, cols, planes=1: o.Tensor(ty(k), a.ctypes.data, cols, rows, planes)  # noqa: E731
        self.layers = (o.MlaLayer * len(mc.layers))()
        self.keep = []
        H, kd = mc.n_heads, mc.nope + mc.rope
        for L, c in zip(mc.layers, self.layers):
            c.attn_norm, c.kv_a_norm, c.ffn_norm = (L[k].ctypes.data for k in ("attn_norm", "kv_a_norm", "ffn_norm"))
            c.wq = T("wq", L["wq"], H * kd, mc.dim)
            c.kv_a = T("kv_a", L["kv_a"], mc.kvr + mc.rope, mc.dim)
            c.kv_b = T("kv_b", L["kv_b"], H * (mc.nope + mc.vd), mc.kvr)
            c.attn_out = T("attn_out", L["attn_out"], mc.dim, H * mc.vd)
            c.is_moe = int(L["is_moe"])
            if L["is_moe"]:
                w = o.MoeWeights(mc.dim, mc.ffn, mc.n_expert, mc.n_used, L["router"], L["gate"], L["up"], L["down"],
                                 12, 12, ty("down"), gating=o.GATING_SIGMOID, weights_norm=True,
                                 weights_scale=mc.wscale, shexp=(L["sg"], L["su"], L["sd"], 12, 12, ty("sd"),
                                                                 mc.sffn))
                self.keep.append(w)
                c.moe = w.cstruct()
            else:
                c.dgate = T("dgate", L["dgate"], mc.dffn, mc.dim)
                c.dup = T("dup", L["dup"], mc.dffn, mc.dim)
                c.ddown = T("ddown", L["ddown"], mc.dim, mc.dffn)
        self.model = o.MlaModel(mc.dim, H, mc.nope, mc.rope, mc.kvr, mc.vd, len(mc.layers), mc.ctx, mc.vocab, mc.eps,
                                mc.scale, mc.rope_base, mc.yarn_factor, mc.yarn_orig_ctx,
                                C.cast(self.layers, C.c_void_p), mc.out_norm.ctypes.data,
                                o.Tensor(ty("output"), mc.output.ctypes.data, mc.dim, mc.vocab, 1))
        self.c_kv = np.zeros((len(mc.layers), mc.ctx, mc.kvr), np.float32)
        self.k_rope = np.zeros((len(mc.layers), mc.ctx, mc.rope), np.float32)

    def embed(self, tok):
        return np.ascontiguousarray(self.o.dequant_row(12, self.mc.embed, int(tok), self.mc.dim), np.float32)

    def step(self, x, pos):
        """x [dim] in place (the residual stream after the last layer);
        returns the logits."""
        logits = np.empty(self.mc.vocab, np.float32)
        rc = self.o.lib().lo_mla_step(C.byref(self.model), self.c_kv.ctypes.data, self.k_rope.ctypes.data, pos,
                                      x.ctypes.data, logits.ctypes.data)
        assert rc == 0
        return logits
