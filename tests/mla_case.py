"""Seeded MLA attention inputs (test helper): one layer's compressed cache
rows, the absorbed-query inputs and a quantized fused kv_b, shaped as
deepseek.zig's attnLayer hands them to mlaAttnHeads (deepseek.zig:977-988):
c_kv [ctx][kvr] (rmsnorm outputs, ~N(0, 1)), k_rope [ctx][rope], q_nope
[n_heads][nope], q_rope [n_heads][rope], kv_b rows h*(nope+vd) .. +nope =
head h's W_k and the next vd its W_v, N(0, 1/sqrt(kvr)) quantized by the
oracle's quantizers."""
from __future__ import annotations

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
