"""Host mirror of Loom's compute-backend seam (src/compute/backend.zig) over
libloomhip.

Names, argument meaning and decline behaviour follow the reference:

* ``matvec`` / ``matmul`` / ``dequantRow`` fill ``out`` and return True when the
  device served the call; False means "declined" (type or shape not served),
  and the caller runs its own CPU path -- the reference's GPU backends fall
  back to ``cpu.matvec`` the same way (src/vulkan/backend.zig:365-378).
* ``moeRoute`` / ``moeFfnBlockRouted`` return a bool like the reference
  (src/compute/cpu.zig:68,86): False means declined before anything ran.
* Hard errors (device faults, bad arguments) raise ``LoomHipError``.

Host arrays are numpy; the ``*_dev`` helpers take torch device tensors and
run on torch's current stream, so they order with torch's own allocations.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import (COMBINE_EXPERT_ASC, COMBINE_SELECTION, DECLINED, F32, GATING_SIGMOID,
               GATING_SOFTMAX, OK, MlaAttnDesc, MoeLayerDesc, check, lib, take_launch_count)

MAX_BATCH = 256  # tokens per grouped MoE launch (the reference caps batching at 8)


def _p(a):
    return None if a is None else a.ctypes.data


@dataclass
class WeightRef:
    """src/compute/cpu.zig:21 WeightRef: a GGML-typed tensor's raw bytes."""

    ty: int
    data: np.ndarray  # uint8


@dataclass
class RoutedCfg:
    """src/compute/cpu.zig:61 RoutedCfg."""

    n_expert: int
    n_used: int
    gating_sigmoid: bool
    weights_norm: bool
    weights_scale: float


def parallelBegin(n: int = 0, device: int = 0) -> None:
    """Device bring-up (the GPU backends do theirs in parallelBegin)."""
    from . import init

    init(device)


def parallelEnd() -> None:
    pass


def takeCmdBufCount() -> int:
    """Launches since the last call (src/compute/backend.zig:112-116)."""
    return take_launch_count()


def _served(rc: int, what: str) -> bool:
    return check(rc, what) == OK


def matvec(t: int, out: np.ndarray, data: np.ndarray, x: np.ndarray, rows: int, cols: int) -> bool:
    assert out.dtype == np.float32 and out.size >= rows and x.size >= cols
    x = np.ascontiguousarray(x, np.float32)
    return _served(lib().loomhip_matvec(t, _p(out), _p(data), _p(x), rows, cols), "matvec")


def matmul(t: int, out: np.ndarray, data: np.ndarray, xs: np.ndarray, n: int, rows: int,
           cols: int) -> bool:
    assert out.dtype == np.float32 and out.size >= n * rows and xs.size >= n * cols
    xs = np.ascontiguousarray(xs, np.float32)
    return _served(lib().loomhip_matmul(t, _p(out), _p(data), _p(xs), n, rows, cols), "matmul")


def dequantRow(t: int, out: np.ndarray, data: np.ndarray, r: int, cols: int) -> bool:
    assert out.dtype == np.float32 and out.size >= cols
    return _served(lib().loomhip_dequant_row(t, _p(out), _p(data), r, cols), "dequantRow")


def moeRoute(logits: np.ndarray, bias, ids_out: np.ndarray, gates_out: np.ndarray,
             gating_sigmoid: bool, weights_norm: bool, weights_scale: float) -> bool:
    """src/compute/cpu.zig:86 / src/vulkan/backend.zig:437."""
    logits = np.ascontiguousarray(logits, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    assert ids_out.dtype == np.uint32 and gates_out.dtype == np.float32
    if ids_out.size != gates_out.size:
        return False
    rc = lib().loomhip_moe_route(_p(logits), _p(b), logits.size, ids_out.size,
                                 GATING_SIGMOID if gating_sigmoid else GATING_SOFTMAX,
                                 int(weights_norm), weights_scale, _p(ids_out), _p(gates_out))
    return _served(rc, "moeRoute")


def moeFfnBlockRouted(normed: np.ndarray, logits: np.ndarray, bias, gate_w: WeightRef,
                      up_w: WeightRef, down_w: WeightRef, shexp, ffn: int, shexp_ffn: int,
                      cfg: RoutedCfg, out: np.ndarray, n_tok: int = 1,
                      combine: int = COMBINE_SELECTION) -> bool:
    """src/compute/cpu.zig:68 moeFfnBlockRouted, generalised to n_tok tokens.

    ``normed`` is [n_tok][dim], ``logits`` [n_tok][n_expert]; ``out`` [n_tok][dim]
    receives the gated sum (SELECTION) or has it added (EXPERT_ASC).  ``shexp``
    is None or the shared expert's three WeightRefs (gate, up, down) of width
    ``shexp_ffn``, whose FFN is added after the routed sum."""
    sg = su = sd = WeightRef(0, None)
    if shexp is not None:
        sg, su, sd = shexp
    normed = np.ascontiguousarray(normed, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    dim = normed.size // n_tok
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    rc = lib().loomhip_moe_ffn_routed(
        _p(normed), n_tok, dim, _p(logits), _p(b), cfg.n_expert, cfg.n_used,
        GATING_SIGMOID if cfg.gating_sigmoid else GATING_SOFTMAX, int(cfg.weights_norm),
        cfg.weights_scale, gate_w.ty, _p(gate_w.data), up_w.ty, _p(up_w.data), down_w.ty,
        _p(down_w.data), sg.ty, _p(sg.data), su.ty, _p(su.data), sd.ty, _p(sd.data), ffn, shexp_ffn,
        combine, _p(out))
    return _served(rc, "moeFfnBlockRouted")


@dataclass
class ExpertRef:
    """src/compute/cpu.zig:23 ExpertRef: one expert's gate/up/down slices
    (GGML bytes of one plane each), its router weight and hidden width."""

    gate: WeightRef
    up: WeightRef
    down: WeightRef
    weight: float
    ffn: int


def _refs(experts: list):
    from . import ExpertRefDesc

    arr = (ExpertRefDesc * max(1, len(experts)))()
    for i, e in enumerate(experts):
        arr[i] = ExpertRefDesc(e.gate.ty, e.up.ty, e.down.ty, _p(e.gate.data), _p(e.up.data), _p(e.down.data),
                               float(e.weight), e.ffn)
    return arr


def moeFfnBlock(normed: np.ndarray, experts: list, out: np.ndarray) -> bool:
    """src/compute/cpu.zig:27 moeFfnBlock: out = sum over experts, in order, of
    weight * FFN(normed); each slice is copied into the library's HBM LRU
    (kept across calls when it lies in a registered arena).  False when
    declined (the caller runs its own loop)."""
    normed = np.ascontiguousarray(normed, np.float32)
    assert out.dtype == np.float32 and out.size == normed.size
    rc = lib().loomhip_moe_ffn_block(_p(normed), normed.size, _refs(experts), len(experts), _p(out))
    return _served(rc, "moeFfnBlock")


def moeFfnBlockPrefetch(dim: int, experts: list) -> None:
    """Source.prefetchAsync for the HBM tier (src/p2p/expert_fetch.zig:390):
    start the copies of the refs' arena slices; returns at once."""
    check(lib().loomhip_moe_ffn_block_prefetch(dim, _refs(experts), len(experts)), "moe_ffn_block_prefetch")


def registerArena(mem: np.ndarray) -> bool:
    """src/compute/cpu.zig:33 registerArena: a read-only host region whose
    bytes stay fixed (the model's mapping); False when declined."""
    return _served(lib().loomhip_register_arena(_p(mem), mem.nbytes), "registerArena")


def materializeArenas() -> int:
    """src/compute/cpu.zig:38 materializeArenas: the registered arena bytes."""
    return int(lib().loomhip_materialize_arenas())


def moeFfnBlockStats() -> tuple:
    """(hits, misses, bytes_read) of moeFfnBlock's HBM LRU."""
    h, m, b = C.c_uint64(), C.c_uint64(), C.c_uint64()
    check(lib().loomhip_moe_ffn_block_stats(C.byref(h), C.byref(m), C.byref(b)), "moe_ffn_block_stats")
    return h.value, m.value, b.value


def profileKernels(enable: bool) -> None:
    """Record HIP events around every grouped-expert / dense matvec launch
    (resets the totals)."""
    lib().loomhip_profile_kernels(int(enable))


_KERNEL_SYMBOLS = {
    "gate_up": "moe_gateup_decode_kernel (n <= 4) / dmmv_kernel<T, NT, FUSED=true> / from 16 tokens "
               "mmq_kernel<T, 1, FUSED=true, SBW> (grouped gate/up + SwiGLU)",
    "down": "moe_down_decode_kernel (n <= 4) / dmmv_kernel<T, NT, FUSED=false> / from 16 tokens "
            "mmq_kernel<T, 1, false, SBW> (grouped down)",
    "dense": "dmmv_kernel<T, NT, false> / from 16 vectors mmq_kernel<T, MT, false, SBW> (dense matvec)",
    "attn": "attn_direct_kernel (FAST numerics, more than 4 lanes) / attn_partial_kernel (FAST split-context "
            "attention over the fp16 K/V cache)",
    "head": "dmmv_kernel<T, NT, false> / from 16 lanes mmq_stream_kernel<T, MT, false> (output head)",
    "qkv": "dmmv_seg_kernel<NT> / from 16 lanes mmq_seg_kernel<1, SBW> (q, k, v in one launch)",
    "wo": "dmmv_kernel<T, NT, false> / from 16 lanes mmq_kernel<T, 1, false, SBW> (wo + residual)",
    "attn_scores": "attn_scores_kernel<HD> (PARITY, up to 4 lanes: dotF32-order scores with the q/k norm, rope and "
                   "K/V append) / attn_scores_many_kernel<HD> (more lanes: a thread per position, query elements "
                   "as scalar operands)",
    "attn_softmax": "attn_softmax_kernel<512> (PARITY, more than 4 lanes: max, exp, position-ordered sum, p)",
    "attn_pv": "attn_pv_split_kernel<HD, true> (PARITY, up to 4 lanes: the head's softmax, then position-ordered "
               "P.V, and wo's input quantized) / attn_pv_many_kernel<HD, NW> (more lanes: position-ordered P.V, a "
               "wave per head over position-quad value tiles)",
    "mla_absorb": "mla_absorb_kernel (MLA: qa = W_k^T q_nope in axpy order)",
    "mla_scores": "mla_scores_kernel (MLA: dotF32-order scores over the compressed cache)",
    "mla_softmax": "mla_softmax_kernel<1024> (MLA: max, exp, position-ordered sum, p)",
    "mla_wsum": "mla_wsum_kernel (MLA: o = sum_t p_t c_t in position order)",
    "mla_wv": "quant_act_kernel + dmmv_kernel<T, 1, false> (MLA: W_v per head)",
}


def kernelStats() -> dict:
    """{name: {"ms": total, "count": launches, "name": kernel}} for tags with launches."""
    from . import KT_NAMES

    out = {}
    for tag, name in KT_NAMES.items():
        ms, n = C.c_double(), C.c_uint64()
        check(lib().loomhip_kernel_time(tag, C.byref(ms), C.byref(n)), "kernel_time")
        if n.value:
            out[name] = {"ms": ms.value, "count": n.value, "name": _KERNEL_SYMBOLS[name]}
    return out


def registerWeights(t: int, host: np.ndarray, rows: int, cols: int, planes: int = 1) -> int:
    """Pointer-keyed upload; returns the device address."""
    dev = C.c_void_p()
    check(lib().loomhip_register_weights(t, _p(host), rows, cols, planes, C.byref(dev)),
          "register_weights")
    return dev.value


def clearWeightCache() -> None:
    lib().loomhip_clear_weight_cache()


# ---- device-resident helpers (torch tensors as HBM buffers) ------------------


def _stream():
    """torch's current stream as a handle for the C ABI (NULL = the null
    stream for both)."""
    import torch

    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def plane_bytes(t: int, rows: int, cols: int) -> int:
    return int(lib().loomhip_plane_bytes(t, rows, cols))


def synth_ggml_dev(t: int, rows: int, cols: int, planes: int, seed: int, stddev: float,
                   device="cuda"):
    """Allocate and fill `planes` GGML-layout planes with seeded synthetic
    blocks (bench input generator); ``repack_dev`` turns them into the device
    layout."""
    import torch

    from . import ggml_bytes

    buf = torch.empty(ggml_bytes(t, rows, cols) * planes, dtype=torch.uint8, device=device)
    check(lib().loomhip_synth_weights_dev(t, _ptr(buf), rows, cols, planes, seed, stddev,
                                          _stream()), "synth_weights_dev")
    return buf


def repack_dev(t: int, ggml_bytes_dev, rows: int, cols: int, planes: int):
    """GGML bytes (device uint8 tensor) -> device layout."""
    import torch

    out = torch.empty(plane_bytes(t, rows, cols) * planes, dtype=torch.uint8,
                      device=ggml_bytes_dev.device)
    check(lib().loomhip_repack_dev(t, _ptr(out), _ptr(ggml_bytes_dev), rows, cols, planes,
                                   _stream()), "repack_dev")
    return out


def matvec_dev(t: int, out, w, x, n: int, rows: int, cols: int) -> int:
    return check(lib().loomhip_matvec_dev(t, _ptr(out), _ptr(w), _ptr(x), n, rows, cols,
                                          _stream()), "matvec_dev")


def dequant_dev(t: int, out, w, rows: int, cols: int) -> int:
    return check(lib().loomhip_dequant_dev(t, _ptr(out), _ptr(w), rows, cols, _stream()),
                 "dequant_dev")


# ---- the GQA device cache and frames (src/compute/backend.zig:121-160,
# 186-191; src/gguf/llama.zig:1067-1108 stepRecorded) ---------------------------


def _wref(w):
    """A WeightRef (or None) as the C ABI's loomhip_weight_ref."""
    from . import WeightRefDesc

    if w is None:
        return WeightRefDesc(0, None, 0)
    return WeightRefDesc(w.ty, _p(w.data), w.data.nbytes)


def attnInit(layers: int, ctx_len: int, kvd: int) -> bool:
    """backend.attnInit: allocate the device K/V cache (fp16); False declines."""
    return _served(lib().loomhip_attn_init(layers, ctx_len, kvd), "attnInit")


def hasKvCache() -> bool:
    return bool(lib().loomhip_has_kv_cache())


def releaseKvCache() -> None:
    lib().loomhip_release_kv_cache()


def kvAppend(li: int, pos: int, k_new: np.ndarray, v_new: np.ndarray) -> bool:
    """backend.kvAppend: mirror one host cache row into the device cache."""
    k_new = np.ascontiguousarray(k_new, np.float32)
    v_new = np.ascontiguousarray(v_new, np.float32)
    assert k_new.size == v_new.size
    return _served(lib().loomhip_kv_append(li, pos, _p(k_new), _p(v_new), k_new.size), "kvAppend")


def readKvCache(li: int, pos: int, k_out: np.ndarray, v_out: np.ndarray) -> bool:
    """The read-back that keeps the host cache authoritative: the device rows
    of layer li at pos (fp16 widened to f32) into k_out / v_out."""
    assert k_out.dtype == np.float32 and v_out.dtype == np.float32 and k_out.size == v_out.size
    return _served(lib().loomhip_read_kv(li, pos, _p(k_out), _p(v_out), k_out.size), "readKvCache")


def attnHeads(li: int, pos: int, q: np.ndarray, out: np.ndarray, n_heads: int, n_kv_heads: int, hd: int,
              scale: float) -> bool:
    """backend.attnHeads: one layer's GQA attention over the device cache
    (row pos already appended) into out [n_heads * hd]; False declines."""
    q = np.ascontiguousarray(q, np.float32)
    assert out.dtype == np.float32 and out.size == n_heads * hd
    return _served(lib().loomhip_attn_heads(li, pos, _p(q), _p(out), n_heads, n_kv_heads, hd, scale), "attnHeads")


@dataclass
class LayerSpec:
    """src/compute/cpu.zig:116-138 LayerSpec (a dense GQA layer)."""

    li: int
    pos: int
    attn_norm: np.ndarray
    ffn_norm: np.ndarray
    eps: float
    wq: WeightRef
    wk: WeightRef
    wv: WeightRef
    wo: WeightRef
    gate: WeightRef
    up: WeightRef
    down: WeightRef
    dim: int
    ffn: int
    n_heads: int
    n_kv_heads: int
    hd: int
    rope_dim: int
    rope_base: float
    rope_neox: bool
    attn_scale: float


def beginFrame() -> bool:
    return _served(lib().loomhip_begin_frame(), "beginFrame")


def frameOpen() -> bool:
    return bool(lib().loomhip_frame_open())


def frameLoadX(x: np.ndarray) -> bool:
    x = np.ascontiguousarray(x, np.float32)
    return _served(lib().loomhip_frame_load_x(_p(x), x.size), "frameLoadX")


def layerBlock(s: LayerSpec) -> bool:
    """backend.layerBlock: one whole dense layer recorded into the open
    frame; False declines before anything of the layer is recorded."""
    from . import LayerSpecDesc

    d = LayerSpecDesc(s.li, s.pos, _p(s.attn_norm), _p(s.ffn_norm), s.eps, *(_wref(w) for w in (
        s.wq, s.wk, s.wv, s.wo, s.gate, s.up, s.down)), s.dim, s.ffn, s.n_heads, s.n_kv_heads, s.hd, s.rope_dim,
        s.rope_base, int(s.rope_neox), s.attn_scale)
    return _served(lib().loomhip_layer_block(C.byref(d)), "layerBlock")


def endFrame() -> None:
    check(lib().loomhip_end_frame(), "endFrame")


def frameStoreX(x: np.ndarray) -> bool:
    assert x.dtype == np.float32
    return _served(lib().loomhip_frame_store_x(_p(x), x.size), "frameStoreX")


@dataclass
class GqaLayerDesc:
    """The qwen3moe counterpart of src/compute/cpu.zig:73 MlaLayerDesc: norms as
    f32 arrays, weights as WeightRefs (3D expert tensors whole), q_norm /
    k_norm / router_bias / sel_bias / shexp optional."""

    attn_norm: np.ndarray
    ffn_norm: np.ndarray
    wq: WeightRef
    wk: WeightRef
    wv: WeightRef
    wo: WeightRef
    is_moe: bool
    q_norm: np.ndarray | None = None
    k_norm: np.ndarray | None = None
    router: WeightRef | None = None
    router_bias: np.ndarray | None = None
    sel_bias: np.ndarray | None = None
    gate: WeightRef | None = None
    up: WeightRef | None = None
    down: WeightRef | None = None
    shexp: tuple | None = None  # (gate, up, down) WeightRefs
    ffn: int = 0
    shexp_ffn: int = 0
    dgate: WeightRef | None = None
    dup: WeightRef | None = None
    ddown: WeightRef | None = None
    dffn: int = 0


@dataclass
class GqaFrameCfg:
    """MlaFrameCfg's GQA counterpart, with its RoutedCfg."""

    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rope_dim: int
    eps: float
    scale: float
    rope_base: float
    rope_neox: bool
    routed: RoutedCfg | None = None
    gating: int = GATING_SOFTMAX


def gqaTokenFrame(descs: list, fc: GqaFrameCfg, x: np.ndarray, pos: int, out_norm: np.ndarray, lm_head: WeightRef,
                  logits: np.ndarray) -> bool:
    """The whole token as one submission (mlaTokenFrame's form): x [dim] in
    (after embedding) and out (after the last layer), logits [vocab] out;
    the device cache holds this position's rows afterwards (readKvCache).
    False declines before anything is launched."""
    from . import GqaFrameCfg as CCfg, GqaLayerDescC

    arr = (GqaLayerDescC * len(descs))()
    for d, c in zip(descs, arr):
        sh = d.shexp or (None, None, None)
        c.attn_norm, c.ffn_norm, c.q_norm, c.k_norm = (_p(a) for a in (d.attn_norm, d.ffn_norm, d.q_norm, d.k_norm))
        c.wq, c.wk, c.wv, c.wo = (_wref(w) for w in (d.wq, d.wk, d.wv, d.wo))
        c.is_moe = int(d.is_moe)
        c.router = _wref(d.router)
        c.router_bias, c.sel_bias = _p(d.router_bias), _p(d.sel_bias)
        c.gate, c.up, c.down = (_wref(w) for w in (d.gate, d.up, d.down))
        c.shexp_gate, c.shexp_up, c.shexp_down = (_wref(w) for w in sh)
        c.ffn, c.shexp_ffn = d.ffn, d.shexp_ffn
        c.dgate, c.dup, c.ddown = (_wref(w) for w in (d.dgate, d.dup, d.ddown))
        c.dffn = d.dffn
    r = fc.routed
    cfg = CCfg(fc.dim, fc.n_heads, fc.n_kv_heads, fc.head_dim, fc.rope_dim, fc.eps, fc.scale, fc.rope_base,
               int(fc.rope_neox), r.n_expert if r else 0, r.n_used if r else 0,
               (GATING_SIGMOID if r.gating_sigmoid else fc.gating) if r else fc.gating,
               int(r.weights_norm) if r else 1, r.weights_scale if r else 1.0)
    assert x.dtype == np.float32 and logits.dtype == np.float32 and x.flags.c_contiguous
    rc = lib().loomhip_gqa_token_frame(arr, len(descs), C.byref(cfg), _p(x), pos, _p(out_norm), _wref(lm_head),
                                       _p(logits), logits.size)
    return _served(rc, "gqaTokenFrame")


# ---- MLA attention over the compressed cache (src/compute/backend.zig:162-169,
# 193-197; src/gguf/deepseek.zig:851-1048) ----------------------------------


def mlaInit(layers: int, ctx_len: int, kvr: int, rope: int) -> bool:
    """backend.mlaInit: record the compressed cache's shape; False declines."""
    return _served(lib().loomhip_mla_init(layers, ctx_len, kvr, rope), "mlaInit")


def hasMlaCache() -> bool:
    return bool(lib().loomhip_has_mla_cache())


def mlaAppend(li: int, pos: int, c_kv: np.ndarray, k_rope: np.ndarray) -> bool:
    """backend.mlaAppend: mirror one position's rows into the device cache."""
    c_kv = np.ascontiguousarray(c_kv, np.float32)
    k_rope = np.ascontiguousarray(k_rope, np.float32)
    return _served(lib().loomhip_mla_append(li, pos, _p(c_kv), c_kv.size, _p(k_rope), k_rope.size), "mlaAppend")


def mlaReadCache(li: int, pos: int, c_kv: np.ndarray, k_rope: np.ndarray) -> bool:
    return _served(lib().loomhip_mla_read_cache(li, pos, _p(c_kv), c_kv.size, _p(k_rope), k_rope.size),
                   "mlaReadCache")


def mlaSetWk(li: int, wk_f32: np.ndarray) -> bool:
    wk_f32 = np.ascontiguousarray(wk_f32, np.float32)
    return _served(lib().loomhip_mla_set_wk(li, _p(wk_f32), wk_f32.size), "mlaSetWk")


def mlaAttnHeads(li: int, pos: int, q_nope: np.ndarray, q_rope: np.ndarray, kv_b: WeightRef, out: np.ndarray,
                 n_heads: int, nope: int, v_head_dim: int, scale: float) -> bool:
    """backend.mlaAttnHeads: every head's attention over the device cache with
    W_v applied, into out [n_heads * v_head_dim]; False declines."""
    q_nope = np.ascontiguousarray(q_nope, np.float32)
    q_rope = np.ascontiguousarray(q_rope, np.float32)
    rc = lib().loomhip_mla_attn_heads(li, pos, _p(q_nope), q_nope.size, _p(q_rope), q_rope.size, kv_b.ty,
                                      _p(kv_b.data), kv_b.data.nbytes, _p(out), out.size, n_heads, nope,
                                      v_head_dim, scale)
    return _served(rc, "mlaAttnHeads")


def mlaLayerTail(li: int, pos: int, x: np.ndarray, q_nope: np.ndarray, q_rope: np.ndarray, kv_b: WeightRef,
                 attn_out_w: WeightRef, ffn_norm: np.ndarray, eps: float, router_w: WeightRef, router_bias,
                 gate_w: WeightRef, up_w: WeightRef, down_w: WeightRef, shexp, ffn: int, shexp_ffn: int,
                 cfg: RoutedCfg, n_heads: int, nope: int, v_head_dim: int, scale: float) -> bool:
    """backend.mlaLayerTail (src/compute/cpu.zig:63): attention over the device
    cache, the output projection and residual, the FFN norm, the routed MoE
    with the shared expert and its residual, one submission; x [dim] in place.
    False declines."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    q_nope = np.ascontiguousarray(q_nope, np.float32)
    q_rope = np.ascontiguousarray(q_rope, np.float32)
    ffn_norm = np.ascontiguousarray(ffn_norm, np.float32)
    b = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
    sg = su = sd = WeightRef(0, None)
    if shexp is not None:
        sg, su, sd = shexp
    rc = lib().loomhip_mla_layer_tail(
        li, pos, _p(x), x.size, _p(q_nope), q_nope.size, _p(q_rope), q_rope.size, kv_b.ty, _p(kv_b.data),
        kv_b.data.nbytes, attn_out_w.ty, _p(attn_out_w.data), _p(ffn_norm), eps, router_w.ty, _p(router_w.data), _p(b),
        gate_w.ty, _p(gate_w.data), up_w.ty, _p(up_w.data), down_w.ty, _p(down_w.data), sg.ty, _p(sg.data), su.ty,
        _p(su.data), sd.ty, _p(sd.data), ffn, shexp_ffn, cfg.n_expert, cfg.n_used,
        GATING_SIGMOID if cfg.gating_sigmoid else GATING_SOFTMAX, int(cfg.weights_norm), cfg.weights_scale, n_heads,
        nope, v_head_dim, scale)
    return _served(rc, "mlaLayerTail")


@dataclass
class MlaLayerDesc:
    """src/compute/cpu.zig:73 MlaLayerDesc: norms as f32 arrays, weights as
    WeightRefs (3D expert tensors whole); shexp (gate, up, down) optional."""

    attn_norm: np.ndarray
    wq: WeightRef
    kv_a: WeightRef
    kv_a_norm: np.ndarray
    kv_b: WeightRef
    attn_out: WeightRef
    ffn_norm: np.ndarray
    is_moe: bool
    router: WeightRef | None = None
    gate: WeightRef | None = None
    up: WeightRef | None = None
    down: WeightRef | None = None
    shexp: tuple | None = None
    ffn: int = 0
    shexp_ffn: int = 0
    dgate: WeightRef | None = None
    dup: WeightRef | None = None
    ddown: WeightRef | None = None
    dffn: int = 0


@dataclass
class MlaFrameCfg:
    """src/compute/cpu.zig:74 MlaFrameCfg."""

    dim: int
    n_heads: int
    nope: int
    rope: int
    kvr: int
    v_head_dim: int
    eps: float
    scale: float
    rope_base: float
    yarn_factor: float
    yarn_orig_ctx: float
    routed: RoutedCfg | None = None


def mlaTokenFrame(descs: list, fc: MlaFrameCfg, x: np.ndarray, pos: int, out_norm: np.ndarray, lm_head: WeightRef,
                  logits: np.ndarray) -> bool:
    """backend.mlaTokenFrame: the whole MLA token as one submission over the
    device cache of mlaInit; x [dim] in (after embedding) and out (after the
    last layer), logits [vocab] out; False declines before anything runs."""
    from . import MlaFrameCfgC, MlaLayerDescC

    arr = (MlaLayerDescC * len(descs))()
    for d, c in zip(descs, arr):
        sh = d.shexp or (None, None, None)
        c.attn_norm, c.kv_a_norm, c.ffn_norm = _p(d.attn_norm), _p(d.kv_a_norm), _p(d.ffn_norm)
        c.wq, c.kv_a, c.kv_b, c.attn_out = (_wref(w) for w in (d.wq, d.kv_a, d.kv_b, d.attn_out))
        c.is_moe = int(d.is_moe)
        c.router, c.gate, c.up, c.down = (_wref(w) for w in (d.router, d.gate, d.up, d.down))
        c.shexp_gate, c.shexp_up, c.shexp_down = (_wref(w) for w in sh)
        c.ffn, c.shexp_ffn = d.ffn, d.shexp_ffn
        c.dgate, c.dup, c.ddown = (_wref(w) for w in (d.dgate, d.dup, d.ddown))
        c.dffn = d.dffn
    r = fc.routed
    cfg = MlaFrameCfgC(fc.dim, fc.n_heads, fc.nope, fc.rope, fc.kvr, fc.v_head_dim, fc.eps, fc.scale, fc.rope_base,
                       fc.yarn_factor, fc.yarn_orig_ctx, r.n_expert if r else 0, r.n_used if r else 0,
                       (GATING_SIGMOID if r.gating_sigmoid else GATING_SOFTMAX) if r else GATING_SOFTMAX,
                       int(r.weights_norm) if r else 1, r.weights_scale if r else 1.0)
    assert x.dtype == np.float32 and logits.dtype == np.float32 and x.flags.c_contiguous
    rc = lib().loomhip_mla_token_frame(arr, len(descs), C.byref(cfg), _p(x), pos, _p(out_norm), _wref(lm_head),
                                       _p(logits), logits.size)
    return _served(rc, "mlaTokenFrame")


class MlaAttn:
    """Device-resident MLA attention of one layer: kv_b (GGML bytes, a torch
    uint8 device tensor) split per head into W_k / W_v planes once."""

    def __init__(self, kvb_type: int, kv_b_ggml, n_heads: int, nope: int, vd: int, kvr: int, rope: int,
                 scale: float):
        import torch

        self.wk = torch.empty(plane_bytes(kvb_type, nope, kvr) * n_heads, dtype=torch.uint8, device="cuda")
        self.wv = torch.empty(plane_bytes(kvb_type, vd, kvr) * n_heads, dtype=torch.uint8, device="cuda")
        check(lib().loomhip_mla_split_kvb_dev(kvb_type, _ptr(kv_b_ggml), n_heads, nope, vd, kvr, _ptr(self.wk),
                                              _ptr(self.wv), _stream()), "mla_split_kvb_dev")
        self.desc = MlaAttnDesc(kvb_type, self.wk.data_ptr(), self.wv.data_ptr(), n_heads, nope, vd, kvr, rope,
                                scale)
        self.n_heads, self.nope, self.vd, self.kvr, self.rope = n_heads, nope, vd, kvr, rope

    def __call__(self, c_kv, k_rope, seq: int, q_nope, q_rope, out, o_lat=None) -> int:
        return check(lib().loomhip_mla_attn_dev(C.byref(self.desc), _ptr(c_kv), _ptr(k_rope), seq, _ptr(q_nope),
                                                _ptr(q_rope), _ptr(out), _ptr(o_lat), _stream()),
                     "mla_attn_dev")

    def tail(self, c_kv, k_rope, seq: int, q_nope, q_rope, attn_out_t: int, attn_out, ffn_norm, eps: float,
             moe: "MoeLayer", x) -> int:
        """The whole layer after the attention head on the device (x in place)."""
        return check(lib().loomhip_mla_layer_tail_dev(C.byref(self.desc), _ptr(c_kv), _ptr(k_rope), seq,
                                                      _ptr(q_nope), _ptr(q_rope), attn_out_t, _ptr(attn_out),
                                                      _ptr(ffn_norm), eps, C.byref(moe.desc), _ptr(x), _stream()),
                     "mla_layer_tail_dev")

    def cached_block(self, c_kvs, k_ropes, seq: int, q_nope, q_rope, attn_out_t: int, attn_out, ffn_norm,
                     eps: float, moe_desc, ec, x, want_ids: bool = False):
        """Config 5's block with its routed experts streamed through the
        expert cache `ec` (loom_amd.expert_cache.ExpertCache), for n =
        len(c_kvs) sequences: x [n][dim] in place; returns the routed ids
        [n][n_used] when want_ids."""
        n = len(c_kvs)
        cp = (C.c_void_p * n)(*[_ptr(c) for c in c_kvs])
        rp = (C.c_void_p * n)(*[_ptr(r) for r in k_ropes])
        ids = np.zeros((n, moe_desc.n_used), np.uint32) if want_ids else None
        check(lib().loomhip_mla_layer_cached_dev(C.byref(self.desc), cp, rp, seq, n, _ptr(q_nope), _ptr(q_rope),
                                                 attn_out_t, _ptr(attn_out), _ptr(ffn_norm), eps,
                                                 C.byref(moe_desc), ec.h, _ptr(x), _p(ids), _stream()),
              "mla_layer_cached_dev")
        return ids


class MoeLayer:
    """Device-resident MoE layer (weights are torch uint8 tensors in the
    device layout, one plane per expert)."""

    def __init__(self, dim, ffn, n_expert, n_used, router, gate, up, down, gate_t, up_t, down_t,
                 router_bias=None, sel_bias=None, gating=GATING_SOFTMAX, weights_norm=True,
                 weights_scale=1.0, shexp=None):
        """shexp: None or the shared expert (gate, up, down device tensors, gate_t, up_t,
        down_t, shexp_ffn)."""
        self.keep = (router, gate, up, down, router_bias, sel_bias, shexp)
        self.desc = MoeLayerDesc(dim, ffn, n_expert, n_used, gating, int(weights_norm),
                                 weights_scale, router.data_ptr(),
                                 None if router_bias is None else router_bias.data_ptr(),
                                 None if sel_bias is None else sel_bias.data_ptr(), gate_t, up_t,
                                 down_t, gate.data_ptr(), up.data_ptr(), down.data_ptr())
        if shexp is not None:
            sg, su, sd, sgt, sut, sdt, sf = shexp
            d = self.desc
            d.shexp_gate_t, d.shexp_up_t, d.shexp_down_t = sgt, sut, sdt
            d.shexp_gate, d.shexp_up, d.shexp_down = sg.data_ptr(), su.data_ptr(), sd.data_ptr()
            d.shexp_ffn = sf
        self.dim, self.ffn, self.n_expert, self.n_used = dim, ffn, n_expert, n_used

    def __call__(self, normed, out, combine=COMBINE_SELECTION, ids=None, gates=None) -> int:
        n = normed.shape[0]
        return check(lib().loomhip_moe_layer_dev(C.byref(self.desc), _ptr(normed), n, combine,
                                                 _ptr(out), _ptr(ids), _ptr(gates), _stream()),
                     "moe_layer_dev")


__all__ = [
    "COMBINE_EXPERT_ASC", "COMBINE_SELECTION", "DECLINED", "ExpertRef", "F32", "MAX_BATCH", "MlaAttn", "MoeLayer",
    "hasMlaCache", "mlaAppend", "mlaAttnHeads", "mlaInit", "mlaLayerTail", "mlaReadCache", "mlaSetWk",
    "moeFfnBlock", "moeFfnBlockStats",
    "RoutedCfg", "WeightRef", "clearWeightCache", "dequantRow", "matmul", "matvec", "moeFfnBlockRouted",
    "moeRoute", "parallelBegin", "parallelEnd", "registerWeights", "takeCmdBufCount",
]
