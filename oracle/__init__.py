"""CPU oracle for Loom's quantized MoE forward -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``oracle/liboracle.so`` (the C restatement of Loom's CPU
SIMD path, built by ``oracle/Makefile``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package, and only as the checker or as the timed CPU column; the product
library (``loom_amd``) never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
QK_0, QK_K, MAX_BATCH = 32, 256, 8
GATING_SOFTMAX, GATING_SIGMOID, GATING_SOFTMAX_TOPK = 1, 2, 3

BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}
NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def row_bytes(t: int, n: int) -> int:
    return (n // BLOCK_ELEMS[t]) * BLOCK_BYTES[t]


class XBlock(C.Structure):
    _fields_ = [("d", C.c_float), ("sum", C.c_int32), ("q", C.c_int8 * 32)]


class XBlockK(C.Structure):
    _fields_ = [("d", C.c_float), ("q", C.c_int8 * 256), ("bsum", C.c_int32 * 16)]


class RouteCfg(C.Structure):
    _fields_ = [
        ("n_expert", C.c_size_t),
        ("n_used", C.c_size_t),
        ("gating", C.c_int),
        ("weights_norm", C.c_int),
        ("weights_scale", C.c_float),
    ]


class Tensor(C.Structure):
    _fields_ = [
        ("ty", C.c_int),
        ("data", C.c_void_p),
        ("ne0", C.c_size_t),
        ("ne1", C.c_size_t),
        ("ne2", C.c_size_t),
    ]


class MoeLayer(C.Structure):
    _fields_ = [
        ("dim", C.c_size_t),
        ("ffn", C.c_size_t),
        ("route", RouteCfg),
        ("router", Tensor),
        ("router_bias", C.c_void_p),
        ("sel_bias", C.c_void_p),
        ("gate_exps", Tensor),
        ("up_exps", Tensor),
        ("down_exps", Tensor),
        ("shexp_gate", Tensor),
        ("shexp_up", Tensor),
        ("shexp_down", Tensor),
    ]


class ExpertRef(C.Structure):
    _fields_ = [("gate", Tensor), ("up", Tensor), ("down", Tensor), ("weight", C.c_float)]


class Layer(C.Structure):
    _fields_ = [
        ("attn_norm", C.c_void_p),
        ("wq", Tensor),
        ("wk", Tensor),
        ("wv", Tensor),
        ("wo", Tensor),
        ("q_norm", C.c_void_p),
        ("k_norm", C.c_void_p),
        ("ffn_norm", C.c_void_p),
        ("is_moe", C.c_int),
        ("ffn_gate", Tensor),
        ("ffn_up", Tensor),
        ("ffn_down", Tensor),
        ("moe", MoeLayer),
    ]


class Model(C.Structure):
    _fields_ = [
        ("dim", C.c_size_t),
        ("head_dim", C.c_size_t),
        ("n_layers", C.c_size_t),
        ("n_heads", C.c_size_t),
        ("n_kv_heads", C.c_size_t),
        ("vocab", C.c_size_t),
        ("ctx_len", C.c_size_t),
        ("rope_dim", C.c_size_t),
        ("rope_base", C.c_float),
        ("eps", C.c_float),
        ("rope_neox", C.c_int),
        ("kv_f16", C.c_int),
        ("embed", Tensor),
        ("out_norm", C.c_void_p),
        ("output", Tensor),
        ("layers", C.c_void_p),
    ]


class MlaLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("wq", Tensor), ("kv_a", Tensor), ("kv_a_norm", C.c_void_p),
                ("kv_b", Tensor), ("attn_out", Tensor), ("ffn_norm", C.c_void_p), ("is_moe", C.c_int),
                ("moe", MoeLayer), ("dgate", Tensor), ("dup", Tensor), ("ddown", Tensor)]


class MlaModel(C.Structure):
    _fields_ = ([(n, C.c_size_t) for n in ("dim", "n_heads", "nope", "rope", "kvr", "vd", "n_layers", "ctx_len",
                                           "vocab")] +
                [(n, C.c_float) for n in ("eps", "scale", "rope_base", "yarn_factor", "yarn_orig_ctx")] +
                [("layers", C.c_void_p), ("out_norm", C.c_void_p), ("output", Tensor)])


class Seq(C.Structure):
    _fields_ = [("k_cache", C.c_void_p), ("v_cache", C.c_void_p), ("pos", C.c_size_t)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, sz, f, i = C.c_void_p, C.c_size_t, C.c_float, C.c_int
        sig = {
            "lo_block_elems": (sz, [i]),
            "lo_block_bytes": (sz, [i]),
            "lo_row_bytes": (sz, [i, sz]),
            "lo_f16_to_f32": (f, [C.c_uint16]),
            "lo_f32_to_f16": (C.c_uint16, [f]),
            "lo_dequant_row": (None, [i, vp, vp, sz, sz]),
            "lo_to_i8_saturating": (C.c_int8, [f]),
            "lo_quantize_x": (None, [vp, sz, vp]),
            "lo_quantize_x256": (None, [vp, sz, vp]),
            "lo_dot_f32": (f, [vp, vp, sz]),
            "lo_axpy": (None, [vp, vp, f, sz]),
            "lo_matvec": (None, [i, vp, vp, vp, sz, sz]),
            "lo_matmul": (None, [i, vp, vp, vp, sz, sz, sz]),
            "lo_parallel_begin": (None, [i]),
            "lo_parallel_end": (None, []),
            "lo_parallel_threads": (i, []),
            "lo_quantize_rows": (None, [i, vp, vp, sz, sz]),
            "lo_fill_normal": (None, [vp, sz, C.c_uint64, f, f]),
            "lo_fill_uniform": (None, [vp, sz, C.c_uint64, f, f]),
            "lo_rmsnorm": (None, [vp, vp, vp, sz, f]),
            "lo_softmax": (None, [vp, sz]),
            "lo_silu": (f, [f]),
            "lo_sigmoid": (f, [f]),
            "lo_swiglu": (None, [vp, vp, vp, sz]),
            "lo_rope_norm": (None, [vp, sz, sz, f]),
            "lo_rope_neox": (None, [vp, sz, sz, f]),
            "lo_head_norm": (None, [vp, vp, sz, sz, f]),
            "lo_argmax": (sz, [vp, sz]),
            "lo_route": (None, [C.POINTER(RouteCfg), vp, vp, vp, vp]),
            "lo_moe_layer_token": (None, [C.POINTER(MoeLayer), vp, vp, vp, vp]),
            "lo_moe_batch_union": (None, [C.POINTER(MoeLayer), vp, vp, sz, vp, vp]),
            "lo_moe_ffn_block": (None, [vp, sz, vp, sz, vp]),
            "lo_seq_cache_bytes": (sz, [C.POINTER(Model)]),
            "lo_step": (i, [C.POINTER(Model), C.POINTER(Seq), C.c_uint32, vp]),
            "lo_decode_batch": (i, [C.POINTER(Model), vp, vp, sz, vp]),
            "lo_attn_heads": (None, [C.POINTER(Model), vp, vp, sz, sz, vp, vp, C.c_float]),
            "lo_mla_step": (i, [C.POINTER(MlaModel), vp, vp, sz, vp, vp]),
            "lo_set_mla_slip": (None, [i]),
            "lo_set_batch_slip": (None, [i]),
            "lo_lru_create": (vp, [sz]),
            "lo_lru_destroy": (None, [vp]),
            "lo_lru_find": (C.c_long, [vp, sz]),
            "lo_lru_reserve": (C.c_long, [vp, sz, C.POINTER(C.c_size_t)]),
            "lo_lru_abort": (None, [vp, sz]),
            "lo_lru_clear": (None, [vp]),
            "lo_cache_replay": (None, [sz, vp, sz, vp, sz, vp, vp]),
            "lo_hottest_within_budget": (sz, [vp, sz, sz, C.c_uint64, vp]),
            "lo_rope_yarn": (None, [vp, sz, sz, f, f, f]),
            "lo_mla_attn_heads": (None, [vp, vp, sz, sz, sz, vp, vp, i, vp, sz, sz, sz, f, vp, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- formats / dequant ------------------------------------------------------


def f16_to_f32(h: int) -> float:
    return lib().lo_f16_to_f32(h)


def f32_to_f16(x: float) -> int:
    return lib().lo_f32_to_f16(x)


def dequant_row(t: int, data: np.ndarray, r: int, cols: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    lib().lo_dequant_row(t, _p(out), _p(data), r, cols)
    return out


def dequant(t: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    for r in range(rows):
        lib().lo_dequant_row(t, out[r].ctypes.data, _p(data), r, cols)
    return out


# ---- activation quantizers -------------------------------------------------


def quantize_x(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    nb = x.size // 32
    out = (XBlock * nb)()
    lib().lo_quantize_x(_p(x), x.size, C.addressof(out))
    d = np.array([b.d for b in out], np.float32)
    s = np.array([b.sum for b in out], np.int32)
    q = np.array([list(b.q) for b in out], np.int8).reshape(nb, 32)
    return d, s, q


def quantize_x256(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    nb = x.size // 256
    out = (XBlockK * nb)()
    lib().lo_quantize_x256(_p(x), x.size, C.addressof(out))
    d = np.array([b.d for b in out], np.float32)
    q = np.array([list(b.q) for b in out], np.int8).reshape(nb, 256)
    bs = np.array([list(b.bsum) for b in out], np.int32).reshape(nb, 16)
    return d, q, bs


def to_i8_saturating(v: float) -> int:
    return lib().lo_to_i8_saturating(v)


# ---- matrix ops -------------------------------------------------------------


def dot_f32(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().lo_dot_f32(_p(a), _p(b), a.size)


def matvec(t: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().lo_matvec(t, _p(out), _p(w), _p(x), rows, cols)
    return out


def matmul(t: int, w: np.ndarray, xs: np.ndarray, n: int, rows: int, cols: int) -> np.ndarray:
    xs = np.ascontiguousarray(xs, np.float32)
    out = np.empty((n, rows), np.float32)
    lib().lo_matmul(t, _p(out), _p(w), _p(xs), n, rows, cols)
    return out


class Pool:
    """Context manager around the reference's row-parallel worker pool."""

    def __init__(self, threads: int):
        self.threads = threads

    def __enter__(self):
        lib().lo_parallel_begin(self.threads)
        return self

    def __exit__(self, *exc):
        lib().lo_parallel_end()


# ---- generators ---------------------------------------------------------------


def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().lo_fill_normal(_p(out), n, seed, mean, std)
    return out


def uniform(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().lo_fill_uniform(_p(out), n, seed, lo, hi)
    return out


def quantize(t: int, w: np.ndarray) -> np.ndarray:
    """Quantize a [rows][cols] f32 matrix row-wise into format t (bytes)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.empty(rows * row_bytes(t, cols), np.uint8)
    lib().lo_quantize_rows(t, _p(out), _p(w), rows, cols)
    return out


# ---- elementwise / routing ------------------------------------------------------


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().lo_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def softmax(x):
    x = np.array(x, np.float32)
    lib().lo_softmax(_p(x), x.size)
    return x


def silu(x: float) -> float:
    return lib().lo_silu(x)


def sigmoid(x: float) -> float:
    return lib().lo_sigmoid(x)


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().lo_swiglu(_p(out), _p(g), _p(u), g.size)
    return out


def rope(vec, rope_dim, pos, base, neox):
    v = np.array(vec, np.float32)
    (lib().lo_rope_neox if neox else lib().lo_rope_norm)(_p(v), rope_dim, pos, base)
    return v


def rope_yarn(vec, pos, base, factor=0.0, orig_ctx=0.0):
    """deepseek.zig:581-629 ropeApply (NORM pairs; YaRN when factor > 1)."""
    v = np.array(vec, np.float32)
    lib().lo_rope_yarn(_p(v), v.size, pos, base, factor, orig_ctx)
    return v


def mla_attn_heads(c_kv, k_rope, seq, q_nope, q_rope, kvb_type, kv_b, n_heads, nope, vd, scale):
    """deepseek.zig:988-1047: (out [n_heads][vd], o_lat [n_heads][kvr]) from
    one layer's cache rows c_kv [>= seq][kvr] and k_rope [>= seq][rope]."""
    c_kv = np.ascontiguousarray(c_kv, np.float32)
    k_rope = np.ascontiguousarray(k_rope, np.float32)
    kvr, rope = c_kv.shape[-1], k_rope.shape[-1]
    q_nope = np.ascontiguousarray(q_nope, np.float32)
    q_rope = np.ascontiguousarray(q_rope, np.float32)
    kv_b = np.ascontiguousarray(kv_b, np.uint8)
    assert q_nope.size == n_heads * nope and q_rope.size == n_heads * rope
    assert kv_b.size >= n_heads * (nope + vd) * row_bytes(kvb_type, kvr)
    out = np.empty(n_heads * vd, np.float32)
    o_lat = np.empty(n_heads * kvr, np.float32)
    lib().lo_mla_attn_heads(_p(c_kv), _p(k_rope), seq, kvr, rope, _p(q_nope), _p(q_rope), kvb_type, _p(kv_b),
                            n_heads, nope, vd, scale, _p(out), _p(o_lat))
    return out, o_lat


def head_norm(vec, w, n_heads, hd, eps):
    v = np.array(vec, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    lib().lo_head_norm(_p(v), _p(w), n_heads, hd, eps)
    return v


def argmax(logits) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().lo_argmax(_p(logits), logits.size)


def route(logits, n_used, gating=GATING_SOFTMAX, weights_norm=True, weights_scale=1.0, bias=None):
    logits = np.ascontiguousarray(logits, np.float32)
    cfg = RouteCfg(logits.size, n_used, gating, int(weights_norm), weights_scale)
    ids = np.empty(n_used, np.uint32)
    gates = np.empty(n_used, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().lo_route(C.byref(cfg), _p(logits), _p(b), _p(ids), _p(gates))
    return ids, gates


# ---- MoE layer ----------------------------------------------------------------


class MoeWeights:
    """Host copy of one MoE layer's tensors (stacked [E][rows] planes)."""

    def __init__(self, dim, ffn, n_expert, n_used, router, gate, up, down, gate_t, up_t, down_t,
                 router_bias=None, sel_bias=None, gating=GATING_SOFTMAX, weights_norm=True,
                 weights_scale=1.0, shexp=None):
        """shexp: optional shared expert (gate, up, down, gate_t, up_t, down_t, shexp_ffn),
        host GGML bytes of one plane each."""
        self.shexp = shexp
        self.dim, self.ffn, self.n_expert, self.n_used = dim, ffn, n_expert, n_used
        self.router = np.ascontiguousarray(router, np.float32)
        self.gate, self.up, self.down = gate, up, down
        self.gate_t, self.up_t, self.down_t = gate_t, up_t, down_t
        self.router_bias = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
        self.sel_bias = None if sel_bias is None else np.ascontiguousarray(sel_bias, np.float32)
        self.gating, self.weights_norm, self.weights_scale = gating, weights_norm, weights_scale

    def cstruct(self) -> MoeLayer:
        L = MoeLayer()
        L.dim, L.ffn = self.dim, self.ffn
        L.route = RouteCfg(self.n_expert, self.n_used, self.gating, int(self.weights_norm),
                           self.weights_scale)
        L.router = Tensor(F32, self.router.ctypes.data, self.dim, self.n_expert, 1)
        L.router_bias = _p(self.router_bias)
        L.sel_bias = _p(self.sel_bias)
        L.gate_exps = Tensor(self.gate_t, self.gate.ctypes.data, self.dim, self.ffn, self.n_expert)
        L.up_exps = Tensor(self.up_t, self.up.ctypes.data, self.dim, self.ffn, self.n_expert)
        L.down_exps = Tensor(self.down_t, self.down.ctypes.data, self.ffn, self.dim, self.n_expert)
        if self.shexp is not None:
            g, u, d, gt, ut, dt, sf = self.shexp
            L.shexp_gate = Tensor(gt, g.ctypes.data, self.dim, sf, 1)
            L.shexp_up = Tensor(ut, u.ctypes.data, self.dim, sf, 1)
            L.shexp_down = Tensor(dt, d.ctypes.data, sf, self.dim, 1)
        return L


def moe_layer_token(w: MoeWeights, normed):
    normed = np.ascontiguousarray(normed, np.float32)
    L = w.cstruct()
    acc = np.empty(w.dim, np.float32)
    ids = np.empty(w.n_used, np.uint32)
    gates = np.empty(w.n_used, np.float32)
    lib().lo_moe_layer_token(C.byref(L), _p(normed), _p(acc), _p(ids), _p(gates))
    return acc, ids, gates


def moe_ffn_block(normed, refs):
    """backend.moeFfnBlock: refs = [(gate, up, down, gate_t, up_t, down_t, ffn, weight)],
    host GGML bytes of one plane each; returns out[dim]."""
    normed = np.ascontiguousarray(normed, np.float32)
    dim = normed.size
    arr = (ExpertRef * len(refs))()
    for i, (g, u, d, gt, ut, dt, f, wt) in enumerate(refs):
        arr[i] = ExpertRef(Tensor(gt, g.ctypes.data, dim, f, 1), Tensor(ut, u.ctypes.data, dim, f, 1),
                           Tensor(dt, d.ctypes.data, f, dim, 1), wt)
    out = np.empty(dim, np.float32)
    lib().lo_moe_ffn_block(_p(normed), dim, C.cast(arr, C.c_void_p), len(refs), _p(out))
    return out


def moe_batch_union(w: MoeWeights, bnormed, bx):
    bnormed = np.ascontiguousarray(bnormed, np.float32)
    bx = np.array(bx, np.float32)
    n = bnormed.shape[0]
    L = w.cstruct()
    ids = np.empty((n, w.n_used), np.uint32)
    gates = np.empty((n, w.n_used), np.float32)
    lib().lo_moe_batch_union(C.byref(L), _p(bnormed), _p(bx), n, _p(ids), _p(gates))
    return bx, ids, gates


# ---- expert cache -------------------------------------------------------------


class Lru:
    def __init__(self, capacity: int):
        self.h = lib().lo_lru_create(capacity)

    def __del__(self):
        if getattr(self, "h", None):
            lib().lo_lru_destroy(self.h)
            self.h = None

    def find(self, id_: int) -> int:
        return lib().lo_lru_find(self.h, id_)

    def reserve(self, id_: int):
        ev = C.c_size_t()
        slot = lib().lo_lru_reserve(self.h, id_, C.byref(ev))
        return slot, (None if ev.value == 2**64 - 1 else ev.value)

    def abort(self, id_: int):
        lib().lo_lru_abort(self.h, id_)

    def clear(self):
        lib().lo_lru_clear(self.h)


def cache_replay(capacity: int, trace, pinned=None, n_ids: int = 0):
    trace = np.ascontiguousarray(trace, np.uint32)
    counts = np.zeros(3, np.uint64)
    mask = np.zeros(trace.size, np.uint8)
    pin = None if pinned is None else np.ascontiguousarray(pinned, np.uint8)
    lib().lo_cache_replay(capacity, _p(pin), n_ids if pin is not None else 0, _p(trace), trace.size,
                          _p(counts), _p(mask))
    return counts, mask


def hottest_within_budget(access_count, expert_bytes: int, budget: int):
    ac = np.ascontiguousarray(access_count, np.uint64)
    out = np.zeros(max(ac.size, 1), np.uint64)
    m = lib().lo_hottest_within_budget(_p(ac), ac.size, expert_bytes, budget, _p(out))
    return [int(v) for v in out[:m]]
