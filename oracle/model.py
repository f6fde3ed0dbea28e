"""TEST INFRASTRUCTURE: the oracle's restated llama.step / decodeBatch
(model_ref.c: src/gguf/llama.zig:1111-1227, 1939-2043) over host copies of a
device model's GGML bytes, so device and oracle see the same weights.  Used
by tests/ and by bench.py's CPU-baseline leg only."""
from __future__ import annotations

import ctypes as C

import numpy as np


class OracleModel:
    """lo_model over `dm` (a loom_amd.frame.DeviceModel built with
    keep_ggml=True): dm.tensors[name].ggml (device GGML bytes) and dm.f32."""

    def __init__(self, oracle, dm):
        o = oracle
        s = dm.spec
        self.o, self.spec = o, s
        self.keep = []
        self.host = {}

        def host(name):
            a = dm.tensors[name].ggml.cpu().numpy()
            self.host[name] = a
            return a

        def f32(name):
            a = np.ascontiguousarray(dm.f32[name].cpu().numpy(), np.float32)
            self.keep.append(a)
            return a

        def tensor(name, rows, cols, planes=1):
            t = dm.tensors[name]
            return o.Tensor(t.t, host(name).ctypes.data, cols, rows, planes)

        ones_dim, ones_hd = f32("ones_dim"), f32("ones_hd")

        def norm(name, ones):  # the model's own norm weights where it has them
            return f32(name).ctypes.data if name in dm.f32 else ones.ctypes.data

        layers = (o.Layer * s.n_layers)()
        for li in range(s.n_layers):
            p = f"l{li}."
            L = layers[li]
            L.attn_norm = norm(p + "attn_norm", ones_dim)
            L.ffn_norm = norm(p + "ffn_norm", ones_dim)
            L.q_norm = norm(p + "q_norm", ones_hd) if s.qk_norm else None
            L.k_norm = norm(p + "k_norm", ones_hd) if s.qk_norm else None
            L.wq = tensor(p + "wq", s.qd, s.dim)
            L.wk = tensor(p + "wk", s.kvd, s.dim)
            L.wv = tensor(p + "wv", s.kvd, s.dim)
            L.wo = tensor(p + "wo", s.dim, s.qd)
            if s.n_expert:
                L.is_moe = 1
                router = f32(p + "router")
                rb = f32(p + "router_bias") if s.router_bias else None
                L.moe = o.MoeLayer(
                    s.dim, s.moe_ffn,
                    o.RouteCfg(s.n_expert, s.n_used, s.gating, int(s.weights_norm), s.weights_scale),
                    o.Tensor(0, router.ctypes.data, s.dim, s.n_expert, 1),
                    None if rb is None else rb.ctypes.data, None,
                    tensor(p + "gate", s.moe_ffn, s.dim, s.n_expert),
                    tensor(p + "up", s.moe_ffn, s.dim, s.n_expert),
                    tensor(p + "down", s.dim, s.moe_ffn, s.n_expert))
            else:
                L.is_moe = 0
                L.ffn_gate = tensor(p + "ffn_gate", s.ffn, s.dim)
                L.ffn_up = tensor(p + "ffn_up", s.ffn, s.dim)
                L.ffn_down = tensor(p + "ffn_down", s.dim, s.ffn)
        self.layers = layers
        self.model = o.Model(s.dim, s.head_dim, s.n_layers, s.n_heads, s.n_kv_heads, s.vocab,
                             s.ctx_len, s.rope_dim, s.rope_base, s.eps, int(s.rope_neox), 1,
                             tensor("embed", s.vocab, s.dim), norm("out_norm", ones_dim),
                             tensor("output", s.vocab, s.dim), C.cast(layers, C.c_void_p))
        self.cache_bytes = int(o.lib().lo_seq_cache_bytes(C.byref(self.model)))

    def new_seqs(self, n: int):
        seqs = (self.o.Seq * n)()
        bufs = []
        for i in range(n):
            k = np.zeros(self.cache_bytes, np.uint8)
            v = np.zeros(self.cache_bytes, np.uint8)
            bufs += [k, v]
            seqs[i].k_cache, seqs[i].v_cache, seqs[i].pos = k.ctypes.data, v.ctypes.data, 0
        self.keep.append(bufs)
        return seqs, bufs

    def step(self, seq, token: int) -> np.ndarray:
        logits = np.empty(self.spec.vocab, np.float32)
        rc = self.o.lib().lo_step(C.byref(self.model), C.byref(seq), int(token), logits.ctypes.data)
        assert rc == 0
        return logits

    def decode_batch(self, seqs, tokens) -> np.ndarray:
        n = len(tokens)
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty((n, self.spec.vocab), np.float32)
        rc = self.o.lib().lo_decode_batch(C.byref(self.model), C.cast(seqs, C.c_void_p),
                                          toks.ctypes.data, n, out.ctypes.data)
        assert rc == 0
        return out


def attn_heads(om: OracleModel, k_cache: np.ndarray, v_cache: np.ndarray, li: int, pos: int, q: np.ndarray,
               scale: float) -> np.ndarray:
    """backend.attnHeads on the oracle: every query head over cache rows
    [0, pos] of layer li (a lo_seq cache: fp16 bytes as the device keeps)."""
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty(om.spec.n_heads * om.spec.head_dim, np.float32)
    om.o.lib().lo_attn_heads(C.byref(om.model), k_cache.ctypes.data, v_cache.ctypes.data, li, pos,
                             q.ctypes.data, out.ctypes.data, scale)
    return out


def maxrel(got: np.ndarray, want: np.ndarray) -> float:
    return float(np.abs(got - want).max() / max(float(np.abs(want).max()), 1e-30))
