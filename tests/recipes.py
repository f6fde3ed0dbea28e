"""The configs' input recipe (BASELINE.json configs 1 and 3): weights drawn
N(0, 0.02) and quantized by the oracle's quantizers -- the reference's Q4_0
rule (src/gguf/ggml.zig:1861) and GGUF's Q4_K / Q6_K rules -- plane by plane,
in a thread pool (the quantizer releases the GIL), cached per argument set
within a test session."""
from __future__ import annotations

import concurrent.futures as cf
import functools

import numpy as np

from loom_amd import gguf

STD = 0.02


@functools.lru_cache(maxsize=16)
def planes(t: int, rows: int, cols: int, n: int, seed: int) -> np.ndarray:
    """n planes of [rows][cols] N(0, 0.02) weights quantized to type t, as
    one GGML byte array (plane-major)."""
    import oracle as o

    def one(p):
        w = o.normal(rows * cols, seed * 1000 + p, 0.0, STD).reshape(rows, cols)
        return o.quantize(t, w)

    with cf.ThreadPoolExecutor(min(8, max(1, n))) as ex:
        parts = list(ex.map(one, range(n)))
    return np.concatenate(parts)  # shared by the cache: callers must not write to it


def stories15m_gguf(path: str, seed: int, vocab: int = 32000, ctx_len: int = 256) -> None:
    """Config 1 as a GGUF file: the stories15M shape (dim 288, 6 layers, 6
    heads of 48, SwiGLU ffn 768, llama architecture, NORM rope), every matrix
    Q4_0 from N(0, 0.02), norms 1."""
    Q4_0 = 2
    dim, n_layers, heads, ffn = 288, 6, 6, 768
    kvs = [("general.architecture", gguf.STRING, "llama"), ("general.alignment", gguf.U32, 32),
           ("llama.block_count", gguf.U32, n_layers), ("llama.context_length", gguf.U32, ctx_len),
           ("llama.embedding_length", gguf.U32, dim), ("llama.feed_forward_length", gguf.U32, ffn),
           ("llama.attention.head_count", gguf.U32, heads), ("llama.attention.head_count_kv", gguf.U32, heads),
           ("llama.attention.layer_norm_rms_epsilon", gguf.F32, 1e-5),
           ("llama.rope.dimension_count", gguf.U32, dim // heads), ("llama.rope.freq_base", gguf.F32, 10000.0)]
    ones = np.ones(dim, np.float32)
    k = iter(range(1, 1000))
    t = [("token_embd.weight", (dim, vocab), Q4_0, planes(Q4_0, vocab, dim, 1, seed * 100 + next(k))),
         ("output_norm.weight", (dim,), 0, ones),
         ("output.weight", (dim, vocab), Q4_0, planes(Q4_0, vocab, dim, 1, seed * 100 + next(k)))]
    for li in range(n_layers):
        p = f"blk.{li}."
        mat = lambda rows, cols: planes(Q4_0, rows, cols, 1, seed * 100 + next(k))  # noqa: E731
        t += [(p + "attn_norm.weight", (dim,), 0, ones), (p + "attn_q.weight", (dim, dim), Q4_0, mat(dim, dim)),
              (p + "attn_k.weight", (dim, dim), Q4_0, mat(dim, dim)),
              (p + "attn_v.weight", (dim, dim), Q4_0, mat(dim, dim)),
              (p + "attn_output.weight", (dim, dim), Q4_0, mat(dim, dim)), (p + "ffn_norm.weight", (dim,), 0, ones),
              (p + "ffn_gate.weight", (dim, ffn), Q4_0, mat(ffn, dim)),
              (p + "ffn_up.weight", (dim, ffn), Q4_0, mat(ffn, dim)),
              (p + "ffn_down.weight", (ffn, dim), Q4_0, mat(dim, ffn))]
    gguf.write_gguf(path, kvs, t, alignment=32)
