"""GGUF v3 files through libloomhip's reader and writer (src/gguf/gguf.zig).

``GgufFile`` parses a file (gguf.zig:251-332: header, metadata key/values,
tensor table) with the whole file mapped read-only, so each tensor's bytes
are a numpy view into the mapping; the getters follow ``Parsed``'s coercions
(gguf.zig:97-144).  ``write_gguf`` lays a file out the way the reference's
fixture writers do (gguf.zig:643-912), and ``moe_fixture_layout`` /
``write_moe_fixture`` restate ``writeMoeFixture``'s key/values and tensor
table for its five architectures, with the shapes and the tensor bytes left
to the caller (the reference fills every tensor with f32 noise; a quantized
fixture carries GGML blocks instead).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import check, lib

# GGUF value types (gguf.zig:18-33)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32,
           F32: np.float32, BOOL: np.uint8, U64: np.uint64, I64: np.int64, F64: np.float64}


class GgufInfo(C.Structure):
    _fields_ = [("version", C.c_uint32), ("alignment", C.c_uint64), ("n_tensors", C.c_uint64),
                ("n_kv", C.c_uint64), ("data_offset", C.c_uint64), ("file_size", C.c_uint64),
                ("base", C.c_void_p)]


class GgufTensorDesc(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 8),
                ("ggml_type", C.c_uint32), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("data", C.c_void_p)]


class GgufKvDesc(C.Structure):
    _fields_ = [("key", C.c_char_p), ("type", C.c_uint32), ("kind", C.c_int), ("i", C.c_int64),
                ("u", C.c_uint64), ("f", C.c_double), ("s", C.c_void_p), ("s_len", C.c_size_t),
                ("elem_type", C.c_uint32), ("count", C.c_uint64), ("strs", C.POINTER(C.c_char_p)),
                ("f32s", C.POINTER(C.c_float)), ("i32s", C.POINTER(C.c_int32)),
                ("span_start", C.c_uint64), ("span_end", C.c_uint64)]


@dataclass
class TensorInfo:
    """gguf.zig:36-47: name, dims (dims[0] is the row length), GGML type,
    offset from the data section; nbytes and data (a uint8 view into the
    mapping) for the types whose block geometry is known."""

    name: str
    dims: tuple
    ggml_type: int
    offset: int
    nbytes: int
    data: np.ndarray | None


class GgufFile:
    """A parsed, mapped GGUF file (``loomhip_gguf_open``); close() unmaps it,
    after which the tensor views must not be used."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().loomhip_gguf_open(str(path).encode(), C.byref(h)), "gguf_open")
        self._h = h
        info = GgufInfo()
        check(lib().loomhip_gguf_get_info(h, C.byref(info)), "gguf_get_info")
        self.version, self.alignment = info.version, info.alignment
        self.data_offset, self.file_size = info.data_offset, info.file_size
        self.metadata = {}
        self.kv_types = {}
        self.kv_spans = {}
        for i in range(info.n_kv):
            kv = GgufKvDesc()
            check(lib().loomhip_gguf_get_kv(h, i, C.byref(kv)), "gguf_get_kv")
            key = kv.key.decode()
            self.metadata[key] = _kv_value(kv)
            self.kv_types[key] = kv.type
            self.kv_spans[key] = (kv.span_start, kv.span_end)
        self.tensors: list[TensorInfo] = []
        for i in range(info.n_tensors):
            t = GgufTensorDesc()
            check(lib().loomhip_gguf_get_tensor(h, i, C.byref(t)), "gguf_get_tensor")
            data = None
            if t.data and t.nbytes:
                data = np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_uint8)), shape=(t.nbytes,))
            self.tensors.append(TensorInfo(t.name.decode(), tuple(t.dims[:t.n_dims]), t.ggml_type, t.offset,
                                           t.nbytes, data))
        self._by_name = {t.name: t for t in self.tensors}

    # Parsed's getters (gguf.zig:97-144)
    def get_uint(self, key: str):
        v = C.c_uint64()
        return v.value if lib().loomhip_gguf_get_uint(self._h, key.encode(), C.byref(v)) == 0 else None

    def get_float(self, key: str):
        v = C.c_double()
        return v.value if lib().loomhip_gguf_get_float(self._h, key.encode(), C.byref(v)) == 0 else None

    def get_string(self, key: str):
        s, n = C.c_void_p(), C.c_size_t()
        if lib().loomhip_gguf_get_string(self._h, key.encode(), C.byref(s), C.byref(n)) != 0:
            return None
        return C.string_at(s, n.value).decode()

    def get_bool(self, key: str):
        v = C.c_int()
        return bool(v.value) if lib().loomhip_gguf_get_bool(self._h, key.encode(), C.byref(v)) == 0 else None

    def find_tensor(self, name: str) -> TensorInfo | None:
        return self._by_name.get(name)

    def close(self) -> None:
        if self._h:
            lib().loomhip_gguf_close(self._h)
            self._h = None
            for t in self.tensors:
                t.data = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _kv_value(kv: GgufKvDesc):
    k = kv.kind
    if k == 0:
        return int(kv.i)
    if k == 1:
        return int(kv.u)
    if k == 2:
        return float(kv.f)
    if k == 3:
        return bool(kv.u)
    if k == 4:
        return C.string_at(kv.s, kv.s_len).decode("utf-8", "surrogateescape")
    if k == 5:
        return [kv.strs[j].decode("utf-8", "surrogateescape") for j in range(kv.count)]
    if k == 6:
        return np.ctypeslib.as_array(kv.f32s, shape=(kv.count,)).copy() if kv.count else np.zeros(0, np.float32)
    if k == 7:
        return np.ctypeslib.as_array(kv.i32s, shape=(kv.count,)).copy() if kv.count else np.zeros(0, np.int32)
    return ("array", int(kv.elem_type), int(kv.count))


def write_gguf(path: str, kvs: list, tensors: list, alignment: int = 32) -> None:
    """kvs: (key, value type, value) -- scalars, str, or (elem type, list) for
    an array; tensors: (name, dims, ggml type, bytes), in file order."""
    w = C.c_void_p()
    check(lib().loomhip_gguf_writer_begin(alignment, C.byref(w)), "gguf_writer_begin")
    keep = []
    try:
        for key, vt, val in kvs:
            if vt == STRING:
                b = val.encode()
                rc = lib().loomhip_gguf_writer_kv(w, key.encode(), vt, b, len(b), 0)
            elif vt == ARRAY:
                et, items = val
                if et == STRING:
                    arr = (C.c_char_p * max(1, len(items)))(*[s.encode() for s in items])
                    keep.append(arr)
                    rc = lib().loomhip_gguf_writer_kv(w, key.encode(), vt, C.cast(arr, C.c_void_p), len(items), et)
                else:
                    a = np.ascontiguousarray(np.asarray(items, _SCALAR[et]))
                    keep.append(a)
                    rc = lib().loomhip_gguf_writer_kv(w, key.encode(), vt, a.ctypes.data_as(C.c_void_p), a.size, et)
            else:
                a = np.asarray([val], _SCALAR[vt])
                keep.append(a)
                rc = lib().loomhip_gguf_writer_kv(w, key.encode(), vt, a.ctypes.data_as(C.c_void_p), 1, 0)
            check(rc, f"gguf_writer_kv {key}")
        for name, dims, t, data in tensors:
            d = (C.c_uint64 * len(dims))(*dims)
            b = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                                     else np.asarray(data).view(np.uint8).ravel())
            keep.append(b)
            check(lib().loomhip_gguf_writer_tensor(w, name.encode(), len(dims), d, t,
                                                   b.ctypes.data_as(C.c_void_p), b.size), f"gguf_writer_tensor {name}")
    except Exception:
        lib().loomhip_gguf_writer_abort(w)
        raise
    check(lib().loomhip_gguf_writer_finish(w, str(path).encode()), "gguf_writer_finish")


# ---- writeMoeFixture's layout (gguf.zig:643-912) ------------------------------

ARCHES = ("llama", "qwen2moe", "qwen3moe", "glm4moe", "gpt-oss")


@dataclass
class FixtureShape:
    """The fixture's sizes; the defaults are the reference's (gguf.zig:664-686)."""

    dim: int = 64
    n_heads: int = 4
    n_kv_heads: int = 2
    head_dim: int | None = None  # None: 24 for qwen3moe, dim / n_heads otherwise
    ffn: int = 128
    n_expert: int = 8
    n_used: int = 2
    moe_ffn: int = 48
    n_layers: int = 3
    vocab_bytes: bool = True     # the byte-fallback vocab: 3 + 256 tokens
    vocab: int = 259
    context_length: int = 256
    rope_base: float = 10000.0
    eps: float = 1e-6


def moe_fixture_layout(arch: str, shape: FixtureShape | None = None):
    """(kvs, tensors) of writeMoeFixture for `arch`: kvs as write_gguf takes
    them, tensors as (name, dims) in file order."""
    if arch not in ARCHES:
        raise ValueError(f"UnsupportedArchitecture: {arch}")
    s = shape or FixtureShape()
    is_qwen2, is_qwen3, is_glm, is_oai = (arch == a for a in ("qwen2moe", "qwen3moe", "glm4moe", "gpt-oss"))
    qkv_bias = is_qwen2 or is_glm or is_oai
    qk_norm = is_qwen3 or is_glm
    shexp = is_qwen2 or is_glm
    post_norm = is_glm or is_oai
    sigmoid = is_glm
    n_dense = 1 if is_glm else 0
    nextn = 1 if is_glm else 0
    head_dim = s.head_dim if s.head_dim is not None else (24 if is_qwen3 else s.dim // s.n_heads)
    rope_dim = head_dim // 2 if is_glm else head_dim
    n_shared = 1 if shexp else 0
    shexp_ffn = s.ffn if is_qwen2 else n_shared * s.moe_ffn
    n_blocks = s.n_layers + nextn
    vocab = 3 + 256 if s.vocab_bytes else s.vocab

    kvs = [("general.architecture", STRING, arch), ("general.name", STRING, f"loom {arch} fixture"),
           ("general.alignment", U32, 32)]

    def k(name, vt, v):
        kvs.append((f"{arch}.{name}", vt, v))

    k("block_count", U32, n_blocks)
    k("context_length", U32, s.context_length)
    k("embedding_length", U32, s.dim)
    k("feed_forward_length", U32, s.ffn)
    k("attention.head_count", U32, s.n_heads)
    k("attention.head_count_kv", U32, s.n_kv_heads)
    k("attention.layer_norm_rms_epsilon", F32, s.eps)
    k("rope.dimension_count", U32, rope_dim)
    k("rope.freq_base", F32, s.rope_base)
    k("expert_count", U32, s.n_expert)
    k("expert_used_count", U32, s.n_used)
    k("expert_feed_forward_length", U32, s.moe_ffn)
    if is_qwen3:
        k("attention.key_length", U32, head_dim)
    if is_oai:
        k("attention.sliding_window", U32, 4)
        k("rope.scaling.type", STRING, "yarn")
        k("rope.scaling.factor", F32, 32.0)
        k("rope.scaling.original_context_length", F32, 4096.0)
    if shexp:
        k("expert_shared_count", U32, n_shared)
        k("expert_shared_feed_forward_length", U32, shexp_ffn)
    if n_dense:
        k("leading_dense_block_count", U32, n_dense)
    if nextn:
        k("nextn_predict_layers", U32, nextn)
    if sigmoid:
        k("expert_gating_func", U32, 2)
        k("expert_weights_norm", BOOL, True)
        k("expert_weights_scale", F32, 1.0)
    kvs.append(("tokenizer.ggml.model", STRING, "llama"))
    if s.vocab_bytes:
        tokens = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
        types = [2, 3, 3] + [6] * 256
    else:
        tokens = ["<unk>", "<s>", "</s>"] + [f"t{j}" for j in range(3, vocab)]
        types = [2, 3, 3] + [1] * (vocab - 3)
    kvs.append(("tokenizer.ggml.tokens", ARRAY, (STRING, tokens)))
    kvs.append(("tokenizer.ggml.scores", ARRAY, (F32, [0.0] * vocab)))
    kvs.append(("tokenizer.ggml.token_type", ARRAY, (I32, types)))
    kvs.append(("tokenizer.ggml.bos_token_id", U32, 1))
    kvs.append(("tokenizer.ggml.eos_token_id", U32, 2))
    kvs.append(("tokenizer.ggml.unknown_token_id", U32, 0))

    dim, E = s.dim, s.n_expert
    q_dim, kv_dim = s.n_heads * head_dim, s.n_kv_heads * head_dim
    t = [("token_embd.weight", (dim, vocab)), ("output_norm.weight", (dim,)), ("output.weight", (dim, vocab))]
    for li in range(n_blocks):
        p = f"blk.{li}."
        t += [(p + "attn_norm.weight", (dim,)), (p + "attn_q.weight", (dim, q_dim)),
              (p + "attn_k.weight", (dim, kv_dim)), (p + "attn_v.weight", (dim, kv_dim)),
              (p + "attn_output.weight", (q_dim, dim))]
        if qkv_bias:
            t += [(p + "attn_q.bias", (q_dim,)), (p + "attn_k.bias", (kv_dim,)), (p + "attn_v.bias", (kv_dim,))]
        if qk_norm:
            t += [(p + "attn_q_norm.weight", (head_dim,)), (p + "attn_k_norm.weight", (head_dim,))]
        if is_oai:
            t += [(p + "attn_sinks.weight", (s.n_heads,)), (p + "attn_output.bias", (dim,))]
        t.append((p + ("post_attention_norm.weight" if post_norm else "ffn_norm.weight"), (dim,)))
        if li < n_dense:
            t += [(p + "ffn_gate.weight", (dim, s.ffn)), (p + "ffn_up.weight", (dim, s.ffn)),
                  (p + "ffn_down.weight", (s.ffn, dim))]
            continue
        t.append((p + "ffn_gate_inp.weight", (dim, E)))
        if sigmoid:
            t.append((p + "exp_probs_b.bias", (E,)))
        t += [(p + "ffn_gate_exps.weight", (dim, s.moe_ffn, E)), (p + "ffn_up_exps.weight", (dim, s.moe_ffn, E)),
              (p + "ffn_down_exps.weight", (s.moe_ffn, dim, E))]
        if is_oai:
            t += [(p + "ffn_gate_inp.bias", (E,)), (p + "ffn_gate_exps.bias", (s.moe_ffn, E)),
                  (p + "ffn_up_exps.bias", (s.moe_ffn, E)), (p + "ffn_down_exps.bias", (dim, E))]
        if shexp:
            t += [(p + "ffn_gate_shexp.weight", (dim, shexp_ffn)), (p + "ffn_up_shexp.weight", (dim, shexp_ffn)),
                  (p + "ffn_down_shexp.weight", (shexp_ffn, dim))]
            if is_qwen2:
                t.append((p + "ffn_gate_inp_shexp.weight", (dim, 1)))
    if nextn:
        p = f"blk.{s.n_layers}.nextn."
        t += [(p + "enorm.weight", (dim,)), (p + "hnorm.weight", (dim,)), (p + "eh_proj.weight", (2 * dim, dim)),
              (p + "embed_tokens.weight", (dim, vocab)), (p + "shared_head_norm.weight", (dim,)),
              (p + "shared_head_head.weight", (dim, vocab))]
    return kvs, t


def write_moe_fixture(path: str, seed: int, arch: str, shape: FixtureShape | None = None, fill=None) -> None:
    """writeMoeFixture's file.  ``fill(name, dims) -> (ggml type, bytes)``
    gives each tensor's contents; by default f32 values uniform in [-0.1,
    0.1) from a numpy generator seeded with `seed` (the reference draws its
    own generator's values of the same range)."""
    kvs, table = moe_fixture_layout(arch, shape)
    rng = np.random.default_rng(seed)

    def f32_noise(name, dims):
        n = int(np.prod(dims))
        return 0, ((rng.random(n, dtype=np.float32) - np.float32(0.5)) * np.float32(0.2)).astype(np.float32)

    fill = fill or f32_noise
    tensors = []
    for name, dims in table:
        t, data = fill(name, dims)
        tensors.append((name, dims, t, data))
    write_gguf(path, kvs, tensors, alignment=32)


__all__ = ["GgufFile", "TensorInfo", "write_gguf", "moe_fixture_layout", "write_moe_fixture", "FixtureShape",
           "ARCHES"]
