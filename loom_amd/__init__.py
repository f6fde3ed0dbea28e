"""loom_amd -- MI355X (gfx950) backend for Loom's quantized MoE forward.

The product is ``libloomhip.so`` (hand-written HIP kernels behind the C ABI of
``include/loomhip.h``).  This package loads it with ctypes and mirrors the
reference's compute-backend seam (``src/compute/backend.zig``) in
``loom_amd.backend``.  There is no CPU fallback: if the shared library is
missing, importing the bindings raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libloomhip.so")
HEADER = os.path.join(ROOT, "include", "loomhip.h")

OK, DECLINED, ERR_ARG, ERR_HIP, ERR_INIT = 0, 1, -1, -2, -3
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
GATING_SOFTMAX, GATING_SIGMOID, GATING_SOFTMAX_TOPK = 1, 2, 3
COMBINE_SELECTION, COMBINE_EXPERT_ASC, COMBINE_SELECTION_ADD = 0, 1, 2
KT_GATE_UP, KT_DOWN, KT_DENSE, KT_ATTN, KT_HEAD, KT_QKV = 0, 1, 2, 3, 4, 5
KT_WO, KT_ATTN_SCORES, KT_ATTN_SOFTMAX, KT_ATTN_PV = 6, 7, 8, 9
KT_MLA_ABSORB, KT_MLA_SCORES, KT_MLA_SOFTMAX, KT_MLA_WSUM, KT_MLA_WV = 10, 11, 12, 13, 14
NUMERICS_PARITY, NUMERICS_FAST = 0, 1
KT_NAMES = {KT_GATE_UP: "gate_up", KT_DOWN: "down", KT_DENSE: "dense", KT_ATTN: "attn",
            KT_HEAD: "head", KT_QKV: "qkv", KT_WO: "wo", KT_ATTN_SCORES: "attn_scores",
            KT_ATTN_SOFTMAX: "attn_softmax", KT_ATTN_PV: "attn_pv", KT_MLA_ABSORB: "mla_absorb",
            KT_MLA_SCORES: "mla_scores", KT_MLA_SOFTMAX: "mla_softmax", KT_MLA_WSUM: "mla_wsum",
            KT_MLA_WV: "mla_wv"}


class LoomHipError(RuntimeError):
    pass


class MoeLayerDesc(C.Structure):
    """Mirror of ``loomhip_moe_layer`` in include/loomhip.h."""

    _fields_ = [
        ("dim", C.c_size_t),
        ("ffn", C.c_size_t),
        ("n_expert", C.c_size_t),
        ("n_used", C.c_size_t),
        ("gating", C.c_int),
        ("weights_norm", C.c_int),
        ("weights_scale", C.c_float),
        ("router", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("sel_bias", C.c_void_p),
        ("gate_t", C.c_int),
        ("up_t", C.c_int),
        ("down_t", C.c_int),
        ("gate", C.c_void_p),
        ("up", C.c_void_p),
        ("down", C.c_void_p),
        ("shexp_gate_t", C.c_int),
        ("shexp_up_t", C.c_int),
        ("shexp_down_t", C.c_int),
        ("shexp_gate", C.c_void_p),
        ("shexp_up", C.c_void_p),
        ("shexp_down", C.c_void_p),
        ("shexp_ffn", C.c_size_t),
    ]


class LayerDesc(C.Structure):
    """Mirror of ``loomhip_layer`` in include/loomhip.h."""

    _fields_ = [
        ("attn_norm", C.c_void_p),
        ("ffn_norm", C.c_void_p),
        ("q_norm", C.c_void_p),
        ("k_norm", C.c_void_p),
        ("wq_t", C.c_int),
        ("wk_t", C.c_int),
        ("wv_t", C.c_int),
        ("wo_t", C.c_int),
        ("wq", C.c_void_p),
        ("wk", C.c_void_p),
        ("wv", C.c_void_p),
        ("wo", C.c_void_p),
        ("is_moe", C.c_int),
        ("moe", MoeLayerDesc),
        ("ffn_gate_t", C.c_int),
        ("ffn_up_t", C.c_int),
        ("ffn_down_t", C.c_int),
        ("ffn_gate", C.c_void_p),
        ("ffn_up", C.c_void_p),
        ("ffn_down", C.c_void_p),
        ("ffn", C.c_size_t),
    ]


class ModelDesc(C.Structure):
    """Mirror of ``loomhip_model`` in include/loomhip.h."""

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
        ("embed_t", C.c_int),
        ("embed", C.c_void_p),
        ("out_norm", C.c_void_p),
        ("output_t", C.c_int),
        ("output", C.c_void_p),
        ("layers", C.POINTER(LayerDesc)),
        ("rope_cs", C.c_void_p),
        ("numerics", C.c_int),
        ("ids_out", C.c_void_p),
    ]


class WeightRefDesc(C.Structure):
    """Mirror of ``loomhip_weight_ref`` in include/loomhip.h."""

    _fields_ = [("type", C.c_int), ("data", C.c_void_p), ("len", C.c_size_t)]


class LayerSpecDesc(C.Structure):
    """Mirror of ``loomhip_layer_spec`` (src/compute/cpu.zig:116-138 LayerSpec)."""

    _fields_ = ([("li", C.c_size_t), ("pos", C.c_size_t), ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                 ("eps", C.c_float)] + [(n, WeightRefDesc) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")] +
                [(n, C.c_size_t) for n in ("dim", "ffn", "n_heads", "n_kv_heads", "hd", "rope_dim")] +
                [("rope_base", C.c_float), ("rope_neox", C.c_int), ("attn_scale", C.c_float)])


class GqaLayerDescC(C.Structure):
    """Mirror of ``loomhip_gqa_layer_desc`` (the qwen3moe form of MlaLayerDesc)."""

    _fields_ = ([(n, C.c_void_p) for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")] +
                [(n, WeightRefDesc) for n in ("wq", "wk", "wv", "wo")] + [("is_moe", C.c_int),
                ("router", WeightRefDesc), ("router_bias", C.c_void_p), ("sel_bias", C.c_void_p)] +
                [(n, WeightRefDesc) for n in ("gate", "up", "down", "shexp_gate", "shexp_up", "shexp_down")] +
                [("ffn", C.c_size_t), ("shexp_ffn", C.c_size_t)] +
                [(n, WeightRefDesc) for n in ("dgate", "dup", "ddown")] + [("dffn", C.c_size_t)])


class GqaFrameCfg(C.Structure):
    """Mirror of ``loomhip_gqa_frame_cfg`` (MlaFrameCfg's GQA counterpart)."""

    _fields_ = ([(n, C.c_size_t) for n in ("dim", "n_heads", "n_kv_heads", "head_dim", "rope_dim")] +
                [(n, C.c_float) for n in ("eps", "scale", "rope_base")] + [("rope_neox", C.c_int),
                ("n_expert", C.c_size_t), ("n_used", C.c_size_t), ("gating", C.c_int), ("weights_norm", C.c_int),
                ("weights_scale", C.c_float)])


class MlaLayerDescC(C.Structure):
    """Mirror of ``loomhip_mla_layer_desc`` (src/compute/cpu.zig:73 MlaLayerDesc)."""

    _fields_ = ([("attn_norm", C.c_void_p), ("wq", WeightRefDesc), ("kv_a", WeightRefDesc), ("kv_a_norm", C.c_void_p),
                 ("kv_b", WeightRefDesc), ("attn_out", WeightRefDesc), ("ffn_norm", C.c_void_p), ("is_moe", C.c_int)] +
                [(n, WeightRefDesc) for n in ("router", "gate", "up", "down", "shexp_gate", "shexp_up", "shexp_down")] +
                [("ffn", C.c_size_t), ("shexp_ffn", C.c_size_t)] +
                [(n, WeightRefDesc) for n in ("dgate", "dup", "ddown")] + [("dffn", C.c_size_t)])


class MlaFrameCfgC(C.Structure):
    """Mirror of ``loomhip_mla_frame_cfg`` (src/compute/cpu.zig:74 MlaFrameCfg)."""

    _fields_ = ([(n, C.c_size_t) for n in ("dim", "n_heads", "nope", "rope", "kvr", "v_head_dim")] +
                [(n, C.c_float) for n in ("eps", "scale", "rope_base", "yarn_factor", "yarn_orig_ctx")] +
                [("n_expert", C.c_size_t), ("n_used", C.c_size_t), ("gating", C.c_int), ("weights_norm", C.c_int),
                 ("weights_scale", C.c_float)])


class EcStats(C.Structure):
    """Mirror of ``loomhip_ec_stats`` in include/loomhip.h."""

    _fields_ = [(n, C.c_uint64) for n in ("pin_hits", "lru_hits", "misses", "bytes_read",
                                          "warmup_reads", "warmup_bytes")]


class MoeLayerEcDesc(C.Structure):
    """Mirror of ``loomhip_moe_layer_ec`` in include/loomhip.h."""

    _fields_ = [
        ("dim", C.c_size_t),
        ("ffn", C.c_size_t),
        ("n_expert", C.c_size_t),
        ("n_used", C.c_size_t),
        ("gating", C.c_int),
        ("weights_norm", C.c_int),
        ("weights_scale", C.c_float),
        ("router", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("sel_bias", C.c_void_p),
        ("gate_t", C.c_int),
        ("down_t", C.c_int),
        ("id_base", C.c_size_t),
        ("gate_off", C.c_size_t),
        ("up_off", C.c_size_t),
        ("down_off", C.c_size_t),
        ("shexp_gate_t", C.c_int),
        ("shexp_up_t", C.c_int),
        ("shexp_down_t", C.c_int),
        ("shexp_gate", C.c_void_p),
        ("shexp_up", C.c_void_p),
        ("shexp_down", C.c_void_p),
        ("shexp_ffn", C.c_size_t),
    ]


class MlaAttnDesc(C.Structure):
    """Mirror of ``loomhip_mla_attn`` in include/loomhip.h."""

    _fields_ = [
        ("kvb_type", C.c_int),
        ("wk", C.c_void_p),
        ("wv", C.c_void_p),
        ("n_heads", C.c_size_t),
        ("nope", C.c_size_t),
        ("vd", C.c_size_t),
        ("kvr", C.c_size_t),
        ("rope", C.c_size_t),
        ("scale", C.c_float),
    ]


class ExpertRefDesc(C.Structure):
    """Mirror of ``loomhip_expert_ref`` in include/loomhip.h."""

    _fields_ = [
        ("gate_t", C.c_int),
        ("up_t", C.c_int),
        ("down_t", C.c_int),
        ("gate", C.c_void_p),
        ("up", C.c_void_p),
        ("down", C.c_void_p),
        ("weight", C.c_float),
        ("ffn", C.c_size_t),
    ]


def header_symbols() -> list[str]:
    """Every function name declared in include/loomhip.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(loomhip_[a-z0-9_]+)\s*\(", text)))


_lib = None


def lib() -> C.CDLL:
    """Load libloomhip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LoomHipError(
            f"{LIB_PATH} is missing: build it with `python -m loom_amd.build` "
            "(there is no CPU fallback)")
    # torch ships its own libamdhip64.so.7.  Loading torch first makes
    # libloomhip bind to that same runtime (the SONAMEs match), so torch's
    # device buffers and streams and ours live in one HIP runtime; loading
    # ours first would map a second runtime from /opt/rocm.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    vp, sz, i, f = C.c_void_p, C.c_size_t, C.c_int, C.c_float
    u64 = C.c_uint64
    sig = {
        "loomhip_init": (i, [i]),
        "loomhip_shutdown": (None, []),
        "loomhip_last_error": (C.c_char_p, []),
        "loomhip_take_launch_count": (u64, []),
        "loomhip_version": (C.c_char_p, []),
        "loomhip_profile_kernels": (None, [i]),
        "loomhip_kernel_time": (i, [i, C.POINTER(C.c_double), C.POINTER(u64)]),
        "loomhip_plane_bytes": (sz, [i, sz, sz]),
        "loomhip_ggml_bytes": (sz, [i, sz, sz]),
        "loomhip_register_weights": (i, [i, vp, sz, sz, sz, C.POINTER(vp)]),
        "loomhip_clear_weight_cache": (None, []),
        "loomhip_resident_bytes": (sz, []),
        "loomhip_repack_dev": (i, [i, vp, vp, sz, sz, sz, vp]),
        "loomhip_synth_weights_dev": (i, [i, vp, sz, sz, sz, u64, f, vp]),
        "loomhip_matvec": (i, [i, vp, vp, vp, sz, sz]),
        "loomhip_matmul": (i, [i, vp, vp, vp, sz, sz, sz]),
        "loomhip_dequant_row": (i, [i, vp, vp, sz, sz]),
        "loomhip_moe_route": (i, [vp, vp, sz, sz, i, i, f, vp, vp]),
        "loomhip_moe_ffn_routed": (i, [vp, sz, sz, vp, vp, sz, sz, i, i, f, i, vp, i, vp, i, vp,
                                       i, vp, i, vp, i, vp, sz, sz, i, vp]),
        "loomhip_matvec_dev": (i, [i, vp, vp, vp, sz, sz, sz, vp]),
        "loomhip_dequant_dev": (i, [i, vp, vp, sz, sz, vp]),
        "loomhip_moe_layer_dev": (i, [C.POINTER(MoeLayerDesc), vp, sz, i, vp, vp, vp, vp]),
        "loomhip_moe_layer_dev_noalloc": (i, [C.POINTER(MoeLayerDesc), vp, sz, i, vp, vp, vp, vp]),
        "loomhip_token_frame_dev": (i, [C.POINTER(ModelDesc), vp, vp, sz, vp, vp, vp, vp, vp]),
        "loomhip_frame_check": (i, [C.POINTER(ModelDesc), sz]),
        "loomhip_attn_init": (i, [sz, sz, sz]),
        "loomhip_has_kv_cache": (i, []),
        "loomhip_release_kv_cache": (None, []),
        "loomhip_kv_append": (i, [sz, sz, vp, vp, sz]),
        "loomhip_read_kv": (i, [sz, sz, vp, vp, sz]),
        "loomhip_attn_heads": (i, [sz, sz, vp, vp, sz, sz, sz, C.c_float]),
        "loomhip_begin_frame": (i, []),
        "loomhip_frame_open": (i, []),
        "loomhip_frame_load_x": (i, [vp, sz]),
        "loomhip_layer_block": (i, [C.POINTER(LayerSpecDesc)]),
        "loomhip_end_frame": (i, []),
        "loomhip_frame_store_x": (i, [vp, sz]),
        "loomhip_gqa_token_frame": (i, [C.POINTER(GqaLayerDescC), sz, C.POINTER(GqaFrameCfg), vp, sz, vp,
                                        WeightRefDesc, vp, sz]),
        "loomhip_host_alloc": (vp, [sz]),
        "loomhip_host_free": (None, [vp]),
        "loomhip_ec_create": (i, [sz, sz, sz, sz, C.POINTER(vp)]),
        "loomhip_ec_destroy": (None, [vp]),
        "loomhip_ec_set_source": (i, [vp, sz, vp, sz]),
        "loomhip_ec_pin": (i, [vp, vp, sz]),
        "loomhip_ec_get": (i, [vp, sz, vp, C.POINTER(vp)]),
        "loomhip_ec_release": (i, [vp, vp]),
        "loomhip_ec_prefetch": (i, [vp, vp, sz]),
        "loomhip_ec_get_stats": (i, [vp, C.POINTER(EcStats)]),
        "loomhip_ec_access_counts": (i, [vp, vp, sz]),
        "loomhip_ec_clear": (i, [vp]),
        "loomhip_moe_layer_cached": (i, [C.POINTER(MoeLayerEcDesc), vp, vp, sz, vp, vp, vp, vp]),
        "loomhip_moe_ffn_block": (i, [vp, sz, C.POINTER(ExpertRefDesc), sz, vp]),
        "loomhip_moe_ffn_block_stats": (i, [C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
        "loomhip_moe_ffn_block_prefetch": (i, [sz, C.POINTER(ExpertRefDesc), sz]),
        "loomhip_register_arena": (i, [vp, sz]),
        # GGUF (structs from loom_amd.gguf, passed by reference as void *)
        "loomhip_gguf_open": (i, [C.c_char_p, vp]),
        "loomhip_gguf_close": (None, [vp]),
        "loomhip_gguf_get_info": (i, [vp, vp]),
        "loomhip_gguf_get_tensor": (i, [vp, sz, vp]),
        "loomhip_gguf_find_tensor": (i, [vp, C.c_char_p, vp]),
        "loomhip_gguf_get_kv": (i, [vp, sz, vp]),
        "loomhip_gguf_get_uint": (i, [vp, C.c_char_p, vp]),
        "loomhip_gguf_get_float": (i, [vp, C.c_char_p, vp]),
        "loomhip_gguf_get_string": (i, [vp, C.c_char_p, vp, vp]),
        "loomhip_gguf_get_bool": (i, [vp, C.c_char_p, vp]),
        "loomhip_gguf_writer_begin": (i, [u64, vp]),
        "loomhip_gguf_writer_kv": (i, [vp, C.c_char_p, C.c_uint32, vp, u64, C.c_uint32]),
        "loomhip_gguf_writer_tensor": (i, [vp, C.c_char_p, C.c_uint32, vp, C.c_uint32, vp, u64]),
        "loomhip_gguf_writer_finish": (i, [vp, C.c_char_p]),
        "loomhip_gguf_writer_abort": (None, [vp]),
        "loomhip_materialize_arenas": (sz, []),
        "loomhip_mla_init": (i, [sz, sz, sz, sz]),
        "loomhip_has_mla_cache": (i, []),
        "loomhip_mla_append": (i, [sz, sz, vp, sz, vp, sz]),
        "loomhip_mla_read_cache": (i, [sz, sz, vp, sz, vp, sz]),
        "loomhip_mla_set_wk": (i, [sz, vp, sz]),
        "loomhip_mla_attn_heads": (i, [sz, sz, vp, sz, vp, sz, i, vp, sz, vp, sz, sz, sz, sz, f]),
        "loomhip_mla_split_kvb_dev": (i, [i, vp, sz, sz, sz, sz, vp, vp, vp]),
        "loomhip_mla_attn_dev": (i, [C.POINTER(MlaAttnDesc), vp, vp, sz, vp, vp, vp, vp, vp]),
        "loomhip_mla_layer_tail": (i, [sz, sz, vp, sz, vp, sz, vp, sz, i, vp, sz, i, vp, vp, f, i, vp, vp, i, vp, i,
                                       vp, i, vp, i, vp, i, vp, i, vp, sz, sz, sz, sz, i, i, f, sz, sz, sz, f]),
        "loomhip_mla_layer_tail_dev": (i, [C.POINTER(MlaAttnDesc), vp, vp, sz, vp, vp, i, vp, vp, f,
                                           C.POINTER(MoeLayerDesc), vp, vp]),
        "loomhip_mla_token_frame": (i, [C.POINTER(MlaLayerDescC), sz, C.POINTER(MlaFrameCfgC), vp, sz, vp,
                                        WeightRefDesc, vp, sz]),
        "loomhip_mla_layer_cached_dev": (i, [C.POINTER(MlaAttnDesc), C.POINTER(vp), C.POINTER(vp), sz, sz, vp, vp, i,
                                             vp, vp, f, C.POINTER(MoeLayerEcDesc), vp, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    return lib().loomhip_last_error().decode()


def check(rc: int, what: str = "") -> int:
    """Raise on errors; return rc (OK or DECLINED)."""
    if rc < 0:
        raise LoomHipError(f"{what}: {last_error()} (rc={rc})")
    return rc


def init(device: int = 0) -> None:
    check(lib().loomhip_init(device), "loomhip_init")


def take_launch_count() -> int:
    return int(lib().loomhip_take_launch_count())


def plane_bytes(t: int, rows: int, cols: int) -> int:
    return int(lib().loomhip_plane_bytes(t, rows, cols))


def ggml_bytes(t: int, rows: int, cols: int) -> int:
    return int(lib().loomhip_ggml_bytes(t, rows, cols))
