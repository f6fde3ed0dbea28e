"""GGUF v3 (src/gguf/gguf.zig): libloomhip's reader and writer against the
oracle's restated parser (oracle/gguf_ref.py) and the reference's own known
answers for writeMoeFixture's files (the architecture table of
src/gguf/llama.zig:2119-2134 and the fixture constants of gguf.zig:664-686).
CPU only: the GGUF entry points touch no GPU."""
import struct

import numpy as np
import pytest

from loom_amd import gguf
from oracle import gguf_ref

# src/gguf/llama.zig:2129-2134: (arch, qkv_bias, qk_norm, shexp, shexp_gate, n_dense, head_dim, n_layers)
CASES = [("llama", False, False, False, False, 0, 16, 3),
         ("qwen2moe", True, False, True, True, 0, 16, 3),
         ("qwen3moe", False, True, False, False, 0, 24, 3),
         ("glm4moe", True, True, True, False, 1, 16, 3),
         ("gpt-oss", True, False, False, False, 0, 16, 3)]


def _same(ours, ref):
    """The C++ reader's view equals the restated parser's."""
    assert ours.version == ref["version"] and ours.alignment == ref["alignment"]
    assert ours.data_offset == ref["data_offset"] and ours.file_size == ref["file_size"]
    assert list(ours.metadata) == list(ref["metadata"])
    for k, v in ours.metadata.items():
        r = ref["metadata"][k]
        if isinstance(v, np.ndarray):
            assert np.array_equal(v, np.asarray(r, v.dtype)), k
        elif isinstance(r, float):
            assert v == pytest.approx(r, rel=0, abs=0), k
        else:
            assert v == (list(r) if isinstance(r, list) else r), k
        assert ours.kv_types[k] == ref["types"][k] and ours.kv_spans[k] == ref["spans"][k]
    assert [(t.name, t.dims, t.ggml_type, t.offset) for t in ours.tensors] == ref["tensors"]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_moe_fixture_round_trip(tmp_path, case):
    """writeMoeFixture's layout for each architecture, written by the C++
    writer, read back by the C++ reader and by the restated parser: the
    same key/values, spans and tensor table, every tensor's bytes as
    written at a 32-byte aligned offset, and the reference's known answers
    (head_dim from attention.key_length or dim / n_heads, block_count less
    the NextN blocks, which tensors each architecture carries)."""
    arch, qkv_bias, qk_norm, shexp, shexp_gate, n_dense, head_dim, n_layers = case
    path = tmp_path / f"{arch}.gguf"
    kept = {}

    def fill(name, dims):
        rng = np.random.default_rng(abs(hash(name)) % (1 << 32))
        a = ((rng.random(int(np.prod(dims)), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
        kept[name] = a
        return 0, a

    gguf.write_moe_fixture(str(path), 7, arch, fill=fill)
    raw = path.read_bytes()
    ref = gguf_ref.parse(raw)
    with gguf.GgufFile(str(path)) as g:
        _same(g, ref)
        # gguf.zig:8-12 layout
        assert raw[:4] == b"GGUF" and g.version == 3 and g.alignment == 32 and g.data_offset % 32 == 0
        for t in g.tensors:
            assert t.offset % 32 == 0 and t.ggml_type == 0
            assert t.nbytes == 4 * int(np.prod(t.dims))
            assert np.array_equal(t.data.view(np.float32), kept[t.name])
        # the fixture constants (gguf.zig:664-686) and llama.zig's load reading them
        dim = g.get_uint(f"{arch}.embedding_length")
        n_heads = g.get_uint(f"{arch}.attention.head_count")
        hd = g.get_uint(f"{arch}.attention.key_length") or dim // n_heads
        assert (dim, n_heads, g.get_uint(f"{arch}.attention.head_count_kv")) == (64, 4, 2)
        assert hd == head_dim
        assert (hd != dim // n_heads) == (arch == "qwen3moe")
        nextn = g.get_uint(f"{arch}.nextn_predict_layers") or 0
        assert g.get_uint(f"{arch}.block_count") - nextn == n_layers
        assert (g.get_uint(f"{arch}.leading_dense_block_count") or 0) == n_dense
        assert (g.get_uint(f"{arch}.expert_count"), g.get_uint(f"{arch}.expert_used_count"),
                g.get_uint(f"{arch}.expert_feed_forward_length")) == (8, 2, 48)
        last = f"blk.{n_layers - 1}."
        assert (g.find_tensor(last + "attn_q.bias") is not None) == qkv_bias
        assert (g.find_tensor(last + "attn_v.bias") is not None) == qkv_bias
        assert (g.find_tensor(last + "attn_q_norm.weight") is not None) == qk_norm
        assert (g.find_tensor(last + "ffn_gate_shexp.weight") is not None) == shexp
        assert (g.find_tensor(last + "ffn_gate_inp_shexp.weight") is not None) == shexp_gate
        assert g.find_tensor(last + "ffn_gate_exps.weight").dims == (64, 48, 8)
        if n_dense:
            assert g.find_tensor("blk.0.ffn_gate.weight") is not None
            assert g.find_tensor("blk.0.ffn_gate_inp.weight") is None
        # routeCfgFromMeta (src/gguf/moe.zig:63-97): glm4moe gates by sigmoid and renormalises
        assert (g.get_uint(f"{arch}.expert_gating_func") == 2) == (arch == "glm4moe")
        assert len(g.metadata["tokenizer.ggml.tokens"]) == 259
        assert g.metadata["tokenizer.ggml.tokens"][3] == "<0x00>"


def test_getters_follow_parsed_coercions(tmp_path):
    """Parsed.getUint / getFloat / getString / getBool (gguf.zig:97-137):
    unsigned and non-negative signed integers read as uint, a negative one
    does not; integers read as floats; bool reads u/int values as != 0;
    a string is only a string; absent keys read as absent."""
    path = tmp_path / "kv.gguf"
    kvs = [("a.u8", gguf.U8, 200), ("a.i32neg", gguf.I32, -5), ("a.i64", gguf.I64, 7), ("a.f64", gguf.F64, 0.25),
           ("a.bool", gguf.BOOL, True), ("a.str", gguf.STRING, "héllo"), ("a.u64", gguf.U64, 1 << 40),
           ("a.arr_u16", gguf.ARRAY, (gguf.U16, [1, 2, 3])), ("a.nested", gguf.ARRAY, (gguf.I32, [])),
           ("general.alignment", gguf.U32, 64)]
    gguf.write_gguf(str(path), kvs, [("t", (32,), 0, np.arange(32, dtype=np.float32))], alignment=64)
    with gguf.GgufFile(str(path)) as g:
        _same(g, gguf_ref.parse(path.read_bytes()))
        assert g.alignment == 64 and g.data_offset % 64 == 0 and g.tensors[0].offset == 0
        assert g.get_uint("a.u8") == 200 and g.get_uint("a.i32neg") is None and g.get_uint("a.i64") == 7
        assert g.get_uint("a.u64") == 1 << 40
        assert g.get_float("a.f64") == 0.25 and g.get_float("a.u8") == 200.0 and g.get_float("a.i32neg") == -5.0
        assert g.get_float("a.str") is None
        assert g.get_bool("a.bool") is True and g.get_bool("a.u8") is True and g.get_bool("a.str") is None
        assert g.get_string("a.str") == "héllo" and g.get_string("a.u8") is None
        assert g.get_uint("missing") is None
        assert g.metadata["a.arr_u16"] == ("array", gguf.U16, 3)
        assert np.array_equal(g.tensors[0].data.view(np.float32), np.arange(32, dtype=np.float32))


def _header(n_t, n_kv, version=3):
    return struct.pack("<IIQQ", 0x46554747, version, n_t, n_kv)


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


BAD = {
    "NotGguf": b"GGUX" + b"\0" * 60,
    "UnsupportedGgufVersion": _header(0, 0, version=1) + b"\0" * 32,
    "UnsupportedGgufVersion4": _header(0, 0, version=4) + b"\0" * 32,
    "TruncatedGguf": _header(0, 1) + _s("general.name")[:5],
    "TruncatedGgufCount": _header(1 << 21, 0) + b"\0" * 32,
    "UnknownValueType": _header(0, 1) + _s("k") + struct.pack("<I", 13) + b"\0" * 16,
    "ArrayNestingTooDeep": _header(0, 1) + _s("k") + struct.pack("<I", 9) +
    (struct.pack("<IQ", 9, 1)) * 5 + struct.pack("<IQ", 4, 1) + b"\0" * 8,
    "BadTensorDims0": _header(1, 0) + _s("t") + struct.pack("<I", 0) + struct.pack("<IQ", 0, 0) + b"\0" * 32,
    "BadTensorDims9": _header(1, 0) + _s("t") + struct.pack("<I", 9) + b"\0" * 128,
    "BadTensorDimsZero": _header(1, 0) + _s("t") + struct.pack("<IQ", 1, 0) + struct.pack("<IQ", 0, 0) + b"\0" * 32,
    "BadTensorDimsOverflow": _header(1, 0) + _s("t") + struct.pack("<IQQ", 2, 1 << 40, 1 << 40) +
    struct.pack("<IQ", 0, 0) + b"\0" * 32,
    "BadAlignment": _header(0, 1) + _s("general.alignment") + struct.pack("<II", 4, 24) + b"\0" * 32,
}


@pytest.mark.parametrize("name", sorted(BAD))
def test_malformed_files_fail_with_the_reference_error(tmp_path, name):
    """Each of the reference's parse errors (gguf.zig:251-332, with the
    bounds of security issue #29), for the C++ reader and the restated
    parser alike."""
    import loom_amd

    want = name.rstrip("0123456789")
    for suffix in ("Count", "Zero", "Overflow"):
        want = want[:-len(suffix)] if want.endswith(suffix) else want
    path = tmp_path / "bad.gguf"
    path.write_bytes(BAD[name])
    with pytest.raises(gguf_ref.GgufError) as e:
        gguf_ref.parse(BAD[name])
    assert str(e.value) == want
    with pytest.raises(loom_amd.LoomHipError) as e2:
        gguf.GgufFile(str(path))
    assert want in str(e2.value)


def test_every_truncation_fails_cleanly(tmp_path):
    """A fixture cut at any point inside its header reads as TruncatedGguf
    (or a data section past the end), never as a partial parse."""
    import loom_amd

    path = tmp_path / "f.gguf"
    gguf.write_moe_fixture(str(path), 3, "qwen3moe")
    raw = path.read_bytes()
    end = gguf_ref.parse(raw)["data_offset"]
    cut_path = tmp_path / "cut.gguf"
    for cut in list(range(1, 64)) + list(range(64, end, max(1, end // 97))):
        cut_path.write_bytes(raw[:cut])
        with pytest.raises(gguf_ref.GgufError):
            gguf_ref.parse(raw[:cut])
        with pytest.raises(loom_amd.LoomHipError):
            gguf.GgufFile(str(cut_path))


# A qwen3moe file at frame-served shapes, every matrix Q8_0 (any served type
# exercises the same checks; Q8_0 quantizes fastest).
_SHAPE = gguf.FixtureShape(dim=64, n_heads=2, n_kv_heads=1, head_dim=32, ffn=128, n_expert=4, n_used=2,
                           moe_ffn=64, n_layers=2, vocab_bytes=False, vocab=64, context_length=32)


def _q8_file(oracle, path, reshape=None):
    """writeMoeFixture's qwen3moe layout with Q8_0 matrices; ``reshape``
    maps a tensor name to the dims it is written with instead."""
    kvs, table = gguf.moe_fixture_layout("qwen3moe", _SHAPE)
    rng = np.random.default_rng(5)
    tensors = []
    for name, dims in table:
        dims = (reshape or {}).get(name, dims)
        n = int(np.prod(dims))
        if len(dims) == 1 or name.endswith("ffn_gate_inp.weight"):
            tensors.append((name, dims, 0, rng.standard_normal(n).astype(np.float32)))
        else:
            w = (0.02 * rng.standard_normal((n // dims[0], dims[0]))).astype(np.float32)
            tensors.append((name, dims, 8, oracle.quantize(8, w)))
    gguf.write_gguf(str(path), kvs, tensors, alignment=32)


def test_from_gguf_rejects_a_mis_shaped_tensor_before_any_upload(oracle, tmp_path):
    """llama.zig:293-309 expectShape: layer 1's attn_q written as
    [dim, 2*q_dim] (its bytes consistent with those dims) against the q_dim
    rows the metadata implies raises BadTensorShape.  Every tensor is checked
    before the first upload: layer 0's tensors come first in the file, and
    on this GPU-less host an upload would raise a torch error, not this
    ValueError."""
    from loom_amd.frame import DeviceModel

    qd = _SHAPE.n_heads * _SHAPE.head_dim
    path = tmp_path / "bad_q.gguf"
    _q8_file(oracle, path, {"blk.1.attn_q.weight": (_SHAPE.dim, 2 * qd)})
    with gguf.GgufFile(str(path)) as g:
        with pytest.raises(ValueError, match=r"BadTensorShape: tensor blk\.1\.attn_q\.weight"):
            DeviceModel.from_gguf(g)


def test_from_gguf_rejects_a_truncated_tensor_before_any_upload(oracle, tmp_path):
    """llama.zig:258-272 resolve: a file cut inside its last tensor still
    parses (the data section starts inside the file), but that tensor's bytes
    do not lie inside it: TruncatedGguf, before anything is uploaded."""
    from loom_amd.frame import DeviceModel

    path = tmp_path / "cut.gguf"
    _q8_file(oracle, path)
    raw = path.read_bytes()
    path.write_bytes(raw[:-7])
    with gguf.GgufFile(str(path)) as g:
        last = max(g.tensors, key=lambda t: t.offset)
        assert last.data is None and last.nbytes > 0
        with pytest.raises(ValueError, match=f"TruncatedGguf: tensor {last.name}"):
            DeviceModel.from_gguf(g)


def test_tensor_bytes_overflow_reads_as_unknown(tmp_path):
    """ggml.zig:143-153 tensorBytesChecked: an F32 tensor of 2^62 + 1 values
    has a representable element count but 2^64 + 4 bytes.  Unchecked, the
    size wraps to 4 and those 4 bytes pass the in-file test; checked, the
    size reads as unknown (0) and no data pointer is handed out."""
    raw = (_header(1, 0) + _s("t") + struct.pack("<IQ", 1, (1 << 62) + 1) + struct.pack("<IQ", 0, 0))
    raw += b"\0" * ((-len(raw)) % 32) + b"\0" * 64
    path = tmp_path / "wrap.gguf"
    path.write_bytes(raw)
    with gguf.GgufFile(str(path)) as g:
        assert g.tensors[0].dims == ((1 << 62) + 1,)
        assert g.tensors[0].nbytes == 0 and g.tensors[0].data is None
