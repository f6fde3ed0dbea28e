"""TEST INFRASTRUCTURE: a plain-Python restatement of the reference's GGUF v3
parser (src/gguf/gguf.zig:189-332 readValueDepth / parse; layout
gguf.zig:8-12), the checker of libloomhip's C++ reader.  Only tests/ use it.

parse(data) returns a dict {version, alignment, metadata: {key: value},
types: {key: value type}, spans: {key: (start, end)}, tensors: [(name,
dims, ggml_type, offset)], data_offset, file_size} or raises GgufError whose
message is the reference's error name."""
from __future__ import annotations

import struct

MAGIC = 0x46554747


class GgufError(Exception):
    pass


class _Cur:
    def __init__(self, buf: bytes):
        self.b, self.p = buf, 0

    def need(self, n: int) -> bytes:  # gguf.zig:152-157
        if self.p + n > len(self.b):
            raise GgufError("TruncatedGguf")
        s = self.b[self.p:self.p + n]
        self.p += n
        return s

    def u32(self) -> int:
        return struct.unpack("<I", self.need(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.need(8))[0]

    def str(self) -> str:  # gguf.zig:164-168: a 16 MB cap
        n = self.u64()
        if n > 1 << 24:
            raise GgufError("TruncatedGguf")
        return self.need(n).decode("utf-8", "surrogateescape")


def _value(c: _Cur, vt: int, depth: int = 0):
    """gguf.zig:189-247: scalars, strings, and string / f32 / i32 arrays
    kept; other arrays walked and summarised as ('array', elem, count)."""
    if depth > 4:
        raise GgufError("ArrayNestingTooDeep")
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}
    if vt in fmt:
        size = struct.calcsize(fmt[vt])
        v = struct.unpack(fmt[vt], c.need(size))[0]
        return float(v) if vt in (6, 12) else int(v)
    if vt == 7:
        return c.need(1)[0] != 0
    if vt == 8:
        return c.str()
    if vt == 9:
        et = c.u32()
        n = c.u64()
        if n > 1 << 24:
            raise GgufError("TruncatedGguf")
        if et == 8:
            return [c.str() for _ in range(n)]
        if et == 6:
            return [struct.unpack("<f", c.need(4))[0] for _ in range(n)]
        if et == 5:
            return [struct.unpack("<i", c.need(4))[0] for _ in range(n)]
        for _ in range(n):
            _value(c, et, depth + 1)
        return ("array", et, n)
    raise GgufError("UnknownValueType")


def parse(data: bytes) -> dict:
    """gguf.zig:251-332."""
    c = _Cur(data[:64 << 20])
    if c.u32() != MAGIC:
        raise GgufError("NotGguf")
    version = c.u32()
    if version < 2 or version > 3:
        raise GgufError("UnsupportedGgufVersion")
    n_t, n_kv = c.u64(), c.u64()
    if n_t > 1 << 20 or n_kv > 1 << 20:
        raise GgufError("TruncatedGguf")
    meta, types, spans = {}, {}, {}
    for _ in range(n_kv):
        start = c.p
        key = c.str()
        vt = c.u32()
        meta[key] = _value(c, vt)
        types[key] = vt
        spans[key] = (start, c.p)
    tensors = []
    for _ in range(n_t):
        name = c.str()
        nd = c.u32()
        if nd == 0 or nd > 8:
            raise GgufError("BadTensorDims")
        dims, elems = [], 1
        for _ in range(nd):
            d = c.u64()
            if d == 0:
                raise GgufError("BadTensorDims")
            elems *= d
            if elems >= 1 << 64:
                raise GgufError("BadTensorDims")
            dims.append(d)
        t = c.u32()
        off = c.u64()
        tensors.append((name, tuple(dims), t, off))
    alignment = 32
    if "general.alignment" in meta:
        v, vt = meta["general.alignment"], types["general.alignment"]
        if vt in (0, 2, 4, 10):
            alignment = v
        elif vt in (1, 3, 5, 11) and v > 0:
            alignment = v
    if alignment == 0 or alignment & (alignment - 1):
        raise GgufError("BadAlignment")
    data_offset = (c.p + alignment - 1) // alignment * alignment
    if data_offset > len(data):
        raise GgufError("TruncatedGguf")
    return {"version": version, "alignment": alignment, "metadata": meta, "types": types, "spans": spans,
            "tensors": tensors, "data_offset": data_offset, "file_size": len(data)}
