"""Independent numpy decoders for the GGML block formats (test helper).

Written from the format description (block byte offsets, nibble/bit
placement), vectorised over whole tensors, and structured differently from the
C oracle's per-block loops, so an indexing or transposition slip in either one
shows up as a mismatch.  Float arithmetic is done in float32 in the same
two-rounding form the format defines ((d*sc)*q - (dmin*m)), so the comparison
with the oracle's dequant is bit-exact.
"""
import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14


def _f16(lo, hi):
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float32)


def dequant_q4_0(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    b = raw.reshape(rows, cols // 32, 18)
    d = _f16(b[..., 0], b[..., 1])[..., None]
    qs = b[..., 2:]
    lo = (qs & 0xF).astype(np.int32) - 8
    hi = (qs >> 4).astype(np.int32) - 8
    v = np.concatenate([lo, hi], axis=-1).astype(np.float32)  # lanes 0..15 low, 16..31 high
    return (v * d).reshape(rows, cols)


def dequant_q8_0(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    b = raw.reshape(rows, cols // 32, 34)
    d = _f16(b[..., 0], b[..., 1])[..., None]
    q = b[..., 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(rows, cols)


def q4k_scales(sc12: np.ndarray):
    """6-bit (scale, min) pairs for the 8 groups from the 12 packed bytes."""
    s = sc12.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    mn = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, mn


def q4k_quants(raw: np.ndarray, rows: int, cols: int):
    """(q [rows, nb, 8, 32] in 0..15, sc, mn [rows, nb, 8], d, dmin [rows, nb])."""
    b = raw.reshape(rows, cols // 256, 144)
    d = _f16(b[..., 0], b[..., 1])
    dmin = _f16(b[..., 2], b[..., 3])
    sc, mn = q4k_scales(b[..., 4:16])
    qs = b[..., 16:].reshape(rows, cols // 256, 4, 32)  # 4 chunks of 32 bytes
    lo = qs & 0xF  # group 2c
    hi = qs >> 4  # group 2c+1
    q = np.stack([lo, hi], axis=3).reshape(rows, cols // 256, 8, 32).astype(np.int32)
    return q, sc, mn, d, dmin


def dequant_q4_k(raw, rows, cols):
    q, sc, mn, d, dmin = q4k_quants(raw, rows, cols)
    d1 = (d[..., None] * sc.astype(np.float32))[..., None]
    m1 = (dmin[..., None] * mn.astype(np.float32))[..., None]
    return (d1 * q.astype(np.float32) - m1).reshape(rows, cols)


def q6k_quants(raw: np.ndarray, rows: int, cols: int):
    """(q [rows, nb, 256] in -32..31 in value order, sc [rows, nb, 16], d)."""
    b = raw.reshape(rows, cols // 256, 210)
    ql = b[..., 0:128].reshape(rows, cols // 256, 2, 64)
    qh = b[..., 128:192].reshape(rows, cols // 256, 2, 32)
    sc = b[..., 192:208].view(np.int8).astype(np.int32)
    d = _f16(b[..., 208], b[..., 209])
    a, c = ql[..., :32], ql[..., 32:]
    v0 = (a & 0xF) | ((qh & 3) << 4)
    v1 = (c & 0xF) | (((qh >> 2) & 3) << 4)
    v2 = (a >> 4) | (((qh >> 4) & 3) << 4)
    v3 = (c >> 4) | (((qh >> 6) & 3) << 4)
    q = np.stack([v0, v1, v2, v3], axis=3).astype(np.int32) - 32  # [r, nb, half, 4, 32]
    return q.reshape(rows, cols // 256, 256), sc, d


def dequant_q6_k(raw, rows, cols):
    q, sc, d = q6k_quants(raw, rows, cols)
    s = (d[..., None] * sc.astype(np.float32))  # [r, nb, 16] one per 16 values
    s = np.repeat(s, 16, axis=-1)
    return (s * q.astype(np.float32)).reshape(rows, cols)


def dequant(t, raw, rows, cols):
    raw = np.ascontiguousarray(raw, np.uint8)
    if t == Q4_0:
        return dequant_q4_0(raw, rows, cols)
    if t == Q8_0:
        return dequant_q8_0(raw, rows, cols)
    if t == Q4_K:
        return dequant_q4_k(raw, rows, cols)
    if t == Q6_K:
        return dequant_q6_k(raw, rows, cols)
    if t == F32:
        return raw.view(np.float32).reshape(rows, cols).copy()
    if t == F16:
        return raw.view(np.float16).astype(np.float32).reshape(rows, cols)
    raise ValueError(t)


def random_blocks(t, rows, cols, rng: np.random.Generator) -> np.ndarray:
    """Random bytes with one exponent bit of every f16 cleared so no scale is
    NaN/Inf: the reference's fixture recipe (src/gguf/ggml.zig:2047-2048)."""
    from oracle import row_bytes

    raw = rng.integers(0, 256, rows * row_bytes(t, cols), dtype=np.uint8)
    raw[1::2] &= 0xFB
    return raw


def pinned_scale_blocks(t, rows, cols, rng: np.random.Generator, planes: int = 1) -> np.ndarray:
    """Random quants with small pinned f16 scales (the reference's GPU-test
    recipe, src/vulkan/backend.zig:1320-1348), so chained layers stay finite."""
    from oracle import row_bytes

    raw = rng.integers(0, 256, planes * rows * row_bytes(t, cols), dtype=np.uint8)
    if t == Q4_K:
        b = raw.reshape(-1, 144)
        d = rng.uniform(2.0 ** -12, 2.0 ** -10, b.shape[0]).astype(np.float16).view(np.uint16)
        m = rng.uniform(2.0 ** -13, 2.0 ** -11, b.shape[0]).astype(np.float16).view(np.uint16)
        b[:, 0], b[:, 1] = d & 0xFF, d >> 8
        b[:, 2], b[:, 3] = m & 0xFF, m >> 8
    elif t == Q6_K:
        b = raw.reshape(-1, 210)
        d = rng.uniform(2.0 ** -13, 2.0 ** -11, b.shape[0]).astype(np.float16).view(np.uint16)
        b[:, 208], b[:, 209] = d & 0xFF, d >> 8
    elif t in (Q4_0, Q8_0):
        bs = 18 if t == Q4_0 else 34
        b = raw.reshape(-1, bs)
        d = rng.uniform(2.0 ** -9, 2.0 ** -7, b.shape[0]).astype(np.float16).view(np.uint16)
        b[:, 0], b[:, 1] = d & 0xFF, d >> 8
    return raw
