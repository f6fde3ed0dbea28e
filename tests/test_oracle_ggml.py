"""Pins the CPU oracle's GGML layer (oracle/ggml_ref.c, quantize_ref.c) against
the reference's own known-answer tests, an independent numpy decoder, exact
f16 tables and float64 closed forms.  CPU only."""
import json
import math
import os

import numpy as np
import pytest

import npref

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
TYPES = [2, 8, 12, 14]  # q4_0, q8_0, q4_k, q6_k


def test_q4k_handcrafted_block(oracle):
    kat = GOLD["q4_k_handcrafted"]
    blk = np.frombuffer(bytes.fromhex(kat["block_hex"]), np.uint8).copy()
    vals = oracle.dequant_row(oracle.Q4_K, blk, 0, 256)
    for idx, want in kat["expect_vals"].items():
        assert abs(vals[int(idx)] - want) < 1e-4
    out = oracle.matvec(oracle.Q4_K, blk, np.ones(256, np.float32), 1, 256)
    assert abs(out[0] - kat["expect_dot_ones"]) < kat["dot_tol"]


def test_q6k_handcrafted_block(oracle):
    kat = GOLD["q6_k_handcrafted"]
    blk = np.frombuffer(bytes.fromhex(kat["block_hex"]), np.uint8).copy()
    vals = oracle.dequant_row(oracle.Q6_K, blk, 0, 256)
    assert np.all(np.abs(vals - kat["expect_all"]) < 1e-4)


def test_f16_widening_is_exact_for_every_pattern(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    w = want[::7]
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), w[~nan].view(np.uint32))


def test_f32_to_f16_rounds_to_nearest_even(oracle):
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.normal(0, 0.02, 2000), rng.normal(0, 100, 500), rng.uniform(-7e4, 7e4, 200),
        [0.0, -0.0, 1e-8, 6.1e-5, 5.96e-8, 2.98e-8, 65504.0, 65520.0, 1e6, -1e6],
    ]).astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t", TYPES)
def test_dequant_matches_independent_decoder_bit_exact(oracle, t):
    rng = np.random.default_rng(100 + t)
    rows, cols = 7, 512
    raw = npref.random_blocks(t, rows, cols, rng)
    got = oracle.dequant(t, raw, rows, cols)
    want = npref.dequant(t, raw, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _half_away(v):
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_quantize_x_closed_form(oracle):
    x = oracle.normal(32 * 16, 5, 0.0, 3.0)
    x[5] = 0.0
    x[32:64] = 0.0  # an all-zero block gives d = 0, q = 0
    d, s, q = oracle.quantize_x(x)
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    want_q = np.clip(_half_away(blocks * inv[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(q, want_q)
    assert np.array_equal(s, q.astype(np.int32).sum(axis=1))
    assert np.all(np.abs(blocks - d[:, None] * q) <= d[:, None] * 0.5 * (1 + 1e-5) + 1e-30)
    assert d[1] == 0 and not q[1].any()


def test_quantize_x256_closed_form(oracle):
    x = oracle.normal(256 * 4, 6, 0.0, 1.0)
    d, q, bs = oracle.quantize_x256(x)
    blocks = x.reshape(-1, 256)
    assert np.array_equal(d, (np.abs(blocks).max(axis=1) / np.float32(127)).astype(np.float32))
    inv = (np.float32(1) / d).astype(np.float32)
    assert np.array_equal(q, np.clip(_half_away(blocks * inv[:, None]), -127, 127).astype(np.int8))
    assert np.array_equal(bs, q.astype(np.int32).reshape(-1, 16, 16).sum(axis=2))
    # the element of largest magnitude maps to +-127
    i = np.abs(blocks).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(4), i]) == 127)


def test_nonfinite_activations_cannot_escape_the_quantizer(oracle):
    kat = GOLD["nonfinite_quantizer"]
    x = np.array([float(v) for v in kat["x"]], np.float32)
    d, s, q = oracle.quantize_x(x)
    assert len(d) == kat["expect_blocks"]
    assert np.all(np.isfinite(d)) and np.all(np.abs(q.astype(int)) <= 127)
    d2, _, q2 = oracle.quantize_x(np.full(32, np.nan, np.float32))
    assert d2[0] == 0 and not q2.any()
    assert oracle.to_i8_saturating(float("inf")) == 0
    assert oracle.to_i8_saturating(2.5) == 3 and oracle.to_i8_saturating(-2.5) == -3
    assert oracle.to_i8_saturating(300.0) == 127 and oracle.to_i8_saturating(-300.0) == -127


def _int8_matvec_numpy(t, raw, x, rows, cols):
    """Vectorised integer restatement: exact integer block dots, f32 tail in
    the format's order, rows summed block by block."""
    import oracle as o

    out = np.zeros(rows, np.float32)
    if t in (o.Q4_K, o.Q6_K):
        d_x, q_x, bs = o.quantize_x256(x)
        nb = cols // 256
        if t == o.Q4_K:
            q, sc, mn, d, dmin = npref.q4k_quants(raw, rows, cols)
            xq = q_x.reshape(nb, 8, 32).astype(np.int64)
            isum = (np.einsum("rbgi,bgi->rbg", q.astype(np.int64), xq) * sc).sum(axis=2)
            msum = (mn * bs.reshape(nb, 8, 2).sum(axis=2)[None]).sum(axis=2)
            a = (d * isum.astype(np.float32)).astype(np.float32)
            b = (dmin * msum.astype(np.float32)).astype(np.float32)
            r = (d_x[None] * (a - b)).astype(np.float32)
        else:
            q, sc, d = npref.q6k_quants(raw, rows, cols)
            xq = q_x.reshape(nb, 16, 16).astype(np.int64)
            isum = (np.einsum("rbsi,bsi->rbs", q.reshape(rows, nb, 16, 16).astype(np.int64), xq)
                    * sc).sum(axis=2)
            r = ((d_x[None] * d).astype(np.float32) * isum.astype(np.float32)).astype(np.float32)
    else:
        d_x, s_x, q_x = o.quantize_x(x)
        nb = cols // 32
        if t == o.Q4_0:
            b = raw.reshape(rows, nb, 18)
            d = npref._f16(b[..., 0], b[..., 1])
            qs = b[..., 2:]
            w = np.concatenate([qs & 0xF, qs >> 4], axis=-1).astype(np.int64)
            dot = np.einsum("rbi,bi->rb", w, q_x.astype(np.int64)) - 8 * s_x[None].astype(np.int64)
        else:
            b = raw.reshape(rows, nb, 34)
            d = npref._f16(b[..., 0], b[..., 1])
            dot = np.einsum("rbi,bi->rb", b[..., 2:].view(np.int8).astype(np.int64),
                            q_x.astype(np.int64))
        r = ((d * d_x[None]).astype(np.float32) * dot.astype(np.float32)).astype(np.float32)
    for j in range(r.shape[1]):
        out = (out + r[:, j]).astype(np.float32)
    return out


@pytest.mark.parametrize("t", TYPES)
def test_matvec_matches_vectorised_integer_restatement(oracle, t):
    rng = np.random.default_rng(200 + t)
    rows, cols = 9, 768
    raw = npref.random_blocks(t, rows, cols, rng)
    x = oracle.uniform(cols, 300 + t, -2.0, 2.0)
    got = oracle.matvec(t, raw, x, rows, cols)
    want = _int8_matvec_numpy(t, raw, x, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", TYPES + [0])
def test_matvec_agrees_with_f64_dequant_dot(oracle, t):
    # src/gguf/ggml.zig:2021-2087: random bytes (f16 exponent bit cleared),
    # int8 kernels within 0.01 * sum|w*x|, exact kernels 1e-4*max + 1e-3.
    rng = np.random.default_rng(0xC0FFEE + t)
    rows, cols = 3, 256
    if t == 0:
        raw = rng.uniform(-1, 1, rows * cols).astype(np.float32).view(np.uint8)
    else:
        raw = npref.random_blocks(t, rows, cols, rng)
    x = ((rng.random(cols, dtype=np.float32) - 0.5) * 4.0).astype(np.float32)
    got = oracle.matvec(t, raw, x, rows, cols)
    w = npref.dequant(t, raw, rows, cols).astype(np.float64)
    want = w @ x.astype(np.float64)
    mass = np.abs(w * x.astype(np.float64)).sum(axis=1)
    tol = mass * 0.01 if t != 0 else np.maximum(np.abs(want), np.abs(got)) * 1e-4 + 1e-3
    assert np.all(np.abs(got - want) <= tol)


def test_q4_0_and_q8_0_against_f32_reference(oracle):
    # src/gguf/ggml.zig:1906-1936
    kat = GOLD["q4_0_q8_0_vs_f32"]
    rows, cols = kat["rows"], kat["cols"]
    wf = oracle.uniform(rows * cols, 3, -0.5, 0.5).reshape(rows, cols)
    x = oracle.uniform(cols, 4, -0.5, 0.5)
    ref = oracle.matvec(oracle.F32, wf.view(np.uint8).ravel(), x, rows, cols)
    q4 = oracle.quantize(oracle.Q4_0, wf)
    q8 = oracle.quantize(oracle.Q8_0, wf)
    assert np.all(np.abs(oracle.matvec(oracle.Q4_0, q4, x, rows, cols) - ref) < kat["q4_0_abs_tol"])
    assert np.all(np.abs(oracle.matvec(oracle.Q8_0, q8, x, rows, cols) - ref) < kat["q8_0_abs_tol"])


@pytest.mark.parametrize("t", [8, 12, 14])
def test_matmul_is_bit_identical_to_repeated_matvec(oracle, t):
    # src/gguf/ggml.zig:2132-2186, plus n beyond MAX_BATCH (the fallback path)
    rng = np.random.default_rng(0x5EED + t)
    rows, cols = 133, 512
    raw = npref.random_blocks(t, rows, cols, rng)
    for n in (2, 3, 5, 8, 11):
        xs = np.stack([((rng.random(cols) - 0.5) * (k + 1)).astype(np.float32) for k in range(n)])
        want = np.stack([oracle.matvec(t, raw, xs[k], rows, cols) for k in range(n)])
        got = oracle.matmul(t, raw, xs, n, rows, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n
        with oracle.Pool(4):
            got2 = oracle.matmul(t, raw, xs, n, rows, cols)
        assert np.array_equal(got2.view(np.uint32), want.view(np.uint32)), n


@pytest.mark.parametrize("t", [0, 2, 8, 12, 14])
def test_pooled_matvec_is_bit_identical_to_serial(oracle, t):
    # src/gguf/ggml.zig:2089-2130 (repeated as a race probe)
    rng = np.random.default_rng(0xBEEF + t)
    rows, cols = 257, 256
    if t == 0:
        raw = rng.uniform(-1, 1, rows * cols).astype(np.float32).view(np.uint8)
    else:
        raw = npref.random_blocks(t, rows, cols, rng)
    x = ((rng.random(cols) - 0.5) * 4).astype(np.float32)
    serial = oracle.matvec(t, raw, x, rows, cols)
    with oracle.Pool(8):
        for _ in range(8):
            par = oracle.matvec(t, raw, x, rows, cols)
            assert np.array_equal(par.view(np.uint32), serial.view(np.uint32))


@pytest.mark.parametrize("t,bound", [(2, 0.16), (8, 0.01), (12, 0.10), (14, 0.03)])
def test_quantizer_round_trip_error(oracle, t, bound):
    """Input generators: relative RMS error of quantize -> dequant on the
    configs' N(0, 0.02) weights (parity of downstream kernels is defined on
    the emitted bytes, so this only pins that the generators are sane)."""
    rows, cols = 64, 2048
    w = oracle.normal(rows * cols, 77 + t, 0.0, 0.02).reshape(rows, cols)
    raw = oracle.quantize(t, w)
    back = oracle.dequant(t, raw, rows, cols)
    rel = math.sqrt(float(((back - w) ** 2).mean())) / 0.02
    assert rel < bound, rel
    # the same bytes decode identically through the independent decoder
    assert np.array_equal(back.view(np.uint32), npref.dequant(t, raw, rows, cols).view(np.uint32))


def test_q4k_quantizer_keeps_scales_in_range(oracle):
    w = oracle.normal(8 * 256, 9, 0.0, 0.02).reshape(8, 256)
    raw = oracle.quantize(oracle.Q4_K, w)
    q, sc, mn, d, dmin = npref.q4k_quants(raw, 8, 256)
    assert sc.max() <= 63 and mn.max() <= 63 and q.max() <= 15 and q.min() >= 0
    assert np.all(d > 0) and np.all(dmin >= 0)
    # the largest group scale is stored as 63 (d = max_scale/63)
    assert np.all(sc.max(axis=-1) >= 62)


def test_dot_f32_matches_float64_and_order(oracle):
    rng = np.random.default_rng(11)
    for n in (0, 1, 7, 8, 31, 32, 33, 100, 2048):
        a = rng.normal(size=n).astype(np.float32)
        b = rng.normal(size=n).astype(np.float32)
        got = oracle.dot_f32(a, b)
        want = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(got - want) <= 1e-5 * (np.abs(a * b).sum() + 1e-30) + 1e-7
    # exact on small integers regardless of order
    a = np.arange(64, dtype=np.float32)
    assert oracle.dot_f32(a, np.ones(64, np.float32)) == 2016.0
