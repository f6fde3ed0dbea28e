// fmt.hpp -- per-format traits of the int8-activation dequant-fused matvec
// (bit-identical to the reference CPU kernels, src/gguf/ggml.zig:1002-1038
// kBlockDot/matvecK256, 1196-1222 matvecQ40Int, 1277-1294 matvecQ80Int).
//
// A block (32 or 256 weights) is served by LPB lanes: 8 for the K-quants
// (each lane owns 16 bytes of quants = 32 weights), 2 for Q8_0, 1 for Q4_0.
// load_w / load_x fetch a lane's share of a weight block and of the matching
// int8 activation block, dot() gives the lane's exact integer partials, and
// tail() applies the reference's f32 expression once the LPB lanes' integer
// partials are summed.
#pragma once

#include "device.hpp"

namespace lh {

template <int T> struct Fmt;

// ---- Q4_K: lane j owns qs bytes [16j, 16j+16): group pair p=j>>1, half h=j&1.
// Low nibbles are group 2p values 16h..16h+15, high nibbles group 2p+1.
template <> struct Fmt<LH_Q4_K> {
    static constexpr int LPB = 8, BE = 256;
    struct W {
        uint4 hdr;
        int4 qs;
    };
    struct X {
        int4 xa, xb;
        int bs0, bs1;
        float xd;
    };
    __device__ static W load_w(const uint8_t *base, size_t U, size_t unit, int j) {
        W w;
        const uint8_t *blk = base + unit * 144;
        w.hdr = *(const uint4 *)blk;
        w.qs = *(const int4 *)(blk + 16 + 16 * j);
        return w;
    }
    __device__ static X load_x(const int8_t *q, const float *d, const int32_t *s, int cols, int v,
                               int b, int j) {
        const int p = j >> 1, h = j & 1, o0 = b * 256 + 64 * p + 16 * h;
        X x;
        const int8_t *qv = q + (size_t)v * cols;
        x.xa = *(const int4 *)(qv + o0);
        x.xb = *(const int4 *)(qv + o0 + 32);
        const int32_t *sv = s + (size_t)v * (cols / 16) + b * 16;
        x.bs0 = sv[4 * p + h];
        x.bs1 = sv[4 * p + 2 + h];
        x.xd = d[(size_t)v * (cols / 256) + b];
        return x;
    }
    // scaleMinK4 (src/gguf/ggml.zig:1332-1340) for groups 2p and 2p+1.
    __device__ static void scales(const uint4 &hdr, int j, int &sc0, int &mn0, int &sc1, int &mn1) {
        const int p = j >> 1;
        const uint32_t a = hdr.y, b = hdr.z, c = hdr.w;
        if (p < 2) {
            const int s0 = 16 * p, s1 = 16 * p + 8; // byte shifts of groups 2p, 2p+1
            sc0 = (a >> s0) & 63;
            mn0 = (b >> s0) & 63;
            sc1 = (a >> s1) & 63;
            mn1 = (b >> s1) & 63;
        } else {
            const int s0 = 16 * (p - 2), s1 = s0 + 8;
            sc0 = ((c >> s0) & 0xF) | (((a >> s0) >> 6 & 3) << 4);
            mn0 = ((c >> s0) >> 4 & 0xF) | (((b >> s0) >> 6 & 3) << 4);
            sc1 = ((c >> s1) & 0xF) | (((a >> s1) >> 6 & 3) << 4);
            mn1 = ((c >> s1) >> 4 & 0xF) | (((b >> s1) >> 6 & 3) << 4);
        }
    }
    __device__ static void dot(const W &w, const X &x, int j, int &isum, int &msum) {
        int sc0, mn0, sc1, mn1;
        scales(w.hdr, j, sc0, mn0, sc1, mn1);
        const int dlo = dot16(and4(w.qs, 0x0F0F0F0F), x.xa, 0);
        const int dhi = dot16(and4(shr4(w.qs, 4), 0x0F0F0F0F), x.xb, 0);
        isum = sc0 * dlo + sc1 * dhi;
        msum = mn0 * x.bs0 + mn1 * x.bs1;
    }
    // xb.d * (d * f32(isum) - dmin * f32(min_isum))  (ggml.zig:1016-1017)
    __device__ static float tail(const W &w, const X &x, int isum, int msum) {
        const float d = half_bits_to_float(w.hdr.x & 0xffff);
        const float dmin = half_bits_to_float(w.hdr.x >> 16);
        const float a = d * (float)isum;
        const float b = dmin * (float)msum;
        return x.xd * (a - b);
    }
};

// ---- Q6_K (device SoA): lane j: half h=j>>2, quarter q=j&3 of that half's
// ql; its two 16-value runs start at base = 128h + 32(q>>1) + 16(q&1) and
// base + 64, with high bits at shift 2(q>>1) and 4 + 2(q>>1).
template <> struct Fmt<LH_Q6_K> {
    static constexpr int LPB = 8, BE = 256;
    struct W {
        int4 ql, qh;
        uint4 sc;
        uint32_t d;
    };
    struct X {
        int4 xa, xb;
        int bs0, bs1;
        float xd;
    };
    __device__ static W load_w(const uint8_t *base, size_t U, size_t unit, int j) {
        const int h = j >> 2, q = j & 3;
        W w;
        w.ql = *(const int4 *)(base + unit * 128 + 64 * h + 16 * q);
        w.qh = *(const int4 *)(base + U * 128 + unit * 64 + 32 * h + 16 * (q & 1));
        w.sc = *(const uint4 *)(base + U * 192 + unit * 16);
        w.d = *(const uint16_t *)(base + U * 208 + unit * 2);
        return w;
    }
    __device__ static int run_base(int j) {
        const int h = j >> 2, q = j & 3;
        return 128 * h + 32 * (q >> 1) + 16 * (q & 1);
    }
    __device__ static X load_x(const int8_t *q, const float *d, const int32_t *s, int cols, int v,
                               int b, int j) {
        const int base = run_base(j);
        X x;
        const int8_t *qv = q + (size_t)v * cols + b * 256;
        x.xa = *(const int4 *)(qv + base);
        x.xb = *(const int4 *)(qv + base + 64);
        const int32_t *sv = s + (size_t)v * (cols / 16) + b * 16;
        x.bs0 = sv[base / 16];
        x.bs1 = sv[base / 16 + 4];
        x.xd = d[(size_t)v * (cols / 256) + b];
        return x;
    }
    __device__ static void dot(const W &w, const X &x, int j, int &isum, int &msum) {
        const int q = j & 3, sh0 = 2 * (q >> 1), sh1 = 4 + sh0;
        const int s0 = run_base(j) / 16;
        const int4 w0 = make_int4(
            (w.ql.x & 0x0F0F0F0F) | ((((unsigned)w.qh.x >> sh0) & 0x03030303) << 4),
            (w.ql.y & 0x0F0F0F0F) | ((((unsigned)w.qh.y >> sh0) & 0x03030303) << 4),
            (w.ql.z & 0x0F0F0F0F) | ((((unsigned)w.qh.z >> sh0) & 0x03030303) << 4),
            (w.ql.w & 0x0F0F0F0F) | ((((unsigned)w.qh.w >> sh0) & 0x03030303) << 4));
        const int4 w1 = make_int4(
            (((unsigned)w.ql.x >> 4) & 0x0F0F0F0F) | ((((unsigned)w.qh.x >> sh1) & 0x03030303) << 4),
            (((unsigned)w.ql.y >> 4) & 0x0F0F0F0F) | ((((unsigned)w.qh.y >> sh1) & 0x03030303) << 4),
            (((unsigned)w.ql.z >> 4) & 0x0F0F0F0F) | ((((unsigned)w.qh.z >> sh1) & 0x03030303) << 4),
            (((unsigned)w.ql.w >> 4) & 0x0F0F0F0F) | ((((unsigned)w.qh.w >> sh1) & 0x03030303) << 4));
        // weights are q-32; dot(q-32, x) = dot(q, x) - 32*sum(x)
        const int d0 = dot16(w0, x.xa, 0) - 32 * x.bs0;
        const int d1 = dot16(w1, x.xb, 0) - 32 * x.bs1;
        const int sc0 = (int)(int8_t)byte_of(w.sc, s0);
        const int sc1 = (int)(int8_t)byte_of(w.sc, s0 + 4);
        isum = sc0 * d0 + sc1 * d1;
        msum = 0;
    }
    // xb.d * dec.d * f32(isum)  (ggml.zig:1019)
    __device__ static float tail(const W &w, const X &x, int isum, int msum) {
        const float s = x.xd * half_bits_to_float(w.d);
        return s * (float)isum;
    }
};

// ---- Q8_0 (device SoA): two lanes per 32-value block, 16 values each.
template <> struct Fmt<LH_Q8_0> {
    static constexpr int LPB = 2, BE = 32;
    struct W {
        int4 qs;
        uint32_t d;
    };
    struct X {
        int4 xa;
        float xd;
    };
    __device__ static W load_w(const uint8_t *base, size_t U, size_t unit, int j) {
        W w;
        w.qs = *(const int4 *)(base + unit * 32 + 16 * j);
        w.d = *(const uint16_t *)(base + U * 32 + unit * 2);
        return w;
    }
    __device__ static X load_x(const int8_t *q, const float *d, const int32_t *s, int cols, int v,
                               int b, int j) {
        X x;
        x.xa = *(const int4 *)(q + (size_t)v * cols + b * 32 + 16 * j);
        x.xd = d[(size_t)v * (cols / 32) + b];
        return x;
    }
    __device__ static void dot(const W &w, const X &x, int j, int &isum, int &msum) {
        isum = dot16(w.qs, x.xa, 0);
        msum = 0;
    }
    // d * xd * f32(dot)  (ggml.zig:1290)
    __device__ static float tail(const W &w, const X &x, int isum, int msum) {
        const float s = half_bits_to_float(w.d) * x.xd;
        return s * (float)isum;
    }
};

// ---- Q4_0 (device SoA): one lane per block; byte i low nibble = value i,
// high nibble = value i+16.
template <> struct Fmt<LH_Q4_0> {
    static constexpr int LPB = 1, BE = 32;
    struct W {
        int4 qs;
        uint32_t d;
    };
    struct X {
        int4 xa, xb;
        int xs;
        float xd;
    };
    __device__ static W load_w(const uint8_t *base, size_t U, size_t unit, int j) {
        W w;
        w.qs = *(const int4 *)(base + unit * 16);
        w.d = *(const uint16_t *)(base + U * 16 + unit * 2);
        return w;
    }
    __device__ static X load_x(const int8_t *q, const float *d, const int32_t *s, int cols, int v,
                               int b, int j) {
        X x;
        const int8_t *qv = q + (size_t)v * cols + b * 32;
        x.xa = *(const int4 *)qv;
        x.xb = *(const int4 *)(qv + 16);
        x.xs = s[(size_t)v * (cols / 32) + b];
        x.xd = d[(size_t)v * (cols / 32) + b];
        return x;
    }
    __device__ static void dot(const W &w, const X &x, int j, int &isum, int &msum) {
        int acc = dot16(and4(w.qs, 0x0F0F0F0F), x.xa, 0);
        acc = dot16(and4(shr4(w.qs, 4), 0x0F0F0F0F), x.xb, acc);
        isum = acc - 8 * x.xs;
        msum = 0;
    }
    // d * xd * f32(dot - 8*sum)  (ggml.zig:1218)
    __device__ static float tail(const W &w, const X &x, int isum, int msum) {
        const float s = half_bits_to_float(w.d) * x.xd;
        return s * (float)isum;
    }
};

// silu(g) * u with silu(x) = x / (1 + exp(-x))  (src/core/tensor.zig:30-57)
__device__ inline float swiglu1(float g, float u) {
    const float e = exp_f32_poly(-g);
    const float s = g / (1.0f + e);
    return s * u;
}

constexpr int WAVES = 4; // waves per work group of the matvec kernels

// Row r's value: its blocks summed in block order (the reference's
// sequential `acc += r`), SwiGLU(gate, up) when FUSED.
template <bool FUSED>
__device__ inline float row_value(const float *lds, size_t lds_mat, size_t idx, int nb) {
    const float *r = lds + idx * nb;
    float acc = 0.0f;
    for (int bb = 0; bb < nb; bb++)
        acc = acc + r[bb];
    if constexpr (FUSED) {
        const float *r2 = lds + lds_mat + idx * nb;
        float acc2 = 0.0f;
        for (int bb = 0; bb < nb; bb++)
            acc2 = acc2 + r2[bb];
        return swiglu1(acc, acc2);
    }
    return acc;
}


} // namespace lh
