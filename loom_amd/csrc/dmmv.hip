// dmmv.hip -- grouped dequant-fused matvec for Q4_0 / Q8_0 / Q4_K / Q6_K with
// int8 activations, bit-identical to the reference CPU kernels
// (src/gguf/ggml.zig:1002-1038 kBlockDot/matvecK256, 1196-1222 matvecQ40Int,
// 1277-1294 matvecQ80Int).
//
// Work map (wave64).  A block (32 or 256 weights) is served by LPB lanes:
// 8 for the K-quants (each lane owns 16 bytes of quants = 32 weights), 2 for
// Q8_0, 1 for Q4_0, so a wave covers BPI = 64/LPB blocks per step.  A wave
// walks its rows with the lane->block map fixed, so each lane's int8
// activation chunk is loaded once and reused for every row (and every token
// of its group).  Each lane computes exact integer partial dots with
// v_dot4_i32_i8, the LPB lanes of a block reduce them with DPP, and the block
// leader applies the reference's f32 tail.  Per-block results go to LDS and
// each output row is summed over its blocks sequentially in block order --
// the reference's `acc += r` -- so the result is bit-identical to the CPU.
#include "kernels.hpp"

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
    const float e = expf(-g);
    const float s = g / (1.0f + e);
    return s * u;
}

constexpr int WAVES = 4;

template <int T, int NT, bool FUSED>
__global__ __launch_bounds__(256) void dmmv_kernel(DmmvParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB, BPI = 64 / LPB;
    extern __shared__ float lds[];

    const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
    if ((int)blockIdx.y >= ng)
        return;
    const DmmvGroup g = p.groups[blockIdx.y];
    const int n = g.n;
    const int rows = p.rows, cols = p.cols, nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int TR = WAVES * p.rpw;
    const int row0 = blockIdx.x * TR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / LPB, j = lane % LPB;
    const bool wide = nb >= BPI;
    const int C = wide ? nb / BPI : 1;
    const int RPI = wide ? 1 : BPI / nb;
    const int ro = wide ? 0 : grp / nb;
    const bool active = wide || grp < RPI * nb;
    const int nit = (p.rpw + RPI - 1) / RPI;
    const uint8_t *wb = p.w + (size_t)g.plane * p.plane_bytes;
    const uint8_t *wb2 = FUSED ? p.w2 + (size_t)g.plane * p.plane_bytes : nullptr;
    const size_t lds_mat = (size_t)NT * TR * nb; // floats per matrix

    for (int c = 0; c < C; c++) {
        const int b = wide ? c * BPI + grp : (grp % nb);
        typename F::X xr[NT];
#pragma unroll
        for (int k = 0; k < NT; k++) {
            const int v = p.pair_src[g.first + (k < n ? k : 0)];
            xr[k] = F::load_x(p.xq, p.xd, p.xs, cols, v, b, j);
        }
#pragma unroll 2
        for (int it = 0; it < nit; it++) {
            const int rw = it * RPI + ro;           // row within this wave's span
            const int rl = wave * p.rpw + rw;        // row within the tile
            const int row = row0 + rl;
            const bool valid = active && rw < p.rpw && row < rows;
            const size_t unit = (size_t)(valid ? row : 0) * nb + b;
            const typename F::W w = F::load_w(wb, U, unit, j);
            typename F::W w2;
            if constexpr (FUSED)
                w2 = F::load_w(wb2, U, unit, j);
#pragma unroll
            for (int k = 0; k < NT; k++) {
                if (k < n) {
                    int is, ms;
                    F::dot(w, xr[k], j, is, ms);
                    is = group_sum<LPB>(is);
                    ms = group_sum<LPB>(ms);
                    if (valid && j == 0)
                        lds[((size_t)k * TR + rl) * nb + b] = F::tail(w, xr[k], is, ms);
                    if constexpr (FUSED) {
                        F::dot(w2, xr[k], j, is, ms);
                        is = group_sum<LPB>(is);
                        ms = group_sum<LPB>(ms);
                        if (valid && j == 0)
                            lds[lds_mat + ((size_t)k * TR + rl) * nb + b] = F::tail(w2, xr[k], is, ms);
                    }
                }
            }
        }
    }
    __syncthreads();
    // Row sums in block order (the reference's sequential `acc += r`).
    for (int idx = threadIdx.x; idx < n * TR; idx += blockDim.x) {
        const int k = idx / TR, rl = idx % TR, row = row0 + rl;
        if (row >= rows)
            continue;
        const float *r = lds + ((size_t)k * TR + rl) * nb;
        float acc = 0.0f;
        for (int bb = 0; bb < nb; bb++)
            acc = acc + r[bb];
        float val = acc;
        if constexpr (FUSED) {
            const float *r2 = lds + lds_mat + ((size_t)k * TR + rl) * nb;
            float acc2 = 0.0f;
            for (int bb = 0; bb < nb; bb++)
                acc2 = acc2 + r2[bb];
            val = swiglu1(acc, acc2);
        }
        p.out[(size_t)p.pair_dst[g.first + k] * p.out_stride + row] = val;
    }
}

bool dmmv_supported(int t, int cols) {
    switch (t) {
    case LH_Q4_K:
    case LH_Q6_K: {
        if (cols % 256)
            return false;
        const int nb = cols / 256;
        return nb <= 8 || nb % 8 == 0;
    }
    case LH_Q8_0: {
        if (cols % 32)
            return false;
        const int nb = cols / 32;
        return nb <= 32 || nb % 32 == 0;
    }
    case LH_Q4_0: {
        if (cols % 32)
            return false;
        const int nb = cols / 32;
        return nb <= 64 || nb % 64 == 0;
    }
    default:
        return false;
    }
}

static int lpb_of(int t) { return (t == LH_Q4_K || t == LH_Q6_K) ? 8 : t == LH_Q8_0 ? 2 : 1; }

int dmmv_pick_rpw(int t, int cols, int rows, int groups, int nt, bool fused) {
    // Aim for >= ~2048 work groups across the chip (256 CUs x 8 waves), keep
    // at least one full wave step of rows, and stay inside the LDS budget of
    // the per-block partials ((fused ? 2 : 1) * nt * 4 * rpw * nb floats).
    const int nb = cols / block_elems(t);
    const int bpi = 64 / lpb_of(t);
    const int rpi = nb >= bpi ? 1 : bpi / nb;
    int rpw = 16;
    while (rpw > 2 && (long)((rows + WAVES * rpw - 1) / (WAVES * rpw)) * groups < 2048)
        rpw /= 2;
    if (rpw < rpi)
        rpw = rpi;
    const long per_row = (long)(fused ? 2 : 1) * nt * WAVES * nb * (long)sizeof(float);
    while (rpw > 1 && rpw > rpi && per_row * rpw > DMMV_LDS_BUDGET)
        rpw--;
    return rpw;
}

size_t dmmv_lds_bytes(int t, int cols, int nt, bool fused, int rpw) {
    return (size_t)(fused ? 2 : 1) * nt * WAVES * rpw * (cols / block_elems(t)) * sizeof(float);
}

template <int T, int NT, bool FUSED>
static void launch_t(const DmmvParams &p, hipStream_t st) {
    const int TR = WAVES * p.rpw;
    const size_t lds = dmmv_lds_bytes(T, p.cols, NT, FUSED, p.rpw);
    dim3 grid((p.rows + TR - 1) / TR, p.n_groups);
    hipLaunchKernelGGL((dmmv_kernel<T, NT, FUSED>), grid, dim3(256), lds, st, p);
}

template <int T, bool FUSED>
static void launch_nt(int nt, const DmmvParams &p, hipStream_t st) {
    switch (nt) {
    case 1:
        launch_t<T, 1, FUSED>(p, st);
        break;
    case 2:
        launch_t<T, 2, FUSED>(p, st);
        break;
    case 4:
        launch_t<T, 4, FUSED>(p, st);
        break;
    default:
        launch_t<T, 8, FUSED>(p, st);
        break;
    }
}

template <int T>
static void launch_f(int nt, bool fused, const DmmvParams &p, hipStream_t st) {
    if (fused)
        launch_nt<T, true>(nt, p, st);
    else
        launch_nt<T, false>(nt, p, st);
}

bool launch_dmmv(int t, int nt, bool fused, const DmmvParams &p, hipStream_t st) {
    if (dmmv_lds_bytes(t, p.cols, nt, fused, p.rpw) > 64 * 1024)
        return false;
    switch (t) {
    case LH_Q4_K:
        launch_f<LH_Q4_K>(nt, fused, p, st);
        break;
    case LH_Q6_K:
        launch_f<LH_Q6_K>(nt, fused, p, st);
        break;
    case LH_Q8_0:
        launch_f<LH_Q8_0>(nt, fused, p, st);
        break;
    case LH_Q4_0:
        launch_f<LH_Q4_0>(nt, fused, p, st);
        break;
    default:
        return false;
    }
    note_launch();
    return true;
}

} // namespace lh
