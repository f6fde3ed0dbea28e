// frame.hpp -- shapes and device helpers shared by the decode frame's kernels
// (frame.hip) and the reference-order attention (attn_exact.hip).
#pragma once

#include "device.hpp"

namespace lh {

constexpr int ATT_TC = 64;  // positions per attention work group (one per lane of a wave)
constexpr int MAX_HD = 256; // head_dim limit
constexpr int MAX_G = 16;   // query heads per KV head limit

struct FrameDims {
    int dim, hd, n_heads, n_kv, qd, kvd, ctx, rope_dim, rope_neox, n_layers, vocab;
    float rope_base, eps, scale;
};

// ---- reductions ----------------------------------------------------------------

__device__ inline float wave_sum_f(float v) {
    v = v + dpp_f<0xB1>(v, v);
    v = v + dpp_f<0x4E>(v, v);
    v = v + dpp_f<0x141>(v, v);
    v = v + dpp_f<0x140>(v, v);
    v = v + dpp_f<0x142, 0xA>(v, v);
    v = v + dpp_f<0x143, 0xC>(v, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the work group's waves (each value is already wave-uniform),
// added in wave order.
__device__ inline float block_sum_waves(float wave_total, float *lds) {
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        lds[wave] = wave_total;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < nw; w++)
        s = s + lds[w];
    return s;
}

// ---- attention over 64 positions for one KV head group (llama.zig:1162-1192) -------

// dotF32 (src/gguf/ggml.zig:198-217) of a query head (f32, LDS, read as
// broadcasts) and a cached key row (fp16, a padded LDS row), 8 values per
// 16-byte read: 32 accumulators over whole 32-steps, leftover 8-chunks into
// the first 8, ((a0 + a1) + a2) + a3 per lane, the lanes summed in order
// from -0 (HD is a multiple of 8).
template <int HD>
__device__ __forceinline__ float dot_f32_key(const float *a, const uint16_t *krow) {
    float acc[32];
#pragma unroll
    for (int u = 0; u < 32; u++)
        acc[u] = 0.0f;
#pragma unroll
    for (int i = 0; i < HD; i += 8) {
        const uint4 kv = *(const uint4 *)(krow + i);
        const float4 qa = *(const float4 *)(a + i), qb = *(const float4 *)(a + i + 4);
        const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
        const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const int base = i < HD / 32 * 32 ? i % 32 : 0; // whole 32-steps, then chunks into acc[0..8)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float k = half_bits_to_float((uint16_t)(kw[e >> 1] >> (16 * (e & 1))));
            const float pr = qv[e] * k;
            acc[base + e] = acc[base + e] + pr;
        }
    }
    float s = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++)
        s = s + (((acc[l] + acc[8 + l]) + acc[16 + l]) + acc[24 + l]);
    return s;
}


// ---- the sequential sum of non-negative values, by speculative composition ----
// The reference sums softmax's exponentials and rmsnorm's squares in index
// order (tensor.zig:12,22-25): a chain of n dependent f32 adds.  Here the n
// values (LDS, zero-padded to whole 64-value chunks) are cut into chunks of
// 64; a double prefix sum estimates the running sum at each chunk's start;
// each lane of a wave runs the chunk's chain from one of the 64 f32 values
// around that estimate (consecutive bit patterns; chunk 0 from +0, the
// reference's start); one wave then follows the exact running sum through
// the chunks, taking each chunk's end from the lane whose start equals the
// running sum, or re-running the chunk from the exact value when the window
// missed it.  Every value produced is one the reference's loop produces, so
// the result is the sequential sum itself.  All NW waves of the work group
// call it; C = n/64 <= 128; ends holds 64 floats per chunk, csum C doubles,
// fst C words, out one float (all LDS).  Adding +0 to a sum of non-negative
// values leaves it unchanged, which makes the zero padding exact.
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int m = 32; m >= 1; m >>= 1)
        v = v + __shfl_xor(v, m);
    return v;
}

template <int NW>
__device__ float seq_sum_nonneg(const float *v, int C, float *ends, double *csum, uint32_t *fst, float *out) {
    const int wave = threadIdx.x >> 6, ln = threadIdx.x & 63;
    for (int c = wave; c < C; c += NW) {
        const double s = wave_sum_d((double)v[64 * c + ln]);
        if (ln == 0)
            csum[c] = s;
    }
    __syncthreads();
    if (wave == 0) { // exclusive prefix of the chunk sums: the estimates (their order is free)
        const double ca = ln < C ? csum[ln] : 0.0, cb = 64 + ln < C ? csum[64 + ln] : 0.0;
        double a = ca, b = cb;
        for (int o = 1; o < 64; o <<= 1) {
            const double ta = __shfl_up(a, o), tb = __shfl_up(b, o);
            if (ln >= o) {
                a = a + ta;
                b = b + tb;
            }
        }
        b = b + __shfl(a, 63);
        if (ln < C)
            fst[ln] = __float_as_uint((float)(a - ca));
        if (64 + ln < C)
            fst[64 + ln] = __float_as_uint((float)(b - cb));
    }
    __syncthreads();
    for (int c = wave; c < C; c += NW) {
        const int b = c == 0 ? 0 : max((int)fst[c] + ln - 32, 0);
        float4 ev[16];
#pragma unroll
        for (int k = 0; k < 16; k++)
            ev[k] = *(const float4 *)(v + 64 * c + 4 * k);
        float s = __uint_as_float((uint32_t)b);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            s = s + ev[k].x;
            s = s + ev[k].y;
            s = s + ev[k].z;
            s = s + ev[k].w;
        }
        ends[c * 64 + ln] = s;
    }
    __syncthreads();
    if (wave == 0) {
        const uint32_t fa = ln < C ? fst[ln] : 0u, fb = 64 + ln < C ? fst[64 + ln] : 0u;
        float run = ends[0];
        float cur = C > 1 ? ends[64 + ln] : 0.0f;
        for (int c = 1; c < C; c++) {
            const float nxt = c + 1 < C ? ends[(c + 1) * 64 + ln] : 0.0f;
            const int f = (int)(c < 64 ? __builtin_amdgcn_readlane(fa, c) : __builtin_amdgcn_readlane(fb, c - 64));
            const int idx = __builtin_amdgcn_readfirstlane((int)__float_as_uint(run) - f + 32);
            if (idx >= 0 && idx < 64) {
                run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur), idx));
            } else { // outside the window: this chunk's chain from the exact value
                for (int j = 64 * c; j < 64 * c + 64; j++)
                    run = run + v[j];
            }
            cur = nxt;
        }
        if (ln == 0)
            *out = run;
    }
    __syncthreads();
    return *out;
}

// ---- the reference-order attention (attn_exact.hip), PARITY numerics --------
// Scores, softmax and P.V of llama.zig:1162-1192 in the reference's own
// evaluation order over any context: one launch of scores per 64 positions,
// one softmax launch per (head, lane), one P.V launch per (64 columns, KV
// head, lane).  S is [n][n_heads][s_stride] f32 (scores, then p in place),
// att the f32 attention output [n][n_heads * head_dim].
constexpr int EXACT_MAX_CTX = 7936; // the softmax's LDS: e[ctx] + 64 chain ends per 64 positions
size_t exact_softmax_lds(int s_stride);
bool launch_attn_exact(const FrameDims &D, const float *q, const float *k, const float *v, const float *q_norm,
                       const float *k_norm, const float *rope_cs, uint16_t *kc, uint16_t *vc, const int32_t *pos,
                       int li, bool fuse, float *S, int s_stride, float *att, size_t n, hipStream_t st);

} // namespace lh
