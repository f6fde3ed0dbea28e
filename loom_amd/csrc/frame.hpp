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
