// frame.hip -- the whole-token decode frame: embedding, every GQA layer
// (attention + dense FFN or routed MoE), the output head and the greedy pick,
// stream-ordered on the device with no host round trip
// (src/gguf/llama.zig step 1111-1227 at one lane, decodeBatch 1939-2043 at
// n lanes; the one-submission shape of the reference's frames,
// src/compute/backend.zig:141-191).
//
// Per layer:
//   norm_quant     rmsnorm(x) * attn_norm, int8-quantized for wq/wk/wv
//   dmmv_seg       q, k and v in one launch (bit-identical to the CPU kernels)
//   qk_rope        (more than 4 lanes) per-head Q/K RMSNorm, RoPE, K/V append
//   attn_partial   per 64 positions x one KV head group: (up to 4 lanes) the
//                  group's query heads' RMSNorm and RoPE, the new K/V row's
//                  (appended, fp16, by the chunk that holds it), then scores, softmax pieces
//                  and P.V (split over the context, flash-decoding style;
//                  within 64 positions the reference's own order)
//   attn_combine   partials merged per head, int8-quantized for wo
//   dmmv (+=)      x += wo . attn
//   norm_quant     rmsnorm(x) * ffn_norm (f32 for the router, or int8; FAST
//                  numerics at few lanes: folded into the router launch)
//   MoE layer      (moe_host.hip) with the residual add, or the dense SwiGLU
//                  FFN with x += down . act
// then norm_quant + the output matvec + argmax (sampler.zig:7-15), pos += 1.
//
// Numerics: every matvec is bit-identical to the reference's int8 kernels
// on identical inputs, and so are the attention scores (dotF32 order), the
// per-head Q/K RMSNorm and, up to 64 positions, the softmax and P.V in the
// reference's order.  RoPE's cos/sin come from a host table in ropeTheta's
// own expressions, and exp is the once-rounded double exponential.
// rmsnorm's sum of squares is the reference's sequential sum in PARITY mode
// (and always for the embedding row) and a fixed tree in FAST mode; past 64
// positions softmax's sum and P.V are a split-context merge.  Last-bit
// differences from these can move one int8 step of a quantized matvec
// input (the 2e-3 layer/logit tolerance).
#include "frame_host.hpp"

#include <cmath>
#include <string>
#include <vector>

namespace lh {

// ---- embedding: x[lane] = dequantRow(embed, token) (llama.zig:1122) -------------

__global__ void embed_kernel(int t, const uint8_t *__restrict__ w, int vocab, int dim,
                             const uint32_t *__restrict__ tokens, float *__restrict__ x) {
    const int lane = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= dim)
        return;
    const uint32_t tok = tokens[lane];
    const size_t r = tok < (uint32_t)vocab ? tok : (uint32_t)(vocab - 1); // never past the table
    x[(size_t)lane * dim + c] = dequant_value(t, w, vocab, dim, r, c);
}

// ---- rmsnorm (tensor.zig:9-15) + int8 quantization for weight type QB --------------
constexpr int EXACT_NORM_MAX_DIM = 7936; // the squares and the sequential sum's LDS fit 64 KB
// One work group per lane; thread c < dim / 32 owns the 32-value chunk c
// (dim <= 8192).  out_i = (x_i * scale) * w_i with scale = 1 / sqrt(ss/n +
// eps).  EXACT: ss is the reference's sequential sum of the squares in index
// order (seq_sum_nonneg, over 16 waves: the chunk chains are what takes the
// time, so the group has 1024 threads); otherwise per chunk in order, then
// across chunks as a fixed tree (256 threads).  qa (QB = 32 or 256) and
// normed are each optional.
constexpr int norm_threads(bool exact) { return exact ? 1024 : 256; }

// The rmsnorm of one row (xrow: global or LDS, dim values) by the calling
// work group, as laid out above; the kernel below and combine_norm_kernel.
// The norm weights of thread c's chunk (zero for the sum's helper threads).
__device__ __forceinline__ void norm_weights(const float *__restrict__ w, int dim, float4 (&gw)[8]) {
    const int c = threadIdx.x, chunks = dim / 32, cc = c < chunks ? c : chunks - 1;
#pragma unroll
    for (int i = 0; i < 8; i++)
        gw[i] = c < 256 ? *(const float4 *)(w + (size_t)cc * 32 + 4 * i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// PRE: gw holds norm_weights(w) already (requested earlier by the caller).
template <int QB, bool EXACT, bool PRE = false>
__device__ __forceinline__ void norm_quant_row(const float *xrow, int dim, const float *__restrict__ w, float eps,
                                               QAct qa, float *__restrict__ normed, int lane_v, float *red, float *sq,
                                               SeqSumLds &seq, float4 (&gw)[8]) {
    const int c = threadIdx.x, chunks = dim / 32;
    const bool live = c < chunks;
    const int cc = live ? c : chunks - 1;
    const float *xv = xrow + (size_t)cc * 32;
    float4 v[8]; // the norm weights are requested with x, not after the reduction
    if (c < 256) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = *(const float4 *)(xv + 4 * i);
        if constexpr (!PRE) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                gw[i] = *(const float4 *)(w + (size_t)cc * 32 + 4 * i);
        }
    } else { // the sum's helper threads (EXACT) own no chunk
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = gw[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        ss = ss + v[i].x * v[i].x;
        ss = ss + v[i].y * v[i].y;
        ss = ss + v[i].z * v[i].z;
        ss = ss + v[i].w * v[i].w;
    }
    ss = live ? ss : 0.0f;
    float total;
    if constexpr (EXACT) {
        // the squares in order, zero-padded to whole 64-value chunks, summed
        // sequentially (speculative composition: the reference's own sum)
        const int C = (dim + 63) / 64;
        if (c < 2 * C) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float4 p = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (live) {
                    p.x = v[i].x * v[i].x;
                    p.y = v[i].y * v[i].y;
                    p.z = v[i].z * v[i].z;
                    p.w = v[i].w * v[i].w;
                }
                *(float4 *)(sq + c * 32 + 4 * i) = p;
            }
        }
        __syncthreads();
        total = seq_sum_nonneg<norm_threads(EXACT) / 64>(sq, dim, seq);
    } else {
        total = block_sum_waves(wave_sum_f(ss), red);
    }
    const float scale = 1.0f / sqrtf(total / (float)dim + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 g = gw[i];
        v[i].x = (v[i].x * scale) * g.x;
        v[i].y = (v[i].y * scale) * g.y;
        v[i].z = (v[i].z * scale) * g.z;
        v[i].w = (v[i].w * scale) * g.w;
    }
    if (normed && live) {
        float *o = normed + (size_t)lane_v * dim + (size_t)c * 32;
#pragma unroll
        for (int i = 0; i < 8; i++)
            *(float4 *)(o + 4 * i) = v[i];
    }
    if constexpr (QB == 32 || QB == 256) {
        if (qa.q) {
            const int ns = QB == 256 ? dim / 16 : dim / 32;
            quant_chunk32<QB>(v, live, c, qa.q + (size_t)lane_v * dim, qa.d + (size_t)lane_v * (dim / QB),
                              qa.s + (size_t)lane_v * ns);
        }
    }
}

template <int QB, bool EXACT>
__global__ __launch_bounds__(norm_threads(EXACT)) void norm_quant_kernel(const float *__restrict__ x, int dim,
                                                                        const float *__restrict__ w, float eps,
                                                                        QAct qa, float *__restrict__ normed) {
    __shared__ float red[4];
    __shared__ __align__(16) float sq[EXACT ? EXACT_NORM_MAX_DIM : 1];
    __shared__ SeqSumLds seq;
    const int lane_v = blockIdx.x;
    float4 gw[8];
    norm_quant_row<QB, EXACT>(x + (size_t)lane_v * dim, dim, w, eps, qa, normed, lane_v, red, sq, seq, gw);
}

// ---- the batched MoE combine with the next rmsnorm ----------------------------------
// One work group per token: the token's gated expert rows added to its
// residual in ascending expert id, each distinct expert once (the combine
// of moeBatchUnion, combine_kernel's mode 1, in that kernel's order), the
// row stored and kept in LDS, then the rmsnorm of the next consumer of x
// (the next layer's attention, or the output head) formed from LDS exactly
// as norm_quant_kernel forms it from memory -- the same bits, one launch and
// one HBM round trip fewer.
template <int QB, bool EXACT>
__global__ __launch_bounds__(norm_threads(EXACT)) void combine_norm_kernel(
    const float *__restrict__ y, const float *__restrict__ gates, const uint32_t *__restrict__ ids,
    const int *__restrict__ pair_of, int k, int dim, float *__restrict__ out, const float *__restrict__ w, float eps,
    QAct qa) {
    __shared__ float red[4];
    __shared__ __align__(16) float sq[EXACT ? EXACT_NORM_MAX_DIM : 1];
    __shared__ __align__(16) float xs[EXACT_NORM_MAX_DIM];
    __shared__ SeqSumLds seq;
    __shared__ int ord[MAX_K], nord, sid[MAX_K], spair[MAX_K];
    __shared__ float sgate[MAX_K];
    const int t = blockIdx.x;
    const size_t base = (size_t)t * k;
    float4 gw[8];
    norm_weights(w, dim, gw); // in flight through the combine
    if ((int)threadIdx.x < k) {
        sid[threadIdx.x] = (int)ids[base + threadIdx.x];
        sgate[threadIdx.x] = gates[base + threadIdx.x];
        spair[threadIdx.x] = pair_of[base + threadIdx.x];
    }
    __syncthreads();
    if (threadIdx.x == 0) { // the slots in ascending expert id, the first slot of a repeated id
        int prev = -1, m = 0;
        for (int step = 0; step < k; step++) {
            int bs = -1, be = 0x7fffffff;
            for (int s2 = 0; s2 < k; s2++) {
                const int e = sid[s2];
                if (e > prev && e < be) {
                    be = e;
                    bs = s2;
                }
            }
            if (bs < 0)
                break;
            ord[m++] = bs;
            prev = be;
        }
        nord = m;
    }
    __syncthreads();
    const int m = nord;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        float acc = out[(size_t)t * dim + i];
        for (int j = 0; j < m; j++) {
            const int bs = ord[j];
            const float pr = sgate[bs] * y[(size_t)spair[bs] * dim + i];
            acc = acc + pr;
        }
        out[(size_t)t * dim + i] = acc;
        xs[i] = acc;
    }
    __syncthreads();
    norm_quant_row<QB, EXACT, true>(xs, dim, w, eps, qa, nullptr, t, red, sq, seq, gw);
}

template <int QB, bool EXACT>
static void launch_combine_norm_t(const float *y, const float *gates, const uint32_t *ids, const int *pair_of,
                                  int n, int k, int dim, float *out, const NextNorm &nx, hipStream_t st) {
    hipLaunchKernelGGL((combine_norm_kernel<QB, EXACT>), dim3(n), dim3(norm_threads(EXACT)), 0, st, y, gates, ids,
                       pair_of, k, dim, out, nx.w, nx.eps, nx.qa);
}

// Exact norms only: with the tree sum the norm launch is cheap, and the
// combine's 256-column work groups beat one work group per token (measured:
// FAST batch 32 8.77 against 8.72 ms/step fused).
bool launch_combine_norm(const float *y, const float *gates, const uint32_t *ids, const int *pair_of, int n,
                         int k, int dim, float *out, const NextNorm &nx, hipStream_t st) {
    if (!nx.exact || dim <= 0 || dim % 32 || dim > EXACT_NORM_MAX_DIM || k > MAX_K || (nx.qb != 32 && nx.qb != 256))
        return false;
    if (nx.qb == 256)
        launch_combine_norm_t<256, true>(y, gates, ids, pair_of, n, k, dim, out, nx, st);
    else
        launch_combine_norm_t<32, true>(y, gates, ids, pair_of, n, k, dim, out, nx, st);
    note_launch();
    return true;
}

// ---- per-head Q/K RMSNorm (llama.zig:938-949), RoPE (821-855), K/V append ----------
// Work group (head, lane): heads [0, n_heads) are query heads, the next
// n_kv are KV heads (their k rotated and appended, v appended as is).
__global__ __launch_bounds__(64) void qk_rope_kernel(FrameDims D, const float *__restrict__ q,
                                                     const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     const float *__restrict__ q_norm,
                                                     const float *__restrict__ k_norm,
                                                     const int32_t *__restrict__ pos, int li,
                                                     const float *__restrict__ rope_cs,
                                                     float *__restrict__ q_out,
                                                     uint16_t *__restrict__ q_split,
                                                     uint16_t *__restrict__ kc,
                                                     uint16_t *__restrict__ vc) {
    __shared__ float hv[MAX_HD];
    const int h = blockIdx.x, t = blockIdx.y, hd = D.hd, tid = threadIdx.x;
    const bool isq = h < D.n_heads;
    const int kvh = h - D.n_heads;
    const float *src = isq ? q + (size_t)t * D.qd + (size_t)h * hd : k + (size_t)t * D.kvd + (size_t)kvh * hd;
    const float *nw = isq ? q_norm : k_norm;
    __shared__ float s_inv;
    // the position, norm weights, value row and rope entries are requested
    // up front: none of them waits behind the norm's reduction
    constexpr int HPT = MAX_HD / 64, RPT = MAX_HD / 128;
    const int p = pos[t];
    const int half = D.rope_dim / 2;
    float nwv[HPT], vv[HPT];
#pragma unroll
    for (int u = 0; u < HPT; u++) {
        const int i = tid + 64 * u;
        nwv[u] = nw && i < hd ? nw[i] : 0.0f;
        vv[u] = !isq && i < hd ? v[(size_t)t * D.kvd + (size_t)kvh * hd + i] : 0.0f;
    }
    for (int i = tid; i < hd; i += 64)
        hv[i] = src[i];
    const float *csp = rope_cs + (size_t)min(max(p, 0), D.ctx - 1) * half * 2;
    float2 csv[RPT];
#pragma unroll
    for (int u = 0; u < RPT; u++) {
        const int i = tid + 64 * u;
        csv[u] = i < half ? make_float2(csp[2 * i], csp[2 * i + 1]) : make_float2(0.0f, 0.0f);
    }
    if (nw) {
        // headNorm's sum of squares in the reference's order (hd dependent
        // adds on one thread: the normalised heads feed the attention scores
        // and, through them, an int8-quantized matvec input)
        __syncthreads();
        if (tid == 0) {
            float ss = 0.0f;
            for (int i = 0; i < hd; i++) {
                const float pr = hv[i] * hv[i];
                ss = ss + pr;
            }
            s_inv = 1.0f / sqrtf(ss / (float)hd + D.eps);
        }
        __syncthreads();
        const float inv = s_inv;
#pragma unroll
        for (int u = 0; u < HPT; u++) {
            const int i = tid + 64 * u;
            if (i < hd)
                hv[i] = (hv[i] * inv) * nwv[u];
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < RPT; u++) {
        const int i = tid + 64 * u;
        if (i < half) {
            const float cs = csv[u].x, sn = csv[u].y;
            const int ia = D.rope_neox ? i : 2 * i, ib = D.rope_neox ? i + half : 2 * i + 1;
            const float a = hv[ia], b = hv[ib];
            hv[ia] = a * cs - b * sn;
            hv[ib] = a * sn + b * cs;
        }
    }
    __syncthreads();
    if (isq) {
        const size_t qo = (size_t)t * D.qd + (size_t)h * hd;
        for (int i = tid; i < hd; i += 64)
            q_out[qo + i] = hv[i];
        if (q_split) { // (f16 hi, f16 lo) with hi + lo = q to 22 bits, for the MFMA scores
            const size_t nq = (size_t)gridDim.y * D.qd;
            for (int i = tid; i < hd; i += 64) {
                const _Float16 hi = (_Float16)hv[i];
                const _Float16 lo = (_Float16)(hv[i] - (float)hi);
                q_split[qo + i] = __builtin_bit_cast(uint16_t, hi);
                q_split[nq + qo + i] = __builtin_bit_cast(uint16_t, lo);
            }
        }
        return;
    }
    if (p < 0 || p >= D.ctx) // a full cache takes no more rows
        return;
    const size_t base = (((size_t)t * D.n_layers + li) * D.ctx + p) * D.kvd + (size_t)kvh * hd;
#pragma unroll
    for (int u = 0; u < HPT; u++) {
        const int i = tid + 64 * u;
        if (i < hd) {
            kc[base + i] = __half_raw(__float2half(hv[i])).x;
            vc[base + i] = __half_raw(__float2half(vv[u])).x;
        }
    }
}

// Work group (chunk, kv head, lane), 8 waves.  Waves 0-3 load the chunk's
// keys and the group's query heads, waves 4-7 its values, all loads issued
// up front (rows past nt repeat row nt-1: finite, never weighted).
//
// One chunk (position < 64): the reference's own arithmetic (softmax,
// tensor.zig:18-28, then out += p * v in position order), on the VALU.
// Wave w takes query heads w, w+8, ...: lane j scores key j in dotF32 order
// (keys in LDS rows padded by 16 bytes), m = max, e = exp(s - m), l = sum of e
// in position order, p = e * (1/l); P.V with each lane on CPL columns,
// positions in order.  Record: m, l = 1, o = sum_t p_t v_t.
//
// Split context in FAST numerics (HD a multiple of 32): matrix cores.  (In
// PARITY numerics a split context takes the VALU path above, its scores in
// dotF32 order and l a tree sum, for the merge.)  The group's query
// heads are the 16 rows of the MFMA tiles (G <= 16; rows past G are zero).
// Scores S = Q K^T with v_mfma_f32_16x16x32_f16: the f32 query split into
// two f16 parts (hi = f16(q), lo = f16(q - hi), 22 significant bits) against
// the exact fp16 keys, f32 accumulation; wave w < 4 scores positions 16w..
// 16w+15.  Per head m = max, e = exp(s - m), l = a tree sum of e.  Then
// O = P V with p split the same way against the fp16 values (staged by
// waves 4-7 while the scores run, rows padded by 4 bytes, each lane
// gathering its 8 positions of one column); wave w computes columns
// 16w..16w+15.  Record: m, l, o = sum_t e_t v_t,
// unnormalised, for the merge.  Record per (lane, kv head, chunk): m[G],
// l[G], o[G][HD].
constexpr int ATT_WAVES = 8;
constexpr size_t ATT_FUSE_MAX_LANES = 4; // lanes up to which rope/append run inside the attention
constexpr int ATT_TC_DIRECT = 128;         // positions per work group of attn_direct_kernel

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// 8 floats -> (f16 hi, f16 lo) with hi + lo = v to 22 significant bits.
__device__ __forceinline__ void split_f16(const float4 &a, const float4 &b, half8_t &hi, half8_t &lo) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const _Float16 h = (_Float16)v[i];
        hi[i] = h;
        lo[i] = (_Float16)(v[i] - (float)h);
    }
}

template <int HD>
__global__ __launch_bounds__(64 * ATT_WAVES) void attn_partial_kernel(FrameDims D, const float *__restrict__ qraw,
                                                                      const float *__restrict__ kraw,
                                                                      const float *__restrict__ vraw,
                                                                      const float *__restrict__ q_norm,
                                                                      const float *__restrict__ k_norm,
                                                                      const float *__restrict__ rope_cs,
                                                                      uint16_t *__restrict__ kc,
                                                                      uint16_t *__restrict__ vc,
                                                                      const int32_t *__restrict__ pos, int li,
                                                                      int n_chunks, int use_mfma, int fuse,
                                                                      float *__restrict__ part) {
    extern __shared__ __align__(16) float smem[];
    constexpr int KS = HD + 8;                 // padded key row (halves)
    constexpr int VS = HD + 2;                 // padded value row (halves)
    constexpr int PR = HD / 8;                 // 16-byte pieces per row
    constexpr int CPL = HD > 64 ? 2 : 1;       // VALU P.V columns per lane
    constexpr int NPW = (ATT_TC * PR + 255) / 256; // 16-byte pieces per thread of a half work group
    constexpr bool MF = HD % 32 == 0;
    const int ch = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int G = D.n_heads / D.n_kv;
    const int p_raw = pos[t];
    const int p = min(p_raw, D.ctx - 1);
    const int t0 = ch * ATT_TC, nt = min(ATT_TC, p + 1 - t0);
    if (nt <= 0)
        return; // past the current position: the merge reads no record from here
    const bool single = p + 1 <= ATT_TC;
    // fuse (few lanes): the query heads arrive raw and get their RMSNorm and
    // RoPE here; the chunk that holds the new position appends the step's
    // K/V row (a full cache takes no more rows) and uses it from LDS.
    // Otherwise qk_rope_kernel did both and qraw holds the rotated queries.
    const bool own = fuse && p_raw >= 0 && p_raw < D.ctx && p_raw >= t0 && p_raw < t0 + ATT_TC;
    const int rp = min(max(p_raw, 0), D.ctx - 1); // rope position
    float *qs = smem;                                  // [G][HD] f32
    float *sc = qs + G * HD;                           // [16][TC] f32: p of head g, position j
    uint16_t *ks = (uint16_t *)(sc + 16 * ATT_TC);     // [TC][KS]
    uint16_t *vs = ks + ATT_TC * KS;                   // [TC][VS]
    __shared__ float red[2][4][16];
    __shared__ float kn[HD], sinv[MAX_G + 1];
    const int wave = tid >> 6, ln = tid & 63, half = tid >> 8, ht = tid & 255;
    const size_t row0 = (((size_t)t * D.n_layers + li) * D.ctx + t0) * D.kvd + (size_t)kvh * HD;
    const float *qsrc = qraw + (size_t)t * D.qd + (size_t)kvh * G * HD;
    const size_t kvo = (size_t)t * D.kvd + (size_t)kvh * HD;
    // half 0: keys and the group's query heads, half 1: values (and the new row)
    const uint16_t *src = half ? vc : kc;
    uint4 pc[NPW];
#pragma unroll
    for (int u = 0; u < NPW; u++) {
        const int i = ht + 256 * u;
        pc[u] = *(const uint4 *)(src + row0 + (size_t)min(i / PR, nt - 1) * D.kvd + 8 * (i % PR));
    }
    float vnew = 0.0f;
    if (half == 0) {
        for (int i = ht; i < G * HD; i += 256)
            qs[i] = qsrc[i];
#pragma unroll
        for (int u = 0; u < NPW; u++) {
            const int i = ht + 256 * u;
            if (i < ATT_TC * PR)
                *(uint4 *)(ks + (i / PR) * KS + 8 * (i % PR)) = pc[u];
        }
    } else {
        if (own && ht < HD) {
            kn[ht] = kraw[kvo + ht];
            vnew = vraw[kvo + ht];
        }
#pragma unroll
        for (int u = 0; u < NPW; u++) { // values: 4-byte stores into the padded rows
            const int i = ht + 256 * u;
            if (i < ATT_TC * PR) {
                uint32_t *vrow = (uint32_t *)(vs + (i / PR) * VS + 8 * (i % PR));
                vrow[0] = pc[u].x;
                vrow[1] = pc[u].y;
                vrow[2] = pc[u].z;
                vrow[3] = pc[u].w;
            }
        }
    }
    __syncthreads();
    if (fuse) {
    // per-head RMSNorm (llama.zig:938-949): PARITY sums the squares in the
    // reference's order, one thread per head; FAST (use_mfma) one wave per
    // head, a fixed tree
    if (q_norm) {
        if (use_mfma) {
            if (half == 0)
                for (int g = wave; g < G; g += 4) {
                    float ss = 0.0f;
                    for (int i = ln; i < HD; i += 64)
                        ss = ss + qs[g * HD + i] * qs[g * HD + i];
                    ss = wave_sum_f(ss);
                    if (ln == 0)
                        sinv[g] = 1.0f / sqrtf(ss / (float)HD + D.eps);
                }
        } else if (tid < G) {
            float ss = 0.0f;
            for (int i = 0; i < HD; i++) {
                const float pr = qs[tid * HD + i] * qs[tid * HD + i];
                ss = ss + pr;
            }
            sinv[tid] = 1.0f / sqrtf(ss / (float)HD + D.eps);
        }
    }
    if (own && k_norm) {
        if (use_mfma) {
            if (wave == 4) {
                float ss = 0.0f;
                for (int i = ln; i < HD; i += 64)
                    ss = ss + kn[i] * kn[i];
                ss = wave_sum_f(ss);
                if (ln == 0)
                    sinv[MAX_G] = 1.0f / sqrtf(ss / (float)HD + D.eps);
            }
        } else if (tid == 256) {
            float ss = 0.0f;
            for (int i = 0; i < HD; i++) {
                const float pr = kn[i] * kn[i];
                ss = ss + pr;
            }
            sinv[MAX_G] = 1.0f / sqrtf(ss / (float)HD + D.eps);
        }
    }
    __syncthreads();
    if (half == 0) {
        if (q_norm)
            for (int i = ht; i < G * HD; i += 256)
                qs[i] = (qs[i] * sinv[i / HD]) * q_norm[i % HD];
    } else if (own && k_norm && ht < HD) {
        kn[ht] = (kn[ht] * sinv[MAX_G]) * k_norm[ht];
    }
    __syncthreads();
    // RoPE (llama.zig:821-855) from the (cos, sin) table at the position
    {
        const int hr = D.rope_dim / 2;
        const float *csp = rope_cs + (size_t)rp * hr * 2;
        if (half == 0) {
            for (int i = ht; i < G * hr; i += 256) {
                const int g = i / hr, r = i % hr;
                const float cs = csp[2 * r], sn = csp[2 * r + 1];
                const int ia = D.rope_neox ? r : 2 * r, ib = D.rope_neox ? r + hr : 2 * r + 1;
                const float a = qs[g * HD + ia], b = qs[g * HD + ib];
                qs[g * HD + ia] = a * cs - b * sn;
                qs[g * HD + ib] = a * sn + b * cs;
            }
        } else if (own && ht < hr) {
            const float cs = csp[2 * ht], sn = csp[2 * ht + 1];
            const int ia = D.rope_neox ? ht : 2 * ht, ib = D.rope_neox ? ht + hr : 2 * ht + 1;
            const float a = kn[ia], b = kn[ib];
            kn[ia] = a * cs - b * sn;
            kn[ib] = a * sn + b * cs;
        }
    }
    __syncthreads();
    if (own && half && ht < HD) { // the new row: to the cache and over its stale LDS copy
        const uint16_t kh = __half_raw(__float2half(kn[ht])).x, vh = __half_raw(__float2half(vnew)).x;
        const size_t crow = (((size_t)t * D.n_layers + li) * D.ctx + p_raw) * D.kvd + (size_t)kvh * HD;
        kc[crow + ht] = kh;
        vc[crow + ht] = vh;
        ks[(p_raw - t0) * KS + ht] = kh;
        vs[(p_raw - t0) * VS + ht] = vh;
    }
    __syncthreads();
    }
    float *rec = part + (((size_t)t * D.n_kv + kvh) * n_chunks + ch) * (size_t)G * (HD + 2);

    if (!MF || single || !use_mfma) {
        const uint16_t *krow = ks + min(ln, nt - 1) * KS;
        for (int g = wave; g < G; g += ATT_WAVES) {
            const float s = ln < nt ? dot_f32_key<HD>(qs + g * HD, krow) * D.scale : -INFINITY;
            const float m = wave_max(s);
            float e = ln < nt ? exp_f32(s - m) : 0.0f;
            float l;
            if (single) {
                l = 0.0f;
                for (int j = 0; j < nt; j++) // the reference's sum order
                    l = l + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
                const float inv = 1.0f / l;
                e = e * inv;
            } else {
                l = wave_sum_f(e);
            }
            sc[g * ATT_TC + ln] = e;
            if (ln == 0) {
                rec[g] = m;
                rec[G + g] = single ? 1.0f : l;
            }
        }
        __syncthreads();
        const int d0 = CPL * ln;
        if (d0 >= HD)
            return;
        for (int g = wave; g < G; g += ATT_WAVES) {
            const float *pg = sc + g * ATT_TC;
            float a0 = 0.0f, a1 = 0.0f;
            for (int j0 = 0; j0 < nt; j0 += 8) {
                const float4 pa = *(const float4 *)(pg + j0), pb = *(const float4 *)(pg + j0 + 4);
                const float pj[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
                uint32_t vw[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int j = min(j0 + u, ATT_TC - 1);
                    if constexpr (CPL == 2)
                        vw[u] = *(const uint32_t *)(vs + j * VS + d0);
                    else
                        vw[u] = vs[j * VS + d0];
                }
                // positions past nt have p = 0 and a finite v (a repeated row):
                // they add +0 to accumulators that are never -0, no change
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    a0 = a0 + pj[u] * half_bits_to_float((uint16_t)(vw[u] & 0xffff));
                    if constexpr (CPL == 2)
                        a1 = a1 + pj[u] * half_bits_to_float((uint16_t)(vw[u] >> 16));
                }
            }
            rec[2 * G + g * HD + d0] = a0;
            if constexpr (CPL == 2)
                rec[2 * G + g * HD + d0 + 1] = a1;
        }
        return;
    }

    if constexpr (MF) {
        const int r16 = ln & 15, q4 = ln >> 4; // tile row/column, k-quarter
        float sv[4];
        if (half == 0) {
            // scores of positions 16w..16w+15
            const int j = 16 * wave + r16;
            const uint16_t *krow = ks + min(j, nt - 1) * KS;
            const bool hrow = r16 < G;
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < HD / 32; kk++) {
                const int d = 32 * kk + 8 * q4;
                const half8_t b = *(const half8_t *)(krow + d);
                float4 qa = {0.0f, 0.0f, 0.0f, 0.0f}, qb = qa;
                if (hrow) {
                    qa = *(const float4 *)(qs + r16 * HD + d);
                    qb = *(const float4 *)(qs + r16 * HD + d + 4);
                }
                half8_t ahi, alo;
                split_f16(qa, qb, ahi, alo);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, acc, 0, 0, 0);
            }
            // lane: position j, heads 4*q4 .. 4*q4+3
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sv[r] = j < nt ? acc[r] * D.scale : -INFINITY;
                const float v = group16_max(sv[r]);
                if (r16 == 0)
                    red[0][wave][4 * q4 + r] = v;
            }
        }
        __syncthreads();
        if (half == 0) {
            const int j = 16 * wave + r16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int hh = 4 * q4 + r;
                const float m = fmaxf(fmaxf(red[0][0][hh], red[0][1][hh]), fmaxf(red[0][2][hh], red[0][3][hh]));
                // FAST numerics only: the hardware exp (a few ulp) in place of
                // the once-rounded double exp
                const float e = j < nt ? __expf(sv[r] - m) : 0.0f;
                sc[hh * ATT_TC + j] = e;
                const float v = group16_sum(e);
                if (r16 == 0)
                    red[1][wave][hh] = v;
                if (wave == 0 && r16 == 0 && hh < G)
                    rec[hh] = m;
            }
        }
        __syncthreads();
        if (tid < G)
            rec[G + tid] = ((red[1][0][tid] + red[1][1][tid]) + red[1][2][tid]) + red[1][3][tid];
        if (wave < HD / 16) {
            // O columns 16w..16w+15: rows = heads, k = positions
            const int dcol = 16 * wave + r16;
            const bool hrow = r16 < G;
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks2 = 0; ks2 < ATT_TC / 32; ks2++) {
                const int j = 32 * ks2 + 8 * q4;
                half8_t b;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    b[e] = __builtin_bit_cast(_Float16, vs[(j + e) * VS + dcol]);
                float4 pa = {0.0f, 0.0f, 0.0f, 0.0f}, pb = pa;
                if (hrow) {
                    pa = *(const float4 *)(sc + r16 * ATT_TC + j);
                    pb = *(const float4 *)(sc + r16 * ATT_TC + j + 4);
                }
                half8_t ahi, alo;
                split_f16(pa, pb, ahi, alo);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, acc, 0, 0, 0);
            }
            // lane: column dcol, heads 4*q4 .. 4*q4+3
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int hh = 4 * q4 + r;
                if (hh < G)
                    rec[2 * G + hh * HD + dcol] = acc[r];
            }
        }
    }
}

// ---- attention, FAST with rope done apart (more than ATT_FUSE_MAX_LANES lanes) -------
// Work group (chunk of TC positions, KV head, lane), 8 waves.  Wave w scores
// positions 16w + 16*8*i .. (TC/16 tiles over the 8 waves) on the matrix cores
// from keys loaded straight from HBM into the MFMA operands and the queries
// pre-split into (f16 hi, f16 lo) by qk_rope_kernel; every thread stages its
// share of the values into LDS meanwhile.  Then p = exp(s - m) against the
// chunk max of each head (hardware exp: FAST numerics), the chunk sums, and
// O = P V with p split the same way, wave w taking columns 16w..16w+15.
// Record per (lane, KV head, chunk): m[G], l[G], o[G][HD] unnormalised.
template <int HD, int TC>
__global__ __launch_bounds__(64 * ATT_WAVES) __attribute__((amdgpu_waves_per_eu(6))) void attn_direct_kernel(FrameDims D, const uint16_t *__restrict__ kc,
                                                                     const uint16_t *__restrict__ vc,
                                                                     const int32_t *__restrict__ pos, int li,
                                                                     int n_chunks,
                                                                     const uint16_t *__restrict__ qsplit,
                                                                     float *__restrict__ part) {
    static_assert(HD % 32 == 0 && (TC == 64 || TC % 128 == 0), "MFMA head size; 64 or a multiple of 128 positions");
    extern __shared__ __align__(16) float smem[];
    constexpr int VS = HD + 2;                      // padded value row (halves)
    constexpr int PR = HD / 8;                      // 16-byte pieces per row
    constexpr int NPW = (TC * PR + 511) / 512;      // value pieces per thread
    constexpr int NK = HD / 32;
    constexpr int NT = TC / 16 / ATT_WAVES > 0 ? TC / 16 / ATT_WAVES : 1; // score tiles per wave
    constexpr int SW = TC / 16 < ATT_WAVES ? TC / 16 : ATT_WAVES;        // waves that score
    const int ch = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int G = D.n_heads / D.n_kv;
    const int p = min(pos[t], D.ctx - 1);
    const int t0 = ch * TC, nt = min(TC, p + 1 - t0);
    if (nt <= 0)
        return; // past the current position: the merge reads no record from here
    float *sc = smem;                              // [16][TC] f32: p of head g, position j
    uint16_t *vs = (uint16_t *)(sc + 16 * TC);     // [TC][VS]
    __shared__ float red[2][ATT_WAVES][16];
    const int wave = tid >> 6, ln = tid & 63;
    const int r16 = ln & 15, q4 = ln >> 4;
    const size_t row0 = (((size_t)t * D.n_layers + li) * D.ctx + t0) * D.kvd + (size_t)kvh * HD;
    const bool hrow = r16 < G;
    const bool scorer = wave < SW;
    // 1. the loads: keys and split queries (scoring waves), values (all)
    half8_t kb[NT][NK], qh[NK], ql[NK];
    if (scorer) {
#pragma unroll
        for (int i = 0; i < NT; i++) {
            const int j = 16 * (wave + ATT_WAVES * i) + r16;
            const uint16_t *kr = kc + row0 + (size_t)min(j, nt - 1) * D.kvd + 8 * q4;
#pragma unroll
            for (int kk = 0; kk < NK; kk++)
                kb[i][kk] = *(const half8_t *)(kr + 32 * kk);
        }
        const size_t qo = (size_t)t * D.qd + ((size_t)kvh * G + min(r16, G - 1)) * HD + 8 * q4;
        const size_t nq = (size_t)gridDim.z * D.qd;
        const half8_t zh = {};
#pragma unroll
        for (int kk = 0; kk < NK; kk++) {
            qh[kk] = hrow ? *(const half8_t *)(qsplit + qo + 32 * kk) : zh;
            ql[kk] = hrow ? *(const half8_t *)(qsplit + nq + qo + 32 * kk) : zh;
        }
    }
    uint4 pv[NPW];
#pragma unroll
    for (int u = 0; u < NPW; u++) {
        const int i = tid + 512 * u;
        pv[u] = *(const uint4 *)(vc + row0 + (size_t)min(i / PR, nt - 1) * D.kvd + 8 * (i % PR));
    }
    // 2. scores and the chunk max per head
    float sv[NT][4];
    if (scorer) {
#pragma unroll
        for (int i = 0; i < NT; i++) {
            const int j = 16 * (wave + ATT_WAVES * i) + r16;
            f32x4_t a = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < NK; kk++) {
                a = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[kk], kb[i][kk], a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[kk], kb[i][kk], a, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++)
                sv[i][r] = j < nt ? a[r] * D.scale : -INFINITY;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float m = sv[0][r];
#pragma unroll
            for (int i = 1; i < NT; i++)
                m = fmaxf(m, sv[i][r]);
            const float v = group16_max(m);
            if (r16 == 0)
                red[0][wave][4 * q4 + r] = v;
        }
    }
#pragma unroll
    for (int u = 0; u < NPW; u++) { // values: 4-byte stores into the padded rows
        const int i = tid + 512 * u;
        if (i < TC * PR) {
            uint32_t *vrow = (uint32_t *)(vs + (i / PR) * VS + 8 * (i % PR));
            vrow[0] = pv[u].x;
            vrow[1] = pv[u].y;
            vrow[2] = pv[u].z;
            vrow[3] = pv[u].w;
        }
    }
    __syncthreads();
    // 3. p = exp(s - m), the chunk sums
    float *rec = part + (((size_t)t * D.n_kv + kvh) * n_chunks + ch) * (size_t)G * (HD + 2);
    if (scorer) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int hh = 4 * q4 + r;
            float m = red[0][0][hh];
            for (int w = 1; w < SW; w++)
                m = fmaxf(m, red[0][w][hh]);
            float ssum = 0.0f;
#pragma unroll
            for (int i = 0; i < NT; i++) {
                const int j = 16 * (wave + ATT_WAVES * i) + r16;
                const float e = j < nt ? __expf(sv[i][r] - m) : 0.0f;
                sc[hh * TC + j] = e;
                ssum = ssum + e;
            }
            const float v = group16_sum(ssum);
            if (r16 == 0)
                red[1][wave][hh] = v;
            if (wave == 0 && r16 == 0 && hh < G)
                rec[hh] = m;
        }
    }
    __syncthreads();
    if (tid < G) {
        float l = red[1][0][tid];
        for (int w = 1; w < SW; w++)
            l = l + red[1][w][tid];
        rec[G + tid] = l;
    }
    // 4. O columns 16w..16w+15: rows = heads, k = positions
    if (wave < HD / 16) {
        const int dcol = 16 * wave + r16;
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks2 = 0; ks2 < TC / 32; ks2++) {
            const int j = 32 * ks2 + 8 * q4;
            half8_t b;
#pragma unroll
            for (int e = 0; e < 8; e++)
                b[e] = __builtin_bit_cast(_Float16, vs[(j + e) * VS + dcol]);
            float4 pa = {0.0f, 0.0f, 0.0f, 0.0f}, pb = pa;
            if (hrow) {
                pa = *(const float4 *)(sc + r16 * TC + j);
                pb = *(const float4 *)(sc + r16 * TC + j + 4);
            }
            half8_t ahi, alo;
            split_f16(pa, pb, ahi, alo);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int hh = 4 * q4 + r;
            if (hh < G)
                rec[2 * G + hh * HD + dcol] = acc[r];
        }
    }
}

// ---- merge the partials per head, quantize the attention output for wo -------------
// Work group (256-value slice, lane), 1024 threads: value v = tid % 256 of the
// slice, chunk quarter cq = tid / 256 (chunks cq, cq+4, ...).  Blocks of QB
// values are QB consecutive values (QB = 32: half a wave; 256: the slice).
// The merge weights of the slice's heads (at most CMB_NH of them) are formed
// once, one wave per head: M = max_c m_c, w_c = exp(m_c - M), L = sum_c w_c
// l_c; each quarter then sums w_c o_c[d] over its chunks with the o loads
// issued before the weights are known, and o = (the quarters' sums in order)
// / L.
constexpr int CMB_NH = 8;  // heads a 256-value slice can touch (head_dim >= 48)
constexpr int CMB_OP = 16; // chunks per quarter held in registers (64 chunks in one pass; more in a tail loop)

template <int QB>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(8))) void attn_combine_kernel(FrameDims D, const float *__restrict__ part,
                                                            const int32_t *__restrict__ pos,
                                                            int n_chunks, int span, int merge_one, QAct qa) {
    extern __shared__ float cmb[]; // [4][256] quarter sums, then [CMB_NH][n_chunks] weights
    __shared__ float red[4], Ls[CMB_NH];
    const int t = blockIdx.y, tid = threadIdx.x, v = tid & 255, cq = tid >> 8;
    const int wave = tid >> 6, ln = tid & 63;
    const int idx = blockIdx.x * 256 + v;
    const bool live = idx < D.qd && cq == 0;
    const int hd = D.hd, G = D.n_heads / D.n_kv;
    const int ic = idx < D.qd ? idx : D.qd - 1;
    const int h = ic / hd, d = ic % hd;
    const int h_lo = blockIdx.x * 256 / hd;
    const int nh = (min(blockIdx.x * 256 + 255, D.qd - 1)) / hd - h_lo + 1;
    const int kvh = h / G, g = h % G;
    const int p = min(pos[t], D.ctx - 1);
    const int nc = p < 0 ? 0 : p / span + 1; // records that hold positions (none at a negative position)
    const size_t rs = (size_t)G * (hd + 2);
    const float *rec0 = part + ((size_t)t * D.n_kv + kvh) * n_chunks * rs;
    float val;
    if (nc == 0) { // no context: +0, as the exact path (nc is uniform over the group)
        val = 0.0f;
    } else if (nc == 1 && !merge_one) { // one chunk: its record is already the softmax-weighted sum
        val = rec0[2 * G + (size_t)g * hd + d];
    } else {
        float *wt = cmb + 4 * 256;
        const float *orow = rec0 + 2 * G + (size_t)g * hd + d;
        float ov[CMB_OP];
#pragma unroll
        for (int u = 0; u < CMB_OP; u++) // cq is uniform per wave: chunks past nc are not requested
            ov[u] = cq + 4 * u < nc ? orow[(size_t)(cq + 4 * u) * rs] : 0.0f;
        if (wave < nh) {
            const int hw = h_lo + wave, kw = hw / G, gw = hw % G;
            const float *r0 = part + ((size_t)t * D.n_kv + kw) * n_chunks * rs;
            float M = -INFINITY;
            for (int c = ln; c < nc; c += 64)
                M = fmaxf(M, r0[(size_t)c * rs + gw]);
            M = wave_max(M);
            float lp = 0.0f;
            for (int c = ln; c < nc; c += 64) {
                const float wc = exp_f32(r0[(size_t)c * rs + gw] - M);
                wt[wave * nc + c] = wc;
                lp = lp + r0[(size_t)c * rs + G + gw] * wc;
            }
            const float L = wave_sum_f(lp);
            if (ln == 0)
                Ls[wave] = L;
        }
        __syncthreads();
        const float *wh = wt + (h - h_lo) * nc;
        float o = 0.0f;
#pragma unroll
        for (int u = 0; u < CMB_OP; u++) {
            const int c = cq + 4 * u;
            if (c < nc)
                o = o + wh[c] * ov[u];
        }
        for (int c = cq + 4 * CMB_OP; c < nc; c += 4)
            o = o + wh[c] * orow[(size_t)c * rs];
        cmb[cq * 256 + v] = o;
        __syncthreads();
        val = (((cmb[v] + cmb[256 + v]) + cmb[512 + v]) + cmb[768 + v]) / Ls[h - h_lo];
    }
    // int8 quantization (quantizeX / quantizeX256) of QB-thread blocks
    float a = live && __builtin_isfinite(val) ? fabsf(val) : 0.0f;
    if constexpr (QB == 32) {
        for (int m = 1; m < 32; m <<= 1)
            a = fmaxf(a, __shfl_xor(a, m, 32));
    } else {
        const float wm = wave_max(a);
        if (wave < 4 && ln == 0)
            red[wave] = wm;
        __syncthreads();
        a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
    const float dd = a / 127.0f;
    const float inv = (dd != 0.0f && __builtin_isfinite(dd)) ? 1.0f / dd : 0.0f;
    const int qv = live ? to_i8_sat(val * inv) : 0;
    int sum = qv;
    constexpr int SG = QB == 256 ? 16 : 32; // sum groups: per 16 (K-quants) or per block
    for (int m = 1; m < SG; m <<= 1)
        sum += __shfl_xor(sum, m, SG);
    if (!live)
        return;
    const size_t vb = (size_t)t * D.qd;
    qa.q[vb + idx] = (int8_t)qv;
    if (idx % SG == 0)
        qa.s[(size_t)t * (D.qd / SG) + idx / SG] = sum;
    if (idx % QB == 0)
        qa.d[(size_t)t * (D.qd / QB) + idx / QB] = __builtin_isfinite(dd) ? dd : 0.0f;
}

// ---- greedy pick (engine/sampler.zig:7-15: the first maximum wins), pos += 1 ------

// Two launches: ARGMAX_SLICES work groups per lane each take a contiguous
// slice (threads walk it in index order, strict >, so each keeps its first
// maximum), then one wave per lane merges the slices by (value desc, index
// asc) -- the first maximum overall.  No value above -inf (all -inf or NaN):
// index 0, as the reference's loop leaves it.
constexpr int ARGMAX_SLICES = 64;

__device__ __forceinline__ void argmax_pair(float &best, int &besti, float ov, int oi) {
    if (ov > best || (ov == best && oi < besti)) {
        best = ov;
        besti = oi;
    }
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const float *__restrict__ logits, int vocab,
                                                          float *__restrict__ pv, int *__restrict__ pi) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int s = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int slice = (vocab + ARGMAX_SLICES - 1) / ARGMAX_SLICES;
    const int lo = s * slice, hi = min(vocab, lo + slice);
    const float *lg = logits + (size_t)t * vocab;
    float best = -INFINITY;
    int besti = 0x7fffffff; // no candidate yet
    for (int i = lo + tid; i < hi; i += 256) {
        const float v = lg[i];
        if (v > best) {
            best = v;
            besti = i;
        }
    }
    for (int m = 1; m < 64; m <<= 1)
        argmax_pair(best, besti, __shfl_xor(best, m), __shfl_xor(besti, m));
    if ((tid & 63) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = besti;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; w++)
            argmax_pair(best, besti, bv[w], bi[w]);
        pv[t * ARGMAX_SLICES + s] = best;
        pi[t * ARGMAX_SLICES + s] = besti;
    }
}

__global__ __launch_bounds__(64) void argmax_merge_kernel(const float *__restrict__ pv, const int *__restrict__ pi,
                                                          uint32_t *__restrict__ next, int32_t *__restrict__ pos) {
    const int t = blockIdx.x, ln = threadIdx.x;
    float best = ln < ARGMAX_SLICES ? pv[t * ARGMAX_SLICES + ln] : -INFINITY;
    int besti = ln < ARGMAX_SLICES ? pi[t * ARGMAX_SLICES + ln] : 0x7fffffff;
    for (int m = 1; m < 64; m <<= 1)
        argmax_pair(best, besti, __shfl_xor(best, m), __shfl_xor(besti, m));
    if (ln == 0) {
        if (next)
            next[t] = besti == 0x7fffffff ? 0u : (uint32_t)besti;
        pos[t] = pos[t] + 1;
    }
}

// ---- host -------------------------------------------------------------------------


static Scratch g_frame; // per-call workspace

// RoPE tables computed on the host in ropeTheta's expressions
// (llama.zig:821-826): exponent = i / rope_dim for the even index i,
// freq = powf(base, -exponent), angle = pos * freq; kept per (ctx, rope_dim,
// base) for the process.
static const float *rope_table(int ctx, int rope_dim, float base) {
    static std::unordered_map<std::string, float *> tables;
    char key[96];
    snprintf(key, sizeof key, "%d/%d/%a", ctx, rope_dim, base);
    auto it = tables.find(key);
    if (it != tables.end())
        return it->second;
    const int half = rope_dim / 2;
    std::vector<float> h((size_t)ctx * half * 2);
    for (int p = 0; p < ctx; p++)
        for (int i = 0; i < half; i++) {
            const float exponent = (float)(2 * i) / (float)rope_dim;
            const float freq = powf(base, -exponent);
            const float angle = (float)p * freq;
            h[((size_t)p * half + i) * 2] = cosf(angle);
            h[((size_t)p * half + i) * 2 + 1] = sinf(angle);
        }
    float *d = nullptr;
    if (hipMalloc(&d, h.size() * 4) != hipSuccess)
        return nullptr;
    if (hipMemcpy(d, h.data(), h.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return nullptr;
    }
    tables[key] = d;
    return d;
}

static FrameWs frame_layout(char *base, size_t n, const loomhip_model *m, size_t ffn_max,
                            int n_chunks, bool parity) {
    FrameWs w{};
    size_t off = 0;
    auto take = [&](size_t b) {
        size_t o = off;
        off += align16(b);
        return base ? base + o : nullptr;
    };
    const size_t dim = m->dim, qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
    const size_t G = m->n_heads / m->n_kv_heads;
    auto qtake = [&](size_t cols) {
        QAct q;
        q.q = (int8_t *)take(n * cols);
        q.d = (float *)take(n * (cols / 32) * 4);
        q.s = (int32_t *)take(n * (cols / 16) * 4);
        return q;
    };
    w.x = (float *)take(n * dim * 4);
    w.normed = (float *)take(n * dim * 4);
    w.q = (float *)take(n * qd * 4);
    w.k = (float *)take(n * kvd * 4);
    w.v = (float *)take(n * kvd * 4);
    w.qrot = (float *)take(n * qd * 4);
    w.qsplit = (uint16_t *)take(n * qd * 4);
    w.part = (float *)take(n * m->n_kv_heads * (size_t)n_chunks * G * (m->head_dim + 2) * 4);
    w.act = (float *)take(n * (ffn_max ? ffn_max : 1) * 4);
    w.s_stride = (int)((m->ctx_len + 63) / 64 * 64);
    w.S = (float *)take(parity ? n * m->n_heads * (size_t)w.s_stride * 4 : 16);
    w.att = (float *)take(parity ? n * qd * 4 : 16);
    w.amax_v = (float *)take(n * ARGMAX_SLICES * 4);
    w.amax_i = (int *)take(n * ARGMAX_SLICES * 4);
    w.qa_dim = qtake(dim);
    w.qa_att = qtake(qd);
    w.qa_ffn = qtake(ffn_max ? ffn_max : 32);
    w.bytes = off;
    return w;
}

// mmq_ok: the matrix cores from MMQ_MIN_TOK lanes on, in groups of mmq_group
// lanes (16 for wo: more work groups for its 2048 rows; 32 for the head,
// whose 255 MB would be read once per group).
static bool frame_matvec(int t, const void *wt, int rows, int cols, const FrameWs &w, size_t n,
                         QAct x, float *out, int accumulate, hipStream_t st, int tag = LOOMHIP_KT_DENSE,
                         bool mmq_ok = false, int mmq_group = 32) {
    DmmvParams p{};
    p.w = (const uint8_t *)wt;
    p.plane_bytes = 0;
    p.rows = rows;
    p.cols = cols;
    p.xq = x.q;
    p.xd = x.d;
    p.xs = x.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = w.groups;
    p.n_groups = w.n_groups;
    p.out = out;
    p.out_stride = rows;
    p.accumulate = accumulate;
    const bool mq = mmq_ok && use_mmq(t, cols, (int)n, 32, false);
    if (mq)
        p.ident_n = (int)n;
    p.rpw = mq ? 0 : dmmv_pick_rpw(t, cols, rows, w.n_groups, w.nt, false);
    const int ph = prof_begin(tag, st);
    const bool ok = mq ? launch_mmq(t, mmq_group, false, p, st) : launch_dmmv(t, w.nt, false, p, st);
    prof_end(ph, st);
    return ok;
}

// q, k and v of one layer against the normalised input, one launch.  With
// fused: one lane in PARITY, the launch normalises x itself (the exact sum)
// and true means both steps ran; false with *fused cleared: not served, the
// caller normalises and calls again without.
static bool frame_qkv(const loomhip_layer &l, const FrameDims &D, const FrameWs &w, size_t n, hipStream_t st,
                      bool *fused = nullptr) {
    DmmvSegParams sp{};
    DmmvParams &p = sp.base;
    p.cols = D.dim;
    p.xq = w.qa_dim.q;
    p.xd = w.qa_dim.d;
    p.xs = w.qa_dim.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = w.groups;
    p.n_groups = w.n_groups;
    sp.seg[0] = DmmvSeg{(const uint8_t *)l.wq, l.wq_t, D.qd, w.q, 0, 0};
    sp.seg[1] = DmmvSeg{(const uint8_t *)l.wk, l.wk_t, D.kvd, w.k, 0, 0};
    sp.seg[2] = DmmvSeg{(const uint8_t *)l.wv, l.wv_t, D.kvd, w.v, 0, 0};
    sp.n_seg = 3;
    if (fused) { // one lane only, before any other path
        *fused = false;
        if (n != 1)
            return false;
        const int ph = prof_begin(LOOMHIP_KT_QKV, st);
        *fused = launch_norm_seg(sp, w.x, l.attn_norm, D.eps, st);
        prof_end(ph, st);
        return *fused;
    }
    // from MMQ_MIN_TOK lanes: the matrix cores, the three matrices in one
    // launch, lanes in groups of 16
    if (use_mmq(l.wq_t, D.dim, (int)n, 32, false) && use_mmq(l.wk_t, D.dim, (int)n, 32, false) &&
        use_mmq(l.wv_t, D.dim, (int)n, 32, false)) {
        DmmvSegParams mp = sp;
        mp.base.ident_n = (int)n;
        const int ph = prof_begin(LOOMHIP_KT_QKV, st);
        const bool ok = launch_mmq_seg(mp, st);
        prof_end(ph, st);
        if (ok)
            return true;
    }
    const int ph = prof_begin(LOOMHIP_KT_QKV, st);
    const bool ok = launch_dmmv_seg(w.nt, sp, st);
    prof_end(ph, st);
    return ok;
}

template <bool EXACT>
static void launch_norm_t(int qb, const float *x, int dim, const float *w, float eps, QAct qa,
                          float *normed, size_t n, hipStream_t st) {
    if (qb == 256)
        hipLaunchKernelGGL((norm_quant_kernel<256, EXACT>), dim3(n), dim3(norm_threads(EXACT)), 0, st, x, dim, w, eps, qa,
                           normed);
    else if (qb == 32)
        hipLaunchKernelGGL((norm_quant_kernel<32, EXACT>), dim3(n), dim3(norm_threads(EXACT)), 0, st, x, dim, w, eps, qa,
                           normed);
    else
        hipLaunchKernelGGL((norm_quant_kernel<0, EXACT>), dim3(n), dim3(norm_threads(EXACT)), 0, st, x, dim, w, eps,
                           QAct{}, normed);
    note_launch();
}

static void launch_norm(int qb, const float *x, int dim, const float *w, float eps, QAct qa,
                        float *normed, size_t n, hipStream_t st, bool exact = false) {
    if (exact)
        launch_norm_t<true>(qb, x, dim, w, eps, qa, normed, n, st);
    else
        launch_norm_t<false>(qb, x, dim, w, eps, qa, normed, n, st);
}

// tensor.rmsnorm (core/tensor.zig:9-15) of n rows of dim values with the
// squares summed in index order: the norm the reference's FFN input takes.
int rmsnorm_exact_dev(const float *x, int dim, const float *w, float eps, float *normed, size_t n, hipStream_t st) {
    if (dim <= 0 || dim % 32 || dim > EXACT_NORM_MAX_DIM)
        return fail(LOOMHIP_DECLINED, "rmsnorm: dim %d not served (a multiple of 32 up to %d)", dim,
                    EXACT_NORM_MAX_DIM);
    launch_norm(0, x, dim, w, eps, QAct{}, normed, n, st, true);
    return LOOMHIP_OK;
}

int frame_dims_check(const loomhip_model *m, size_t n) {
    if (!m || n == 0 || n > 256)
        return fail(LOOMHIP_ERR_ARG, "token_frame: bad model or lane count %zu (1..256)", n);
    const size_t dim = m->dim, hd = m->head_dim, qd = m->n_heads * hd;
    if (dim == 0 || dim % 32 || dim > (size_t)EXACT_NORM_MAX_DIM || qd % 32 || (hd != 48 && hd != 64 && hd != 128) ||
        m->n_kv_heads == 0 || m->n_heads % m->n_kv_heads || m->n_heads / m->n_kv_heads > MAX_G ||
        m->rope_dim > hd || m->rope_dim % 2 || m->ctx_len == 0)
        return fail(LOOMHIP_DECLINED, "token_frame: dims not served (dim %zu, head_dim %zu, heads %zu/%zu)",
                    dim, hd, m->n_heads, m->n_kv_heads);
    if (m->numerics != LOOMHIP_NUMERICS_PARITY && m->numerics != LOOMHIP_NUMERICS_FAST)
        return fail(LOOMHIP_ERR_ARG, "token_frame: unknown numerics mode %d", m->numerics);
    if (m->numerics == LOOMHIP_NUMERICS_PARITY && m->ctx_len > (size_t)EXACT_MAX_CTX)
        return fail(LOOMHIP_DECLINED, "token_frame: PARITY attention serves contexts up to %d (ctx_len %zu)",
                    EXACT_MAX_CTX, m->ctx_len);
    return LOOMHIP_OK;
}

int frame_layer_check(const loomhip_model *m, const loomhip_layer &l, size_t li, size_t n, size_t *ffn_max) {
    const size_t dim = m->dim, qd = m->n_heads * m->head_dim;
    const int qb = act_block(l.wq_t);
    if (act_block(l.wk_t) != qb || act_block(l.wv_t) != qb || !dmmv_supported(l.wq_t, (int)dim) ||
        !dmmv_supported(l.wk_t, (int)dim) || !dmmv_supported(l.wv_t, (int)dim) ||
        !dmmv_supported(l.wo_t, (int)qd) || (qb == 256 && dim % 256) || (act_block(l.wo_t) == 256 && qd % 256))
        return fail(LOOMHIP_DECLINED, "token_frame: layer %zu attention types not served", li);
    if (!l.attn_norm || !l.ffn_norm || !l.wq || !l.wk || !l.wv || !l.wo)
        return fail(LOOMHIP_ERR_ARG, "token_frame: layer %zu misses a norm or an attention weight", li);
    if (l.is_moe) {
        if (l.moe.dim != dim)
            return fail(LOOMHIP_ERR_ARG, "token_frame: layer %zu MoE dim %zu != %zu", li, l.moe.dim, dim);
        return moe_frame_check(&l.moe, n);
    }
    const int gq = act_block(l.ffn_gate_t);
    if (l.ffn_gate_t != l.ffn_up_t || !dmmv_supported(l.ffn_gate_t, (int)dim) ||
        !dmmv_supported(l.ffn_down_t, (int)l.ffn) || (gq == 256 && dim % 256) ||
        (act_block(l.ffn_down_t) == 256 && l.ffn % 256) || l.ffn % 32 || l.ffn == 0)
        return fail(LOOMHIP_DECLINED, "token_frame: layer %zu dense FFN types not served", li);
    if (!l.ffn_gate || !l.ffn_up || !l.ffn_down)
        return fail(LOOMHIP_ERR_ARG, "token_frame: layer %zu misses a dense FFN weight", li);
    *ffn_max = l.ffn > *ffn_max ? l.ffn : *ffn_max;
    return LOOMHIP_OK;
}

int frame_check(const loomhip_model *m, size_t n, size_t *ffn_max) {
    if (int rc = frame_dims_check(m, n))
        return rc;
    if (!m->layers || m->vocab == 0)
        return fail(LOOMHIP_ERR_ARG, "token_frame: no layers or no vocabulary");
    const int qb_out = act_block(m->output_t);
    if (!dmmv_supported(m->output_t, (int)m->dim) || (qb_out == 256 && m->dim % 256))
        return fail(LOOMHIP_DECLINED, "token_frame: output type %d not served", m->output_t);
    *ffn_max = 0;
    for (size_t li = 0; li < m->n_layers; li++)
        if (int rc = frame_layer_check(m, m->layers[li], li, n, ffn_max))
            return rc;
    return LOOMHIP_OK;
}

int frame_setup(const loomhip_model *m, size_t n, size_t ffn_max, float scale, int32_t *pos, uint16_t *kc,
                uint16_t *vc, hipStream_t st, FrameCall &c) {
    c.n = n;
    c.st = st;
    c.pos = pos;
    c.kc = kc;
    c.vc = vc;
    c.n_chunks = (int)((m->ctx_len + ATT_TC - 1) / ATT_TC);
    c.parity = m->numerics == LOOMHIP_NUMERICS_PARITY;
    const FrameWs probe = frame_layout(nullptr, n, m, ffn_max, c.n_chunks, c.parity);
    if (int rc = g_frame.reserve(probe.bytes))
        return rc;
    c.w = frame_layout((char *)g_frame.ptr, n, m, ffn_max, c.n_chunks, c.parity);
    c.w.nt = pick_nt((int)n);
    c.w.groups = dense_groups((int)n, c.w.nt, &c.w.n_groups); // built once per lane count, before any capture
    if (!c.w.groups)
        return fail(LOOMHIP_ERR_HIP, "token_frame: group table");
    FrameDims &D = c.D;
    D.dim = (int)m->dim;
    D.hd = (int)m->head_dim;
    D.n_heads = (int)m->n_heads;
    D.n_kv = (int)m->n_kv_heads;
    D.qd = D.n_heads * D.hd;
    D.kvd = D.n_kv * D.hd;
    D.ctx = (int)m->ctx_len;
    D.rope_dim = (int)m->rope_dim;
    D.rope_neox = m->rope_neox;
    D.n_layers = (int)m->n_layers;
    D.vocab = (int)m->vocab;
    D.rope_base = m->rope_base;
    D.eps = m->eps;
    D.scale = scale;
    const int G = D.n_heads / D.n_kv;
    c.att_lds = (size_t)G * D.hd * 4 + (size_t)16 * ATT_TC * 4 + (size_t)ATT_TC * (D.hd + 8) * 2 +
                (size_t)ATT_TC * (D.hd + 2) * 2;
    if (c.att_lds > 64 * 1024)
        return fail(LOOMHIP_DECLINED, "token_frame: attention tile exceeds LDS (%zu B)", c.att_lds);
    // the direct form keeps p and the values only
    c.att_lds_direct = (size_t)16 * ATT_TC_DIRECT * 4 + (size_t)ATT_TC_DIRECT * (D.hd + 2) * 2;
    c.cmb_lds = (4 * 256 + (size_t)CMB_NH * c.n_chunks) * 4;
    if (c.cmb_lds > 64 * 1024)
        return fail(LOOMHIP_DECLINED, "token_frame: context %zu exceeds the merge's LDS", m->ctx_len);
    c.rope_cs = m->rope_cs ? m->rope_cs : rope_table(D.ctx, D.rope_dim, D.rope_base);
    if (!c.rope_cs)
        return fail(LOOMHIP_ERR_HIP, "token_frame: rope table");
    return LOOMHIP_OK;
}

int frame_layer(const FrameCall &c, const loomhip_layer &l, size_t li, uint32_t *ids, const NextNorm *next,
                bool *next_done, bool prenormed) {
    const FrameDims &D = c.D;
    const FrameWs &w = c.w;
    const size_t n = c.n;
    const bool parity = c.parity;
    hipStream_t st = c.st;
    // attention block (llama.zig:1127-1201)
    // layer 0 normalises the embedding row: exact sum in either mode; one
    // lane in PARITY: the q/k/v launch normalises its input itself
    bool fused = false;
    if (prenormed) { // the previous layer's combine left the normalised, quantized row in qa_dim
        if (!frame_qkv(l, D, w, n, st))
            return fail(LOOMHIP_ERR_ARG, "token_frame: q/k/v matvec declined");
    } else if (!(parity && frame_qkv(l, D, w, n, st, &fused))) {
        launch_norm(act_block(l.wq_t), w.x, D.dim, l.attn_norm, D.eps, w.qa_dim, nullptr, n, st, parity || li == 0);
        if (!frame_qkv(l, D, w, n, st))
            return fail(LOOMHIP_ERR_ARG, "token_frame: q/k/v matvec declined");
    }
    // few lanes: norm/rope/append inside the attention launch; more lanes:
    // once per head in their own launch (the attention is then
    // throughput-bound and the fused prologue would repeat per chunk)
    const bool fuse_rope = n <= ATT_FUSE_MAX_LANES;
    // FAST with rope done apart and an MFMA head size: the attention takes
    // its query operands pre-split and its keys straight from HBM
    const bool direct = !parity && !fuse_rope && D.hd % 32 == 0;
    uint16_t *qsplit = direct ? w.qsplit : nullptr;
    if (!fuse_rope) {
        hipLaunchKernelGGL(qk_rope_kernel, dim3(D.n_heads + D.n_kv, n), dim3(64), 0, st, D, w.q, w.k, w.v,
                           l.q_norm, l.k_norm, c.pos, (int)li, c.rope_cs, w.qrot, qsplit, c.kc, c.vc);
        note_launch();
    }
    const float *qin = fuse_rope ? w.q : w.qrot;
    if (parity) {
        // the reference's own order over the whole context: scores, softmax, P.V
        // few lanes: P.V quantizes wo's input itself
        const bool qfuse = attn_exact_quant_fusable(D, n);
        if (!launch_attn_exact(D, qin, w.k, w.v, l.q_norm, l.k_norm, c.rope_cs, c.kc, c.vc, c.pos, (int)li,
                               fuse_rope, w.S, w.s_stride, w.att, n, qfuse ? l.wo_t : -1, w.qa_att, st))
            return fail(LOOMHIP_ERR_ARG, "token_frame: exact attention declined");
        if (!qfuse)
            launch_quant_act(l.wo_t, w.att, D.qd, D.qd, (int)n, w.qa_att, st);
    } else {
        const int ph = prof_begin(LOOMHIP_KT_ATTN, st);
        const dim3 agrid(c.n_chunks, D.n_kv, n);
        // records of the merge: chunks of ATT_TC positions, ATT_TC_DIRECT direct
        const int span = direct ? ATT_TC_DIRECT : ATT_TC;
        const int n_rec = (D.ctx + span - 1) / span;
        if (direct) {
            const dim3 dgrid(n_rec, D.n_kv, n);
            if (D.hd == 128)
                hipLaunchKernelGGL((attn_direct_kernel<128, ATT_TC_DIRECT>), dgrid, dim3(64 * ATT_WAVES),
                                   c.att_lds_direct, st, D, c.kc, c.vc, c.pos, (int)li, n_rec, qsplit, w.part);
            else
                hipLaunchKernelGGL((attn_direct_kernel<64, ATT_TC_DIRECT>), dgrid, dim3(64 * ATT_WAVES),
                                   c.att_lds_direct, st, D, c.kc, c.vc, c.pos, (int)li, n_rec, qsplit, w.part);
        } else if (D.hd == 128)
            hipLaunchKernelGGL(attn_partial_kernel<128>, agrid, dim3(64 * ATT_WAVES), c.att_lds, st, D, qin, w.k,
                               w.v, l.q_norm, l.k_norm, c.rope_cs, c.kc, c.vc, c.pos, (int)li, c.n_chunks, 1,
                               fuse_rope ? 1 : 0, w.part);
        else if (D.hd == 64)
            hipLaunchKernelGGL(attn_partial_kernel<64>, agrid, dim3(64 * ATT_WAVES), c.att_lds, st, D, qin, w.k,
                               w.v, l.q_norm, l.k_norm, c.rope_cs, c.kc, c.vc, c.pos, (int)li, c.n_chunks, 1,
                               fuse_rope ? 1 : 0, w.part);
        else
            hipLaunchKernelGGL(attn_partial_kernel<48>, agrid, dim3(64 * ATT_WAVES), c.att_lds, st, D, qin, w.k,
                               w.v, l.q_norm, l.k_norm, c.rope_cs, c.kc, c.vc, c.pos, (int)li, c.n_chunks, 1,
                               fuse_rope ? 1 : 0, w.part);
        prof_end(ph, st);
        note_launch();
        if (act_block(l.wo_t) == 256)
            hipLaunchKernelGGL(attn_combine_kernel<256>, dim3((D.qd + 255) / 256, n), dim3(1024), c.cmb_lds, st,
                               D, w.part, c.pos, n_rec, span, direct ? 1 : 0, w.qa_att);
        else
            hipLaunchKernelGGL(attn_combine_kernel<32>, dim3((D.qd + 255) / 256, n), dim3(1024), c.cmb_lds, st,
                               D, w.part, c.pos, n_rec, span, direct ? 1 : 0, w.qa_att);
        note_launch();
    }
    if (!frame_matvec(l.wo_t, l.wo, D.dim, D.qd, w, n, w.qa_att, w.x, 1, st, LOOMHIP_KT_WO, true, 16))
        return fail(LOOMHIP_ERR_ARG, "token_frame: wo matvec declined");
    // FFN block (llama.zig:1203-1224)
    if (l.is_moe) {
        const int combine = n == 1 ? LOOMHIP_COMBINE_SELECTION_ADD : LOOMHIP_COMBINE_EXPERT_ASC;
        if (moe_decode_fusable(&l.moe, n, parity))
            // the router launch applies the rmsnorm itself (PARITY: one
            // lane, the squares summed in order in every work group)
            return moe_layer_fused_norm(&l.moe, w.x, l.ffn_norm, D.eps, n, combine, w.x, ids, parity, st);
        launch_norm(0, w.x, D.dim, l.ffn_norm, D.eps, QAct{}, w.normed, n, st, parity);
        // the batched combine also forms the next rmsnorm of x (next)
        return moe_layer_next_norm(&l.moe, w.normed, n, combine, w.x, ids, next, next_done, st);
    }
    launch_norm(act_block(l.ffn_gate_t), w.x, D.dim, l.ffn_norm, D.eps, w.qa_dim, nullptr, n, st, parity);
    DmmvParams p{};
    p.w = (const uint8_t *)l.ffn_gate;
    p.w2 = (const uint8_t *)l.ffn_up;
    p.rows = (int)l.ffn;
    p.cols = D.dim;
    p.xq = w.qa_dim.q;
    p.xd = w.qa_dim.d;
    p.xs = w.qa_dim.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = w.groups;
    p.n_groups = w.n_groups;
    p.out = w.act;
    p.out_stride = (int)l.ffn;
    p.rpw = dmmv_pick_rpw(l.ffn_gate_t, D.dim, (int)l.ffn, w.n_groups, w.nt, true);
    if (!launch_dmmv(l.ffn_gate_t, w.nt, true, p, st))
        return fail(LOOMHIP_ERR_ARG, "token_frame: gate/up matvec declined");
    launch_quant_act(l.ffn_down_t, w.act, (int)l.ffn, (int)l.ffn, (int)n, w.qa_ffn, st);
    if (!frame_matvec(l.ffn_down_t, l.ffn_down, D.dim, (int)l.ffn, w, n, w.qa_ffn, w.x, 1, st))
        return fail(LOOMHIP_ERR_ARG, "token_frame: down matvec declined");
    return LOOMHIP_OK;
}

int frame_head(const FrameCall &c, const loomhip_model *m, float *logits, bool prenormed) {
    const FrameDims &D = c.D;
    if (!prenormed)
        launch_norm(act_block(m->output_t), c.w.x, D.dim, m->out_norm, D.eps, c.w.qa_dim, nullptr, c.n, c.st,
                    c.parity);
    if (!frame_matvec(m->output_t, m->output, D.vocab, D.dim, c.w, c.n, c.w.qa_dim, logits, 0, c.st,
                      LOOMHIP_KT_HEAD, true))
        return fail(LOOMHIP_ERR_ARG, "token_frame: output matvec declined");
    return LOOMHIP_OK;
}

} // namespace lh

using namespace lh;

extern "C" {

int loomhip_frame_check(const loomhip_model *m, size_t n) {
    if (int rc = require_ready())
        return rc;
    size_t ffn_max = 0;
    return frame_check(m, n, &ffn_max);
}

int loomhip_token_frame_dev(const loomhip_model *m, const uint32_t *tokens, int32_t *pos, size_t n,
                            uint16_t *k_cache, uint16_t *v_cache, float *logits, uint32_t *next,
                            void *stream) {
    if (int rc = require_ready())
        return rc;
    if (!tokens || !pos || !k_cache || !v_cache || !logits)
        return fail(LOOMHIP_ERR_ARG, "token_frame: null argument");
    size_t ffn_max = 0;
    if (int rc = frame_check(m, n, &ffn_max))
        return rc;
    FrameCall c;
    if (int rc = frame_setup(m, n, ffn_max, 1.0f / sqrtf((float)m->head_dim), pos, k_cache, v_cache,
                             stream_of(stream), c)) // llama.zig attn scale
        return rc;
    hipLaunchKernelGGL(embed_kernel, dim3((c.D.dim + 255) / 256, n), dim3(256), 0, c.st, m->embed_t,
                       (const uint8_t *)m->embed, c.D.vocab, c.D.dim, tokens, c.w.x);
    note_launch();
    // PARITY: each layer's batched MoE combine may also form the exact rmsnorm
    // its residual row meets next (the next layer's attention norm, the last
    // layer's the output norm), which that consumer then skips
    bool pre = false;
    for (size_t li = 0; li < m->n_layers; li++) {
        const loomhip_layer &l = m->layers[li];
        uint32_t *ids = m->ids_out && l.is_moe ? m->ids_out + li * n * l.moe.n_used : nullptr;
        const NextNorm nx = li + 1 < m->n_layers
                                ? NextNorm{m->layers[li + 1].attn_norm, c.D.eps, act_block(m->layers[li + 1].wq_t),
                                           c.w.qa_dim, c.parity}
                                : NextNorm{m->out_norm, c.D.eps, act_block(m->output_t), c.w.qa_dim, c.parity};
        bool done = false;
        if (int rc = frame_layer(c, l, li, ids, c.parity ? &nx : nullptr, &done, pre))
            return rc;
        pre = done;
    }
    // head (llama.zig:1225-1227) and the greedy pick
    if (int rc = frame_head(c, m, logits, pre))
        return rc;
    hipLaunchKernelGGL(argmax_part_kernel, dim3(ARGMAX_SLICES, n), dim3(256), 0, c.st, logits, c.D.vocab,
                       c.w.amax_v, c.w.amax_i);
    hipLaunchKernelGGL(argmax_merge_kernel, dim3(n), dim3(64), 0, c.st, c.w.amax_v, c.w.amax_i, next, pos);
    note_launch();
    note_launch();
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return hip_fail(e, "token_frame launch");
    return LOOMHIP_OK;
}

} // extern "C"
