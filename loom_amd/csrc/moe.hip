// moe.hip -- router GEMV, routing, token->expert bucketing and the gated
// combine of the MoE layer (src/gguf/moe.zig:106-158; src/gguf/llama.zig
// moeLayer 1262-1272, moeRun 1307-1419, moeBatchUnion 1828-1903).
#include "kernels.hpp"

namespace lh {

// ---- router GEMV in the reference's dotF32 order --------------------------
// dotF32 (src/gguf/ggml.zig:198-217) keeps 4 x 8 f32 accumulators: lane
// L = 8v + l of a half-wave accumulates a[32t + L] * b[32t + L] over t in
// sequence; then per l, ((acc[0][l] + acc[1][l]) + acc[2][l]) + acc[3][l];
// then the eight lanes in order; then the scalar tail.  A half-wave per
// (row, 4 tokens) reproduces that exactly.
constexpr int RG_TOK = 4;

__global__ __launch_bounds__(256) void router_gemv_kernel(const float *__restrict__ w,
                                                          const float *__restrict__ bias,
                                                          const float *__restrict__ x, int n_expert,
                                                          int dim, int n, float *__restrict__ logits) {
    __shared__ float part[8][RG_TOK][32];
    const int hw = threadIdx.x >> 5, L = threadIdx.x & 31;
    const int e = blockIdx.x * 8 + hw;
    const int t0 = blockIdx.y * RG_TOK;
    const int ec = e < n_expert ? e : n_expert - 1;
    const float *row = w + (size_t)ec * dim;
    float acc[RG_TOK];
#pragma unroll
    for (int k = 0; k < RG_TOK; k++)
        acc[k] = 0.0f;
    const int main_end = dim / 32 * 32;
    for (int i = 0; i < main_end; i += 32) {
        const float a = row[i + L];
#pragma unroll
        for (int k = 0; k < RG_TOK; k++) {
            const int t = t0 + k < n ? t0 + k : n - 1;
            const float p = a * x[(size_t)t * dim + i + L];
            acc[k] = acc[k] + p;
        }
    }
    // leftover whole 8-chunks go to accumulator 0 (lanes 0..7)
    for (int i = main_end; i + 8 <= dim; i += 8) {
        if (L < 8) {
            const float a = row[i + L];
#pragma unroll
            for (int k = 0; k < RG_TOK; k++) {
                const int t = t0 + k < n ? t0 + k : n - 1;
                const float p = a * x[(size_t)t * dim + i + L];
                acc[k] = acc[k] + p;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < RG_TOK; k++)
        part[hw][k][L] = acc[k];
    __syncthreads();
    if (L < RG_TOK && e < n_expert && t0 + L < n) {
        const int k = L, t = t0 + k;
        float s = -0.0f;
        for (int l = 0; l < 8; l++) {
            const float lane = ((part[hw][k][l] + part[hw][k][8 + l]) + part[hw][k][16 + l]) +
                               part[hw][k][24 + l];
            s = s + lane;
        }
        for (int i = dim / 8 * 8; i < dim; i++) {
            const float p = row[i] * x[(size_t)t * dim + i];
            s = s + p;
        }
        if (bias)
            s = s + bias[e];
        logits[(size_t)t * n_expert + e] = s;
    }
}

void launch_router_gemv(const float *w, const float *bias, const float *x, int n_expert, int dim,
                        int n, float *logits, hipStream_t st) {
    dim3 grid((n_expert + 7) / 8, (n + RG_TOK - 1) / RG_TOK);
    hipLaunchKernelGGL(router_gemv_kernel, grid, dim3(256), 0, st, w, bias, x, n_expert, dim, n,
                       logits);
    note_launch();
}

// ---- route: one wave per token ------------------------------------------------
constexpr int MAX_E = 256, MAX_K = 16;

__global__ __launch_bounds__(64) void route_kernel(const float *__restrict__ logits,
                                                   const float *__restrict__ sel_bias, int n_expert,
                                                   int n_used, int gating, int weights_norm,
                                                   float weights_scale, uint32_t *__restrict__ ids,
                                                   float *__restrict__ gates) {
    __shared__ float sc[MAX_E];
    __shared__ float gsel[MAX_K];
    __shared__ int isel[MAX_K];
    const int t = blockIdx.x, lane = threadIdx.x;
    const float *lg = logits + (size_t)t * n_expert;
    // scores (moe.zig:110-120)
    if (gating == 2) { // sigmoid
        for (int e = lane; e < n_expert; e += 64)
            sc[e] = 1.0f / (1.0f + expf(-lg[e]));
    } else if (gating == 3) { // softmax_topk: raw logits
        for (int e = lane; e < n_expert; e += 64)
            sc[e] = lg[e];
    } else { // softmax (tensor.zig:18-28): max, exp, sequential sum, * (1/sum)
        float m = -INFINITY;
        for (int e = lane; e < n_expert; e += 64)
            m = fmaxf(m, lg[e]);
        m = wave_max(m);
        for (int e = lane; e < n_expert; e += 64)
            sc[e] = expf(lg[e] - m);
        __syncthreads();
        float inv = 0.0f;
        if (lane == 0) {
            float sum = 0.0f;
            for (int e = 0; e < n_expert; e++)
                sum = sum + sc[e];
            inv = 1.0f / sum;
        }
        inv = __shfl(inv, 0, 64);
        __syncthreads();
        for (int e = lane; e < n_expert; e += 64)
            sc[e] = sc[e] * inv;
    }
    __syncthreads();
    // k rounds of argmax over unused experts, strict '>' (lowest index wins
    // ties), selection on scores + bias, gates from unbiased scores.
    float ch[MAX_E / 64];
    bool used[MAX_E / 64];
#pragma unroll
    for (int i = 0; i < MAX_E / 64; i++) {
        const int e = lane + 64 * i;
        ch[i] = e < n_expert ? (sel_bias ? sc[e] + sel_bias[e] : sc[e]) : -INFINITY;
        used[i] = e >= n_expert;
    }
    for (int s = 0; s < n_used; s++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < MAX_E / 64; i++)
            if (!used[i] && ch[i] > bv) {
                bv = ch[i];
                bi = lane + 64 * i;
            }
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        const int best = (bi == 0x7fffffff) ? 0 : bi; // nothing beat -inf: index 0
#pragma unroll
        for (int i = 0; i < MAX_E / 64; i++)
            if (lane + 64 * i == best)
                used[i] = true;
        if (lane == 0) {
            isel[s] = best;
            gsel[s] = sc[best];
        }
    }
    __syncthreads();
    if (lane == 0) {
        float g[MAX_K];
        for (int s = 0; s < n_used; s++)
            g[s] = gsel[s];
        if (gating == 3) { // softmax over the selected k
            float m = -INFINITY;
            for (int s = 0; s < n_used; s++)
                m = fmaxf(m, g[s]);
            float sum = 0.0f;
            for (int s = 0; s < n_used; s++) {
                g[s] = expf(g[s] - m);
                sum = sum + g[s];
            }
            const float inv = 1.0f / sum;
            for (int s = 0; s < n_used; s++)
                g[s] = g[s] * inv;
        }
        if (weights_norm) {
            float sum = 0.0f;
            for (int s = 0; s < n_used; s++)
                sum = sum + g[s];
            const float denom = fmaxf(sum, 6.103515625e-5f);
            for (int s = 0; s < n_used; s++)
                g[s] = g[s] / denom;
        }
        if (weights_scale != 1.0f)
            for (int s = 0; s < n_used; s++)
                g[s] = g[s] * weights_scale;
        for (int s = 0; s < n_used; s++) {
            ids[(size_t)t * n_used + s] = (uint32_t)isel[s];
            gates[(size_t)t * n_used + s] = g[s];
        }
    }
}

void launch_route(const float *logits, const float *sel_bias, int n_expert, int n_used, int gating,
                  int weights_norm, float weights_scale, int n, uint32_t *ids, float *gates,
                  hipStream_t st) {
    hipLaunchKernelGGL(route_kernel, dim3(n), dim3(64), 0, st, logits, sel_bias, n_expert, n_used,
                       gating, weights_norm, weights_scale, ids, gates);
    note_launch();
}

// ---- bucketing: one work group --------------------------------------------------
// Per expert a token bitmask (order-free atomicOr); an expert's pairs are
// ranked by token index via popcounts, so the pair order is (expert, token)
// and deterministic.
constexpr int BK_MAX_TOK = 256;

int moe_max_groups(int n, int k, int n_expert, int nt) {
    const int P = n * k;
    const int bound = P / nt + (P < n_expert ? P : n_expert);
    return bound < P ? bound : P;
}

__global__ __launch_bounds__(256) void bucket_kernel(const uint32_t *__restrict__ ids, int n, int k,
                                                     int n_expert, int nt, MoeBuckets b) {
    __shared__ uint32_t mask[MAX_E][BK_MAX_TOK / 32];
    __shared__ int cnt[MAX_E], off[MAX_E], goff[MAX_E];
    const int tid = threadIdx.x;
    const int W = (n + 31) / 32;
    for (int i = tid; i < n_expert * W; i += blockDim.x)
        mask[i / W][i % W] = 0;
    __syncthreads();
    const int P = n * k;
    for (int p = tid; p < P; p += blockDim.x) {
        const int t = p / k, e = (int)ids[p];
        atomicOr(&mask[e][t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    for (int e = tid; e < n_expert; e += blockDim.x) {
        int c = 0;
        for (int w = 0; w < W; w++)
            c += __popc(mask[e][w]);
        cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) { // exclusive scans over <= 256 experts
        int o = 0, go = 0;
        for (int e = 0; e < n_expert; e++) {
            off[e] = o;
            goff[e] = go;
            o += cnt[e];
            go += (cnt[e] + nt - 1) / nt;
        }
        *b.n_groups = go;
    }
    __syncthreads();
    for (int p = tid; p < P; p += blockDim.x) {
        const int t = p / k, e = (int)ids[p];
        int rank = 0;
        for (int w = 0; w < (t >> 5); w++)
            rank += __popc(mask[e][w]);
        rank += __popc(mask[e][t >> 5] & ((1u << (t & 31)) - 1u));
        const int pos = off[e] + rank;
        b.pair_tok[pos] = t;
        b.pair_of[p] = pos;
        b.iota[p] = p;
    }
    for (int e = tid; e < n_expert; e += blockDim.x) {
        const int c = cnt[e];
        for (int gi = 0; gi * nt < c; gi++) {
            DmmvGroup g;
            g.plane = e;
            g.first = off[e] + gi * nt;
            g.n = (c - gi * nt) < nt ? (c - gi * nt) : nt;
            b.groups[goff[e] + gi] = g;
        }
    }
}

void launch_bucket(const uint32_t *ids, int n, int k, int n_expert, int nt, MoeBuckets b,
                   hipStream_t st) {
    hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(256), 0, st, ids, n, k, n_expert, nt, b);
    note_launch();
}

// ---- combine ----------------------------------------------------------------------
// mode 0 (moeRun): out = ((0 + g0*y0) + g1*y1) + ... in selection order.
// mode 1 (moeBatchUnion): out += g*y per expert in ascending expert id.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y,
                                                      const float *__restrict__ gates,
                                                      const uint32_t *__restrict__ ids,
                                                      const int *__restrict__ pair_of, int k,
                                                      int dim, int mode, float *__restrict__ out) {
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim)
        return;
    const size_t base = (size_t)t * k;
    if (mode == 0) {
        float acc = 0.0f;
        for (int s = 0; s < k; s++) {
            const float p = gates[base + s] * y[(size_t)pair_of[base + s] * dim + i];
            acc = acc + p;
        }
        out[(size_t)t * dim + i] = acc;
    } else {
        float acc = out[(size_t)t * dim + i];
        int prev = -1;
        for (int step = 0; step < k; step++) {
            int bs = -1, be = 0x7fffffff;
            for (int s = 0; s < k; s++) {
                const int e = (int)ids[base + s];
                if (e > prev && e < be) {
                    be = e;
                    bs = s;
                }
            }
            if (bs < 0)
                break;
            const float p = gates[base + bs] * y[(size_t)pair_of[base + bs] * dim + i];
            acc = acc + p;
            prev = be;
        }
        out[(size_t)t * dim + i] = acc;
    }
}

void launch_combine(const float *y, const float *gates, const uint32_t *ids, const int *pair_of,
                    int n, int k, int dim, int mode, float *out, hipStream_t st) {
    hipLaunchKernelGGL(combine_kernel, dim3((dim + 255) / 256, n), dim3(256), 0, st, y, gates, ids,
                       pair_of, k, dim, mode, out);
    note_launch();
}

} // namespace lh
