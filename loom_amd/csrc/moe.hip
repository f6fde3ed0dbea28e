// moe.hip -- the gate kernel of the MoE layer: router GEMV, routing,
// token->expert bucketing and int8 quantization of the layer input in one
// launch (src/gguf/moe.zig:106-158; src/gguf/llama.zig moeLayer 1262-1272,
// moeRun 1307-1419, moeBatchUnion 1828-1903).
//
// Work split.  Workgroups [0, gemv_wgs) each own up to GT_ROWS router rows
// (one half-wave per row) for one chunk of GT_TOK tokens; workgroups
// [gemv_wgs, +quant_wgs) quantize the input for the expert kernels.  The
// last workgroup to finish a token chunk routes that chunk (one wave per
// token), and the last router of all chunks buckets every (token, slot) pair
// by expert.  "Last" is decided by self-resetting completion counters with
// agent-scope fences on both sides; nothing ever waits on another workgroup.
#include "device.hpp"
#include "frame.hpp"

namespace lh {

// ---- the gate kernel ------------------------------------------------------------

constexpr int GT_THREADS = 256;
constexpr int GT_ROWS = GT_THREADS / 32; // router rows per workgroup (a half-wave each)
constexpr int GT_TOK = 2;                // tokens per chunk = tokens per half-wave pass
constexpr int GT_UNROLL = 64; // router elements in flight per lane (dim 2048: one chunk)
constexpr int GT_COLS = 32 * GT_UNROLL; // columns per staged chunk
static_assert(GT_TOK == 2 || GT_TOK == 4, "a staged column's tokens are one float2 or float4");
static_assert(SYNC_GATE_CHUNK + MAX_TOK / GT_TOK <= SYNC_GATE_FINAL, "a completion counter per token chunk");

// A staged column's GT_TOK token values, one 8- or 16-byte LDS read.
__device__ __forceinline__ void xs_tokens(const float *src, float (&o)[GT_TOK]) {
    if constexpr (GT_TOK == 4) {
        const float4 v = *(const float4 *)src;
        o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
    } else {
        const float2 v = *(const float2 *)src;
        o[0] = v.x, o[1] = v.y;
    }
}

// Router GEMV for up to GT_TOK tokens in dotF32 order (src/gguf/ggml.zig:
// 198-217): lane L of a half-wave accumulates row[32i + L] * x[32i + L] over
// i in sequence (acc0..acc3 x 8 lanes), then per l: ((acc0 + acc1) + acc2) +
// acc3, the eight lanes in order, and the scalar tail.  Every half-wave owns
// one row (e < n_expert: valid); the whole work group calls this.  A chunk of
// GT_COLS columns is processed at a time: the half-wave's row loads (64 per
// lane) are issued together, and the tokens' matching x columns are staged
// in LDS by the whole work group as [GT_COLS][GT_TOK] (a column's token
// values in one read).
__device__ void router_rows(const GateParams &p, int e, bool valid, int t0, int nt, int hw, int L,
                            float (*part)[GT_TOK][32], float *xs) {
    const int dim = p.dim;
    const float *row = p.router + (size_t)(valid ? e : 0) * dim;
    float acc[GT_TOK];
#pragma unroll
    for (int k = 0; k < GT_TOK; k++)
        acc[k] = 0.0f;
    const int main_end = dim / 32 * 32;
    for (int c0 = 0; c0 < main_end; c0 += GT_COLS) {
        const int ccols = (main_end - c0) < GT_COLS ? (main_end - c0) : GT_COLS;
        const int cnt = ccols / 32;
        // the tokens' x columns are requested first, then the row, so one
        // round trip covers both; the barriers below wait on LDS only.
        // Thread item q: the column quad 4 (tid + q GT_THREADS) of every token.
        constexpr int XPT = GT_COLS / 4 / GT_THREADS;
        float4 xv[XPT][GT_TOK];
#pragma unroll
        for (int q = 0; q < XPT; q++) {
            const int col = 4 * ((int)threadIdx.x + q * GT_THREADS);
#pragma unroll
            for (int k = 0; k < GT_TOK; k++)
                xv[q][k] = k < nt && col < ccols ? *(const float4 *)(p.x + (size_t)(t0 + k) * dim + c0 + col)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // unconditional loads (steps past cnt re-read the chunk's last step,
        // their products are never added), so they all go out together
        float wv[GT_UNROLL];
#pragma unroll
        for (int u = 0; u < GT_UNROLL; u++)
            wv[u] = row[c0 + 32 * min(u, cnt - 1) + L];
        if (c0 > 0)
            lds_barrier(); // the previous chunk's readers are done with xs
#pragma unroll
        for (int q = 0; q < XPT; q++) {
            const int col = 4 * ((int)threadIdx.x + q * GT_THREADS);
            if (col < ccols) {
#pragma unroll
                for (int k = 0; k < GT_TOK; k++) {
                    xs[GT_TOK * (col + 0) + k] = xv[q][k].x;
                    xs[GT_TOK * (col + 1) + k] = xv[q][k].y;
                    xs[GT_TOK * (col + 2) + k] = xv[q][k].z;
                    xs[GT_TOK * (col + 3) + k] = xv[q][k].w;
                }
            }
        }
        lds_barrier();
        // tokens past nt compute on zeros and are not stored.  A full
        // chunk has no per-step guard, so its LDS reads issue back to back
        // (a guard per step compiles to a branch around each read).
        if (cnt == GT_UNROLL) {
            // tokens innermost: GT_TOK independent sums, each still in
            // column order
#pragma unroll
            for (int u = 0; u < GT_UNROLL; u++) {
                float xk[GT_TOK];
                xs_tokens(xs + GT_TOK * (32 * u + L), xk);
#pragma unroll
                for (int k = 0; k < GT_TOK; k++) {
                    const float pr = wv[u] * xk[k];
                    acc[k] = acc[k] + pr;
                }
            }
        } else {
            // steps past cnt add +0 (acc starts at +0 and a sum of products
            // is never -0)
#pragma unroll
            for (int k = 0; k < GT_TOK; k++) {
#pragma unroll
                for (int u = 0; u < GT_UNROLL; u++) {
                    const float xv = xs[GT_TOK * (32 * min(u, cnt - 1) + L) + k];
                    const float pr = u < cnt ? wv[u] * xv : 0.0f;
                    acc[k] = acc[k] + pr;
                }
            }
        }
    }
    if (!valid)
        return;
    int i = main_end;
    // leftover whole 8-chunks go to accumulator 0 (lanes 0..7)
    for (; i + 8 <= dim; i += 8) {
        if (L < 8) {
            const float a = row[i + L];
#pragma unroll
            for (int k = 0; k < GT_TOK; k++)
                if (k < nt) {
                    const float pr = a * p.x[(size_t)(t0 + k) * dim + i + L];
                    acc[k] = acc[k] + pr;
                }
        }
    }
#pragma unroll
    for (int k = 0; k < GT_TOK; k++)
        part[hw][k][L] = acc[k];
    // the reduction below reads only this half-wave's lanes
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    if (L < nt) {
        const int k = L, t = t0 + k;
        float s = -0.0f;
        for (int l = 0; l < 8; l++) {
            const float lane = ((part[hw][k][l] + part[hw][k][8 + l]) + part[hw][k][16 + l]) +
                               part[hw][k][24 + l];
            s = s + lane;
        }
        for (int j = dim / 8 * 8; j < dim; j++) {
            const float pr = row[j] * p.x[(size_t)t * dim + j];
            s = s + pr;
        }
        if (p.router_bias)
            s = s + p.router_bias[e];
        float *dst = p.logits + (size_t)t * p.n_expert + e;
        if (p.chain)
            st_dev(dst, s); // read by the chunk's router in this launch
        else
            *dst = s;
    }
}

// Route one token with one wave and publish ids (read by the bucketing work
// group of this launch) and gates.  The logits are read with device-coherent
// loads either way: written by this launch's other work groups, or by an
// earlier launch (where such a load is merely a plain one).
__device__ __forceinline__ void route_token_wave(const GateParams &p, int t, RouteLds<1> &L) {
    const int lane = threadIdx.x & 63;
    const int E = p.n_expert, K = p.k;
    const float *lg = (p.logits_in ? p.logits_in : p.logits) + (size_t)t * E;
    route_rank<1, true>(lg, p.sel_bias, E, K, p.gating, L);
    bool redo;
    float g = route_finish<1>(L, E, K, p.gating, route_is_exact(p.gating, p.sel_bias),
                              p.weights_norm, p.weights_scale, redo);
    if (redo) {
        route_exact_wave<1, true>(lg, p.sel_bias, E, K, p.gating, L);
        g = route_finish<1>(L, E, K, p.gating, true, p.weights_norm, p.weights_scale, redo);
    }
    if (lane < K) {
        st_dev(p.ids + (size_t)t * K + lane, (uint32_t)L.id[lane]); // read by the bucketing work group
        p.gates[(size_t)t * K + lane] = g;
    }
}

// Exclusive block scan of one int per thread (GT_THREADS threads).
__device__ int block_excl_scan(int v, int *total) {
    __shared__ int wsum[GT_THREADS / 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(inc, o, 64);
        if (lane >= o)
            inc += y;
    }
    if (lane == 63)
        wsum[w] = inc;
    __syncthreads();
    int base = 0, tot = 0;
    for (int i = 0; i < GT_THREADS / 64; i++) {
        if (i < w)
            base += wsum[i];
        tot += wsum[i];
    }
    __syncthreads();
    *total = tot;
    return base + inc - v;
}

// Token -> expert bucketing by the whole workgroup: pairs sorted by
// (expert, token), groups of at most nt pairs per expert, pair_of[t][s] =
// pair index of token t slot s.  Per expert a token bitmask (order-free
// atomicOr) ranks an expert's pairs by token index via popcounts, so the
// order is deterministic.
__device__ void bucket_block(const GateParams &p) {
    __shared__ uint32_t mask[MAX_E][MAX_TOK / 32];
    __shared__ int off[MAX_E], goff[MAX_E], cnt[MAX_E];
    __shared__ uint8_t eid[MAX_TOK * MAX_K]; // each pair's expert, read from ids once
    const int tid = threadIdx.x, n = p.n, K = p.k, E = p.n_expert, nt = p.nt;
    const int W = (n + 31) / 32;
    for (int i = tid; i < E * W; i += GT_THREADS)
        mask[i / W][i % W] = 0;
    __syncthreads();
    const int P = n * K;
    for (int q = tid; q < P; q += GT_THREADS) {
        const int t = q / K, e = min((int)ld_dev(p.ids + q), E - 1);
        eid[q] = (uint8_t)e; // E <= MAX_E = 256
        atomicOr(&mask[e][t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    int c = 0;
    if (tid < E)
        for (int w = 0; w < W; w++)
            c += __popc(mask[tid][w]);
    int tot = 0, gtot = 0;
    const int o = block_excl_scan(c, &tot);
    const int ng = (c + nt - 1) / nt;
    const int go = block_excl_scan(ng, &gtot);
    if (tid < E) {
        off[tid] = o;
        goff[tid] = go;
        cnt[tid] = c;
    }
    if (tid == 0)
        *p.b.n_groups = gtot;
    __syncthreads();
    for (int q = tid; q < P; q += GT_THREADS) {
        const int t = q / K, e = eid[q];
        int rank = 0;
        for (int w = 0; w < (t >> 5); w++)
            rank += __popc(mask[e][w]);
        rank += __popc(mask[e][t >> 5] & ((1u << (t & 31)) - 1u));
        const int pos = off[e] + rank;
        p.b.pair_tok[pos] = t;
        p.b.pair_of[q] = pos;
        p.b.iota[q] = q;
        if (p.b.group_src) {
            // each group's tokens in pair order, the group's last one repeated
            // to nt (read by the expert kernels at the group's index)
            int *row = p.b.group_src + (size_t)(goff[e] + rank / nt) * nt;
            const int i0 = rank % nt;
            const int i1 = rank == cnt[e] - 1 ? nt : i0 + 1;
            for (int i = i0; i < i1; i++)
                row[i] = t;
        }
    }
    if (tid < E)
        for (int gi = 0; gi * nt < c; gi++) {
            DmmvGroup g;
            g.plane = tid;
            g.first = o + gi * nt;
            g.n = (c - gi * nt) < nt ? (c - gi * nt) : nt;
            p.b.groups[go + gi] = g;
        }
}

__global__ __launch_bounds__(GT_THREADS) void moe_gate_kernel(GateParams p) {
    __shared__ float part[GT_ROWS][GT_TOK][32];
    __shared__ RouteLds<1> sc[GT_THREADS / 64];
    __shared__ __align__(16) float xs[GT_TOK * GT_COLS];
    const int bid = blockIdx.x;
    const int wave = threadIdx.x >> 6;

    if (bid >= p.gemv_wgs) {
        // input quantization for the expert kernels: one item per wave
        const int per_vec = quant_items(p.qt, p.dim);
        const int item = (bid - p.gemv_wgs) * (GT_THREADS / 64) + wave;
        if (item < per_vec * p.n) {
            const int v = item / per_vec, it = item % per_vec;
            quant_item_wave(p.qt, p.x + (size_t)v * p.dim, p.dim, v, it, p.qx);
        }
        if (p.chain && last_arrival(p.sync + SYNC_GATE_FINAL, p.n_chunks + p.quant_wgs) &&
            p.b.n_groups)
            bucket_block(p);
        return;
    }

    const int chunk = bid / p.wgs_per_chunk, sub = bid % p.wgs_per_chunk;
    const int t0 = chunk * GT_TOK;
    const int nt = (p.n - t0) < GT_TOK ? (p.n - t0) : GT_TOK;
    if (p.router) {
        const int hw = threadIdx.x >> 5, L = threadIdx.x & 31;
        const int e = sub * GT_ROWS + hw;
        router_rows(p, e, e < p.n_expert, t0, nt, hw, L, part, xs);
    }
    if (!p.chain || !last_arrival(p.sync + SYNC_GATE_CHUNK + chunk, p.wgs_per_chunk))
        return;
    // last workgroup of this chunk: route its tokens, one wave each
    if (wave < nt)
        route_token_wave(p, t0 + wave, sc[wave]);
    if (last_arrival(p.sync + SYNC_GATE_FINAL, p.n_chunks + p.quant_wgs) && p.b.n_groups)
        bucket_block(p);
}

// ---- gated combine (batched path) --------------------------------------------------
// mode 0 (moeRun): out = ((0 + g0*y0) + g1*y1) + ... in selection order.
// mode 1 (moeBatchUnion): out += g*y per expert in ascending expert id.
// mode 2 (moeRun then the residual add, llama.zig:1222): out = out + acc.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y,
                                                      const float *__restrict__ gates,
                                                      const uint32_t *__restrict__ ids,
                                                      const int *__restrict__ pair_of, int k,
                                                      int dim, int mode, float *__restrict__ out) {
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim)
        return;
    const size_t base = (size_t)t * k;
    if (mode != 1) {
        float acc = 0.0f;
        for (int s = 0; s < k; s++) {
            const float pr = gates[base + s] * y[(size_t)pair_of[base + s] * dim + i];
            acc = acc + pr;
        }
        float *o = out + (size_t)t * dim + i;
        *o = mode == 2 ? *o + acc : acc;
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
            const float pr = gates[base + bs] * y[(size_t)pair_of[base + bs] * dim + i];
            acc = acc + pr;
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

// ---- decode-path router: GEMV + input quantization, one wave per work group --------
//
// Work groups [0, ceil(E/2)) hold two router rows each (a half-wave per
// row); the rest quantize one item of the input each.  Lane P of a
// half-wave owns dotF32's accumulator chain P (src/gguf/ggml.zig:198-217):
// columns 32i + P, added in order of i.  For each i the 32 lanes of a row
// read 128 contiguous bytes, so the per-column loads coalesce; the loads of
// up to RS_STEPS steps are issued before the chain starts.  Then
// v_l = ((c_l + c_{8+l}) + c_{16+l}) + c_{24+l} (lanes exchanged with
// ds_bpermute), the sequential reduce over l from -0, and the tail.
constexpr int RS_STEPS = 64; // dotF32 steps (32 columns each) per pass: dim 2048 in one

// rmsnorm of x[dim] into out[dim] by one wave (dim a multiple of 32): lane l
// sums the squares of chunks l, l+64, ... (32 values each, in order), the
// lanes are summed as a fixed tree; out = (x * inv) * w (tensor.zig:9-15's
// expression, FAST-numerics sum order).
__device__ inline void wave_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, int dim, float eps,
                                    float *__restrict__ out) {
    const int lane = threadIdx.x & 63, chunks = dim / 32;
    if (chunks <= 64) { // one chunk per lane: x and w loaded once, together
        const int c = min(lane, chunks - 1);
        float4 xv[8], wv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            xv[i] = *(const float4 *)(x + 32 * c + 4 * i);
            wv[i] = *(const float4 *)(w + 32 * c + 4 * i);
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            ss = ss + xv[i].x * xv[i].x;
            ss = ss + xv[i].y * xv[i].y;
            ss = ss + xv[i].z * xv[i].z;
            ss = ss + xv[i].w * xv[i].w;
        }
        float total = lane < chunks ? ss : 0.0f;
        for (int m = 1; m < 64; m <<= 1)
            total = total + __shfl_xor(total, m);
        const float inv = 1.0f / sqrtf(total / (float)dim + eps);
        if (lane < chunks) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float4 o;
                o.x = (xv[i].x * inv) * wv[i].x;
                o.y = (xv[i].y * inv) * wv[i].y;
                o.z = (xv[i].z * inv) * wv[i].z;
                o.w = (xv[i].w * inv) * wv[i].w;
                *(float4 *)(out + 32 * c + 4 * i) = o;
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int c = lane; c < chunks; c += 64) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = *(const float4 *)(x + 32 * c + 4 * i);
            ss = ss + v.x * v.x;
            ss = ss + v.y * v.y;
            ss = ss + v.z * v.z;
            ss = ss + v.w * v.w;
        }
    }
    float total = ss;
    for (int m = 1; m < 64; m <<= 1)
        total = total + __shfl_xor(total, m);
    const float inv = 1.0f / sqrtf(total / (float)dim + eps);
    for (int i = 4 * lane; i < dim; i += 256) {
        const float4 v = *(const float4 *)(x + i), g = *(const float4 *)(w + i);
        float4 o;
        o.x = (v.x * inv) * g.x;
        o.y = (v.y * inv) * g.y;
        o.z = (v.z * inv) * g.z;
        o.w = (v.w * inv) * g.w;
        *(float4 *)(out + i) = o;
    }
}

constexpr int RS_MAX_DIM = 8192; // fused-norm router: LDS row

// logits[t][e] of half-wave hw's expert e (lanes 32 hw + P) from the normed
// input xt: the dotF32 order of the reference (columns 32 i + P added in order
// of i, then the lanes' sums as below, then the tail).
// FULL: dim is exactly 32 RS_STEPS (one pass, every step live, no tail).
template <bool FULL = false>
__device__ __forceinline__ void router_row_dot(const GateParams &p, int e, bool valid, const float *row,
                                               const float *xt, int t, bool one_pass,
                                               const float (&wpre)[RS_STEPS]) {
    const int lane = threadIdx.x & 63, hw = lane >> 5, P = lane & 31, dim = FULL ? 32 * RS_STEPS : p.dim;
    const int n32 = dim / 32;
    float acc = 0.0f;
    if (FULL) {
#pragma unroll
        for (int u = 0; u < RS_STEPS; u++) {
            const float pr = wpre[u] * xt[32 * u + P];
            acc = acc + pr;
        }
    } else
    for (int i0 = 0; i0 < n32; i0 += RS_STEPS) {
        const int cnt = min(RS_STEPS, n32 - i0);
        float wv[RS_STEPS], xv[RS_STEPS];
#pragma unroll
        for (int u = 0; u < RS_STEPS; u++) { // unconditional: steps past cnt re-read the last
            const int c = 32 * (i0 + min(u, cnt - 1)) + P;
            wv[u] = one_pass ? wpre[u] : row[c];
            xv[u] = xt[c];
        }
        // steps past cnt add +0: acc starts at +0 and a sum of products
        // is never -0, so they change nothing
#pragma unroll
        for (int u = 0; u < RS_STEPS; u++) {
            const float pr = u < cnt ? wv[u] * xv[u] : 0.0f;
            acc = acc + pr;
        }
    }
    // leftover whole 8-chunks go to accumulator 0 (lanes 0..7)
    for (int i = n32 * 32; i + 8 <= dim; i += 8)
        if (P < 8) {
            const float pr = row[i + P] * xt[i + P];
            acc = acc + pr;
        }
    const int src = 32 * hw + (P & 7);
    const float c1 = __int_as_float(__builtin_amdgcn_ds_bpermute((src + 8) << 2, __float_as_int(acc)));
    const float c2 = __int_as_float(__builtin_amdgcn_ds_bpermute((src + 16) << 2, __float_as_int(acc)));
    const float c3 = __int_as_float(__builtin_amdgcn_ds_bpermute((src + 24) << 2, __float_as_int(acc)));
    const float v = ((acc + c1) + c2) + c3; // v_l in lanes 32hw + l, l < 8
    float s0 = -0.0f, s1 = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        s0 = s0 + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
        s1 = s1 + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32 + l));
    }
    if (P == 0 && valid) {
        float s = hw ? s1 : s0;
        for (int j = dim / 8 * 8; j < dim; j++) {
            const float pr = row[j] * xt[j];
            s = s + pr;
        }
        if (p.router_bias)
            s = s + p.router_bias[e];
        p.logits[(size_t)t * p.n_expert + e] = s;
    }
}

__global__ __launch_bounds__(64) void router_small_kernel(GateParams p) {
    __shared__ __align__(16) float xn[RS_MAX_DIM];
    const int lane = threadIdx.x, hw = lane >> 5, P = lane & 31;
    const int gemv_wgs = p.gemv_wgs; // 0 when the caller supplies the logits
    if ((int)blockIdx.x >= gemv_wgs) {
        const int per_vec = quant_items(p.qt, p.dim);
        const int item = blockIdx.x - gemv_wgs;
        if (item < per_vec * p.n) {
            const int v = item / per_vec, it = item % per_vec;
            const float *xv = p.x + (size_t)v * p.dim;
            if (p.norm_w) {
                wave_rmsnorm(xv, p.norm_w, p.dim, p.norm_eps, xn);
                __syncthreads();
                xv = xn;
            }
            quant_item_wave(p.qt, xv, p.dim, v, it, p.qx);
        }
        return;
    }
    const int dim = p.dim;
    const int e = blockIdx.x * 2 + hw;
    const bool valid = e < p.n_expert;
    const float *row = p.router + (size_t)(valid ? e : 0) * dim;
    const int n32 = dim / 32; // whole dotF32 steps
    // one pass of RS_STEPS covers the row: its loads go out before the
    // tokens' inputs (and their norms) are ready
    const bool one_pass = n32 <= RS_STEPS;
    float wpre[RS_STEPS];
    if (one_pass) {
#pragma unroll
        for (int u = 0; u < RS_STEPS; u++)
            wpre[u] = row[32 * min(u, n32 - 1) + P];
    }
    for (int t = 0; t < p.n; t++) {
        const float *xt = p.x + (size_t)t * dim;
        if (p.norm_w) {
            __syncthreads(); // the previous token's reads of xn are done
            wave_rmsnorm(xt, p.norm_w, dim, p.norm_eps, xn);
            __syncthreads();
            xt = xn;
        }
        if (dim == 32 * RS_STEPS)
            router_row_dot<true>(p, e, valid, row, xt, t, one_pass, wpre);
        else
            router_row_dot(p, e, valid, row, xt, t, one_pass, wpre);
    }
}

// PARITY numerics, one token: the fused-norm router with the rmsnorm's sum of
// squares in the reference's order (tensor.zig:9-15; the speculative
// composition of seq_sum_nonneg, which returns that sequential sum itself).
// Every work group (RX_WAVES waves) computes the norm of the token itself --
// there is no norm launch, and the router rows' loads go out before it.
// Gemv groups: two experts per wave; quant groups: one item per wave.
constexpr int RX_WAVES = 8;
constexpr int RX_MAX_DIM = 7936; // the squares, then the normed row, in LDS

constexpr int RX_XV = norm_xv(RX_MAX_DIM, RX_WAVES);

__global__ __launch_bounds__(64 * RX_WAVES) void router_exact_kernel(GateParams p) {
    __shared__ __align__(16) float xn[RX_MAX_DIM];
    __shared__ SeqSumLds seq;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, hw = lane >> 5, P = lane & 31;
    const int dim = p.dim, n32 = dim / 32;
    const bool gemv = (int)blockIdx.x < p.gemv_wgs;
    const int e = ((int)blockIdx.x * RX_WAVES + wave) * 2 + hw;
    const bool valid = gemv && e < p.n_expert;
    const float *row = gemv ? p.router + (size_t)(valid ? e : 0) * dim : nullptr;
    const bool one_pass = n32 <= RS_STEPS;
    // x and the norm weights first: the router rows' loads queue behind them
    float4 xv[RX_XV], wv[RX_XV];
    norm_exact_load<RX_WAVES, RX_XV>(p.x, p.norm_w, dim, xv, wv);
    float wpre[RS_STEPS];
    if (gemv && one_pass) {
#pragma unroll
        for (int u = 0; u < RS_STEPS; u++)
            wpre[u] = row[32 * min(u, n32 - 1) + P];
    }
    norm_exact_block<RX_WAVES, RX_XV>(xv, wv, dim, p.norm_eps, xn, seq);
    if (gemv) {
        if (dim == 32 * RS_STEPS)
            router_row_dot<true>(p, e, valid, row, xn, 0, one_pass, wpre);
        else
            router_row_dot(p, e, valid, row, xn, 0, one_pass, wpre);
    } else {
        const int item = ((int)blockIdx.x - p.gemv_wgs) * RX_WAVES + wave;
        if (item < quant_items(p.qt, dim))
            quant_item_wave(p.qt, xn, dim, 0, item, p.qx);
    }
}

bool router_exact_supported(int n, int dim) { return n == 1 && dim % 32 == 0 && dim <= RX_MAX_DIM; }

void launch_router_small(GateParams p, hipStream_t st) {
    if (p.norm_exact) { // callers check router_exact_supported
        p.gemv_wgs = p.router ? (p.n_expert + 2 * RX_WAVES - 1) / (2 * RX_WAVES) : 0;
        p.quant_wgs = p.qt ? (quant_items(p.qt, p.dim) + RX_WAVES - 1) / RX_WAVES : 0;
        if (p.gemv_wgs + p.quant_wgs == 0)
            return;
        hipLaunchKernelGGL(router_exact_kernel, dim3(p.gemv_wgs + p.quant_wgs), dim3(64 * RX_WAVES), 0, st, p);
        note_launch();
        return;
    }
    p.gemv_wgs = p.router ? (p.n_expert + 1) / 2 : 0; // no router: logits come from the caller
    p.quant_wgs = p.qt ? quant_items(p.qt, p.dim) * p.n : 0;
    if (p.gemv_wgs + p.quant_wgs == 0)
        return;
    hipLaunchKernelGGL(router_small_kernel, dim3(p.gemv_wgs + p.quant_wgs), dim3(64), 0, st, p);
    note_launch();
}

int moe_max_groups(int n, int k, int n_expert, int nt) {
    const int P = n * k;
    const int bound = P / nt + (P < n_expert ? P : n_expert);
    return bound < P ? bound : P;
}

bool gate_supported(int n, int n_expert, int k) {
    return n >= 1 && n <= MAX_TOK && n_expert >= 1 && n_expert <= MAX_E && k >= 1 && k <= MAX_K &&
           k <= n_expert;
}

void launch_gate(GateParams p, hipStream_t st) {
    p.n_chunks = (p.n + GT_TOK - 1) / GT_TOK;
    p.wgs_per_chunk = p.router ? (p.n_expert + GT_ROWS - 1) / GT_ROWS : 1;
    p.gemv_wgs = p.n_chunks * p.wgs_per_chunk;
    p.quant_wgs = p.qt ? (quant_items(p.qt, p.dim) * p.n + GT_THREADS / 64 - 1) / (GT_THREADS / 64) : 0;
    hipLaunchKernelGGL(moe_gate_kernel, dim3(p.gemv_wgs + p.quant_wgs), dim3(GT_THREADS), 0, st, p);
    note_launch();
}

// ---- f32 GEMV for the dense seam (F32 matvec), same dotF32 order ---------------
// One half-wave per (row, up to GT_TOK vectors); no routing.
__global__ __launch_bounds__(GT_THREADS) void f32_gemv_kernel(GateParams p) {
    __shared__ float part[GT_ROWS][GT_TOK][32];
    __shared__ __align__(16) float xs[GT_TOK * GT_COLS];
    const int chunk = blockIdx.x / p.wgs_per_chunk, sub = blockIdx.x % p.wgs_per_chunk;
    const int t0 = chunk * GT_TOK;
    const int nt = (p.n - t0) < GT_TOK ? (p.n - t0) : GT_TOK;
    const int hw = threadIdx.x >> 5, L = threadIdx.x & 31;
    const int e = sub * GT_ROWS + hw;
    router_rows(p, e, e < p.n_expert, t0, nt, hw, L, part, xs);
}

void launch_router_gemv(const float *w, const float *bias, const float *x, int n_expert, int dim,
                        int n, float *logits, hipStream_t st) {
    GateParams p{};
    p.router = w;
    p.router_bias = bias;
    p.x = x;
    p.n = n;
    p.dim = dim;
    p.n_expert = n_expert;
    p.logits = logits;
    p.n_chunks = (n + GT_TOK - 1) / GT_TOK;
    p.wgs_per_chunk = (n_expert + GT_ROWS - 1) / GT_ROWS;
    hipLaunchKernelGGL(f32_gemv_kernel, dim3(p.n_chunks * p.wgs_per_chunk), dim3(GT_THREADS), 0, st,
                       p);
    note_launch();
}

} // namespace lh
