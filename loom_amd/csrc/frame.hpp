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
// values (LDS, zero-padded to a multiple of 64) are cut into at most
// SEQ_MAX_CHUNKS chunks of L values (L a multiple of 64); a double-precision
// prefix sum estimates the running sum at each chunk's start; each lane of a
// wave runs the chunk's chain from one of the 64 f32 values around that
// estimate (consecutive bit patterns; chunk 0 from +0, the reference's
// start); wave 0 then follows the exact running sum through the chunks,
// taking each chunk's end from the lane whose start equals the running sum,
// or re-running the chunk from the exact value when the window missed it.
// Every value produced is one the reference's loop produces, so the result
// is the sequential sum itself.  Adding +0 to a sum of non-negative values
// leaves it unchanged, which makes the zero padding exact.  All NW waves of
// the work group call it.
constexpr int SEQ_MAX_CHUNKS = 32;

struct SeqSumLds {
    float ends[SEQ_MAX_CHUNKS * 64]; // chunk c's end from start lane l
    int nx[SEQ_MAX_CHUNKS * 64];     // the lane of chunk c + 1's window holding it (0x100: none;
                                     // the last chunk: l itself)
    double wtot[16];                 // the estimates' per-wave totals
    uint32_t fst[SEQ_MAX_CHUNKS];    // estimated start (f32 bits) of chunk c
    float out;
};

// DPP move of a double's two halves; out-of-row lanes and rows outside
// ROW_MASK read +0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline double dpp_d0(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, ROW_MASK, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROW_MASK, 0xF, true);
    return __longlong_as_double(((long long)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Inclusive prefix sum over the wave: row_shr 1, 2, 4, 8 within each row of
// 16 lanes, then row_bcast 15 and 31 carry the row totals upward.
__device__ inline double wave_scan_d(double x) {
    x = x + dpp_d0<0x111>(x);
    x = x + dpp_d0<0x112>(x);
    x = x + dpp_d0<0x114>(x);
    x = x + dpp_d0<0x118>(x);
    x = x + dpp_d0<0x142, 0xA>(x);
    x = x + dpp_d0<0x143, 0xC>(x);
    return x;
}

template <int NW>
__device__ __forceinline__ float seq_sum_nonneg(const float *v, int n, SeqSumLds &s) {
    constexpr int NT = 64 * NW;
    if (n <= 0) // the empty sum (n is uniform over the work group)
        return 0.0f;
    const int tid = threadIdx.x, wave = tid >> 6, ln = tid & 63;
    const int n64 = (n + 63) & ~63;
    const int L = 64 * ((n64 / 64 + SEQ_MAX_CHUNKS - 1) / SEQ_MAX_CHUNKS);
    const int C = (n64 + L - 1) / L;
    int K = 1; // values per thread in the estimates: a power of two, so it divides L
    while (K * NT < n64)
        K *= 2;
    // 1. the estimates: an exclusive prefix sum in double at every chunk
    //    start (each thread's K values summed in f32 first: their error is
    //    far below one ulp of the running sum at any chunk start)
    const int j0 = tid * K;
    float ownf = 0.0f;
    if (K >= 4) { // K divides n64: whole float4s, read several at a time
        const int je = min(j0 + K, n64);
#pragma unroll 8
        for (int j = j0; j < je; j += 4) {
            const float4 x = *(const float4 *)(v + j);
            ownf = ownf + x.x;
            ownf = ownf + x.y;
            ownf = ownf + x.z;
            ownf = ownf + x.w;
        }
    } else {
        for (int j = j0; j < min(j0 + K, n64); j++)
            ownf = ownf + v[j];
    }
    const double own = (double)ownf;
    const double inc = wave_scan_d(own);
    if (ln == 63)
        s.wtot[wave] = inc;
    lds_barrier();
    double ex = inc - own;
#pragma unroll
    for (int w = 0; w < NW - 1; w++) // the earlier waves' totals (+0 from the rest: ex >= 0)
        ex = ex + (w < wave ? s.wtot[w] : 0.0);
    if (j0 < n64 && j0 % L == 0)
        s.fst[j0 / L] = __float_as_uint((float)ex);
    lds_barrier();
    // 2. every chunk's chain from 64 starts around its estimate (below).
    //    chain(r, c) is chunk c's chain from the one start r, for the serial
    //    fallback of step 3: blocks of 64 values (16 float4 groups, unrolled),
    //    read eight groups ahead at immediate offsets from the block's base,
    //    one wait per two groups.  Past the chunk's last block the ring
    //    re-reads that block (in range, never added).
    auto chain = [&](float r, int c) {
        constexpr int AH = NW >= 16 ? 4 : 8; // 1024-thread callers keep rows in registers across the sum
        static_assert(16 % AH == 0 && AH % 2 == 0, "the ring wraps at block boundaries, two groups a wait");
        const int nb = min(L, n64 - c * L) / 64;
        const float4 *src = (const float4 *)(v + c * L);
        float4 ring[AH];
#pragma unroll
        for (int a = 0; a < AH; a++)
            ring[a] = src[a];
        for (int bk = 0; bk < nb; bk++) {
            const float4 *cur = src + 16 * bk, *nxt = bk + 1 < nb ? cur + 16 : cur;
#pragma unroll
            for (int g = 0; g < 16; g += 2) {
                const int a = g % AH;
                __builtin_amdgcn_s_waitcnt(0xC07F & ~(0xF << 8) | ((AH - 2) << 8)); // the two oldest reads
                const float4 x0 = ring[a], x1 = ring[a + 1];
                __builtin_amdgcn_sched_barrier(0);
                ring[a] = g + AH < 16 ? cur[g + AH] : nxt[g + AH - 16];
                __builtin_amdgcn_sched_barrier(0);
                r = r + x0.x;
                r = r + x0.y;
                r = r + x0.z;
                r = r + x0.w;
                __builtin_amdgcn_sched_barrier(0);
                ring[a + 1] = g + 1 + AH < 16 ? cur[g + 1 + AH] : nxt[g + 1 + AH - 16];
                __builtin_amdgcn_sched_barrier(0);
                r = r + x1.x;
                r = r + x1.y;
                r = r + x1.z;
                r = r + x1.w;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return r;
    };
    // Lane (quarter qc, slot sl) of a wave runs the four starts 4 sl .. 4 sl + 3
    // of chunk 4 k + qc, so one LDS read (the same address across its
    // quarter) feeds four chains: a quarter of the LDS traffic of one start
    // per lane, and four independent adds per value.
    {
        const int qc = ln >> 4, sl = ln & 15;
        for (int cb = 4 * wave; cb < C; cb += 4 * NW) {
            const int c = min(cb + qc, C - 1); // quarters past the last chunk repeat it and store nothing
            const int nb = min(L, n64 - c * L) / 64;
            const float4 *src = (const float4 *)(v + c * L);
            float r[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                r[k] = c == 0 ? 0.0f : __uint_as_float((uint32_t)max((int)s.fst[c] + 4 * sl + k - 32, 0));
            for (int bk = 0; bk < nb; bk++) {
                const float4 *blk = src + 16 * bk;
#pragma unroll
                for (int g = 0; g < 16; g++) {
                    const float4 x = blk[g];
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        r[k] = r[k] + x.x;
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        r[k] = r[k] + x.y;
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        r[k] = r[k] + x.z;
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        r[k] = r[k] + x.w;
                }
            }
            if (cb + qc < C) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int i = 4 * sl + k;
                    s.ends[c * 64 + i] = r[k];
                    const int n = c + 1 < C ? __float_as_int(r[k]) - (int)s.fst[c + 1] + 32 : i; // the last: itself
                    s.nx[c * 64 + i] = (unsigned)n < 64u ? n : 0x100 | (n & 63);
                }
            }
        }
    }
    lds_barrier();
    // 3. the exact running sum through the chunks: lane i of chunk c has
    //    stored n_c(i), the lane of chunk c + 1's window that holds its end
    //    (flag 0x100: outside the window), so the exact path is a chain of
    //    lane reads idx = n_c(idx) from chunk 0 (which ran from +0 in every
    //    lane).  A flagged step leaves the chain; the chunks are then
    //    followed serially from the start (rare).
    if (wave == 0) {
        const int fa = ln < C ? (int)s.fst[ln] : 0;
        // the path's maps composed as a tree (five levels of lane permutes):
        // (g after f)(l) = g[f(l) & 63], flagged if either step is
        int e[SEQ_MAX_CHUNKS]; // past the last chunk, its row: the identity
#pragma unroll
        for (int c = 0; c < SEQ_MAX_CHUNKS; c++)
            e[c] = s.nx[min(c, C - 1) * 64 + ln];
#pragma unroll
        for (int w = 1; w < SEQ_MAX_CHUNKS; w *= 2) {
#pragma unroll
            for (int c = 0; c < SEQ_MAX_CHUNKS; c += 2 * w)
                e[c] = __builtin_amdgcn_ds_bpermute((e[c] & 63) << 2, e[c + w]) | (e[c] & 0x100);
        }
        const int idx = __builtin_amdgcn_readfirstlane(e[0]); // the path from lane 0 of chunk 0
        const int flags = idx;
        int run;
        if (!(flags & 0x100)) {
            run = __builtin_amdgcn_readfirstlane(__float_as_int(s.ends[(C - 1) * 64 + (idx & 63)]));
        } else { // some start fell outside its window: every chunk in turn
            run = __builtin_amdgcn_readfirstlane(__float_as_int(s.ends[0]));
            for (int c = 1; c < C; c++) {
                const int i = run - __builtin_amdgcn_readlane(fa, c) + 32;
                if ((unsigned)i < 64u) {
                    run = __builtin_amdgcn_readfirstlane(__float_as_int(s.ends[c * 64 + i]));
                } else { // the chain from the exact value (every lane the same)
                    run = __builtin_amdgcn_readfirstlane(__float_as_int(chain(__int_as_float(run), c)));
                }
            }
        }
        if (ln == 0)
            s.out = __int_as_float(run);
    }
    lds_barrier();
    return s.out;
}

// e[j] = exp(sv[k] - m) (j = threadIdx.x + NT*k) for j < P, +0 up to n64:
// the exponentials four at a time, unconditionally inside a group (sv is
// -inf past P); groups wholly past n64 are skipped (uniform).  The library's
// once-rounded double exponential (exp_f32): measured in this loop, 8 values
// per thread at 512 threads, it takes 1.6 us against the polynomial form's
// 2.0 us.
template <int NT, int NV>
__device__ __forceinline__ void softmax_exps(const float (&sv)[NV], float m, int P, int n64, float *e) {
#pragma unroll
    for (int kb = 0; kb < NV; kb += 4) {
        if (NT * kb >= n64)
            break;
        float a[4], y[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[i] = kb + i < NV ? sv[kb + i] - m : -INFINITY;
            y[i] = exp_f32(a[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = (int)threadIdx.x + NT * (kb + i);
            if (kb + i < NV && j < n64)
                e[j] = j < P ? y[i] : 0.0f;
        }
    }
}

// ---- rmsnorm with the reference's sum, computed by a whole work group ----------
// (tensor.zig:9-15) for a kernel that normalises its own input: x and the
// norm weights in registers -- float4 k of thread tid holds values
// 4 tid + 256 NW k, XV of them cover the largest dim served -- then the
// squares in order, zero-padded to whole 64s, summed sequentially
// (seq_sum_nonneg), then xn = (x * scale) * w in LDS.
__host__ __device__ constexpr int norm_xv(int max_dim, int nw) { return (max_dim + 256 * nw - 1) / (256 * nw); }

template <int NW, int XV>
__device__ __forceinline__ void norm_exact_load(const float *__restrict__ x, const float *__restrict__ w, int dim,
                                                float4 (&xv)[XV], float4 (&wv)[XV]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < XV; k++) {
        const int i = 4 * tid + 4 * 64 * NW * k;
        xv[k] = wv[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < dim) { // dim is a multiple of 32
            xv[k] = *(const float4 *)(x + i);
            wv[k] = *(const float4 *)(w + i);
        }
    }
}

template <int NW, int XV>
__device__ __forceinline__ void norm_exact_block(const float4 (&xv)[XV], const float4 (&wv)[XV], int dim,
                                                 float eps, float *xn, SeqSumLds &seq) {
    const int tid = threadIdx.x, n64 = (dim + 63) & ~63;
#pragma unroll
    for (int k = 0; k < XV; k++) {
        const int i = 4 * tid + 4 * 64 * NW * k;
        if (i < n64) {
            float4 q;
            q.x = xv[k].x * xv[k].x;
            q.y = xv[k].y * xv[k].y;
            q.z = xv[k].z * xv[k].z;
            q.w = xv[k].w * xv[k].w;
            *(float4 *)(xn + i) = q;
        }
    }
    lds_barrier();
    const float total = seq_sum_nonneg<NW>(xn, dim, seq); // ends with a barrier: xn is free again
    const float scale = 1.0f / sqrtf(total / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < XV; k++) {
        const int i = 4 * tid + 4 * 64 * NW * k;
        if (i < dim) {
            float4 o;
            o.x = (xv[k].x * scale) * wv[k].x;
            o.y = (xv[k].y * scale) * wv[k].y;
            o.z = (xv[k].z * scale) * wv[k].z;
            o.w = (xv[k].w * scale) * wv[k].w;
            *(float4 *)(xn + i) = o;
        }
    }
    lds_barrier();
}

// ---- the reference-order attention (attn_exact.hip), PARITY numerics --------
// Scores, softmax and P.V of llama.zig:1162-1192 in the reference's own
// evaluation order over any context: one launch of scores per 64 positions,
// one softmax launch per (head, lane), one P.V launch per (64 columns, KV
// head, lane).  S is [n][n_heads][s_stride] f32 (scores, then p in place),
// att the f32 attention output [n][n_heads * head_dim].
constexpr int EXACT_MAX_CTX = 7936; // the softmax's e[] and the sequential sum's LDS in 64 KB

// softmax (tensor.zig:18-28) of one row of P scores in place, in the
// reference's order: m = max (order-free), e_t = exp(s_t - m) rounded once
// from a double exponential (softmax_exps), the position-ordered sum of e
// (speculative composition, exact),
// p_t = e_t * (1 / sum).  e holds 64 * ceil(P / 64) floats of LDS (positions
// past P read +0); all NT threads of the work group call it.

template <int NT>
__device__ __forceinline__ void softmax_row_exact(float *row, int P, float *e, float *redf, SeqSumLds &seq) {
    // the row is read once, every load issued before the first use (a loop
    // over P would wait out one memory round trip per iteration)
    constexpr int NV = (EXACT_MAX_CTX + NT - 1) / NT;
    const int tid = threadIdx.x, wave = tid >> 6, ln = tid & 63;
    const int C = (P + 63) / 64;
    float sv[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int j = tid + NT * k;
        sv[k] = j < P ? row[j] : -INFINITY;
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; k++)
        m = fmaxf(m, sv[k]);
    m = wave_max(m);
    if (ln == 0)
        redf[wave] = m;
    lds_barrier();
    m = redf[0];
    for (int w = 1; w < NT / 64; w++)
        m = fmaxf(m, redf[w]);
    softmax_exps<NT>(sv, m, P, 64 * C, e);
    lds_barrier();
    const float inv = 1.0f / seq_sum_nonneg<NT / 64>(e, P, seq);
    for (int j = tid; j < P; j += NT)
        row[j] = e[j] * inv;
}

size_t exact_softmax_lds(int s_stride);
// qwt >= 0 (attn_exact_quant_fusable): P.V also quantizes att into qa for a
// weight of type qwt, in place of a quantizer launch.
bool attn_exact_quant_fusable(const FrameDims &D, size_t n);
bool launch_attn_exact(const FrameDims &D, const float *q, const float *k, const float *v, const float *q_norm,
                       const float *k_norm, const float *rope_cs, uint16_t *kc, uint16_t *vc, const int32_t *pos,
                       int li, bool fuse, float *S, int s_stride, float *att, size_t n, int qwt, const QAct &qa,
                       hipStream_t st);

} // namespace lh
