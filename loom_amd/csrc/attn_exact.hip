// attn_exact.hip -- GQA attention over the fp16 K/V cache in the reference's
// own evaluation order (src/gguf/llama.zig:1162-1192), for any context length:
//
//   s_t = dotF32(q, k_t) * scale                      (ggml.zig:198-217)
//   m = max s_t;  e_t = exp(s_t - m);  sum = e_0 + e_1 + ... in position order
//   p_t = e_t * (1 / sum)                              (tensor.zig:18-28)
//   o = 0;  o[d] = o[d] + p_t * v_t[d] in position order (axpy, ggml.zig:221-230)
//
// so the attention output -- and with it the int8 input of wo -- is bit-
// identical to Loom's CPU path at every context length, which a
// split-context (flash-decoding) merge is not.  Up to 4 lanes, two launches:
//
//   attn_scores_kernel    per (64 positions, KV head, lane): the group's query
//                         heads against 64 keys, dotF32 order on the VALU, with
//                         the per-head Q/K RMSNorm and RoPE and the K/V append
//   attn_pv_split_kernel  per (32 value columns, head, lane): the head's
//                         softmax, then o = o + p_t * v_t position by position
//                         (a consumer wave fed products by producer waves)
//
// and from 5 lanes (after qk_rope_kernel has rotated the queries and appended
// the rows), three:
//
//   attn_scores_many_kernel  per (256 positions, KV head, lane): a thread per
//                            position, the query elements as scalar operands
//   attn_softmax_kernel      per (query head, lane): the max, e_t, the
//                            position-ordered sum, p_t (in place of the scores)
//   attn_pv_many_kernel      per (64 value columns, KV head, lane): a wave per
//                            head, lane = column, over value tiles staged in LDS
//
// The sequential sum of e_t is a dependent chain of P adds (~5.7 cycles each
// on gfx950).  It is evaluated by speculative composition instead: the
// context is cut into 64-position chunks; a double-precision prefix sum
// estimates the running sum at each chunk's start; each lane of a wave runs
// the chunk's chain from one of the 64 f32 values around that estimate
// (consecutive bit patterns); a single pass over the chunks then follows the
// exact running sum from chunk to chunk, reading each chunk's end from the
// lane whose start equals it.  A start outside the window (rare) re-runs that
// chunk serially from the exact value.  Every value is one the reference's
// loop produces: the result is the sequential sum itself.
#include "frame.hpp"
#include "runtime.hpp"

namespace lh {

constexpr int SC_THREADS = 512;   // scores: 8 waves
constexpr int SM_THREADS = 1024;  // softmax: 16 waves

// ---- scores -------------------------------------------------------------------------
// Work group (chunk of 64 positions, KV head, lane).  All 512 threads load the
// chunk's keys into padded LDS rows and the group's query heads; wave w scores
// query heads w, w+8, ...: lane j takes position t0 + j.  fuse: the query
// heads arrive raw and get headNorm (llama.zig:938-949, the squares summed in
// order) and RoPE here; the chunk holding the new position normalises,
// rotates and appends its K row and appends its V row (a full cache takes no
// more rows), and scores against the new row from LDS.
template <int HD>
__global__ __launch_bounds__(SC_THREADS) void attn_scores_kernel(
    FrameDims D, const float *__restrict__ qraw, const float *__restrict__ kraw, const float *__restrict__ vraw,
    const float *__restrict__ q_norm, const float *__restrict__ k_norm, const float *__restrict__ rope_cs,
    uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const int32_t *__restrict__ pos, int li, int fuse,
    float *__restrict__ S, int s_stride) {
    constexpr int KS = HD + 8;                              // padded key row (halves)
    constexpr int PR = HD / 8;                              // 16-byte pieces per row
    constexpr int NPW = (ATT_TC * PR + SC_THREADS - 1) / SC_THREADS; // pieces per thread
    __shared__ __align__(16) float qs[MAX_G * HD];
    __shared__ __align__(16) uint16_t ks[ATT_TC * KS];
    __shared__ float kn[HD], sinv[MAX_G + 1];
    const int ch = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int wave = tid >> 6, ln = tid & 63;
    const int G = D.n_heads / D.n_kv;
    const int p_raw = pos[t];
    const int p = min(p_raw, D.ctx - 1);
    const int t0 = ch * ATT_TC, nt = min(ATT_TC, p + 1 - t0);
    if (nt <= 0)
        return; // past the current position
    const bool own = fuse && p_raw >= 0 && p_raw < D.ctx && p_raw >= t0 && p_raw < t0 + ATT_TC;
    const int rp = min(max(p_raw, 0), D.ctx - 1); // rope position
    const size_t row0 = (((size_t)t * D.n_layers + li) * D.ctx + t0) * D.kvd + (size_t)kvh * HD;
    const float *qsrc = qraw + (size_t)t * D.qd + (size_t)kvh * G * HD;
    const size_t kvo = (size_t)t * D.kvd + (size_t)kvh * HD;
    uint4 pc[NPW];
#pragma unroll
    for (int u = 0; u < NPW; u++) {
        const int i = tid + SC_THREADS * u;
        pc[u] = i < ATT_TC * PR ? *(const uint4 *)(kc + row0 + (size_t)min(i / PR, nt - 1) * D.kvd + 8 * (i % PR))
                                : make_uint4(0, 0, 0, 0);
    }
    float vnew = 0.0f;
    if (own && tid < HD) {
        kn[tid] = kraw[kvo + tid];
        vnew = vraw[kvo + tid];
    }
    for (int i = tid; i < G * HD; i += SC_THREADS)
        qs[i] = qsrc[i];
#pragma unroll
    for (int u = 0; u < NPW; u++) {
        const int i = tid + SC_THREADS * u;
        if (i < ATT_TC * PR)
            *(uint4 *)(ks + (i / PR) * KS + 8 * (i % PR)) = pc[u];
    }
    __syncthreads();
    if (fuse) {
        // headNorm: the squares summed in the reference's order, one thread per head
        if (q_norm && tid < G) {
            float ss = 0.0f;
            for (int i = 0; i < HD; i++) {
                const float pr = qs[tid * HD + i] * qs[tid * HD + i];
                ss = ss + pr;
            }
            sinv[tid] = 1.0f / sqrtf(ss / (float)HD + D.eps);
        }
        if (own && k_norm && tid == SC_THREADS - 64) {
            float ss = 0.0f;
            for (int i = 0; i < HD; i++) {
                const float pr = kn[i] * kn[i];
                ss = ss + pr;
            }
            sinv[MAX_G] = 1.0f / sqrtf(ss / (float)HD + D.eps);
        }
        __syncthreads();
        if (q_norm)
            for (int i = tid; i < G * HD; i += SC_THREADS)
                qs[i] = (qs[i] * sinv[i / HD]) * q_norm[i % HD];
        if (own && k_norm && tid < HD)
            kn[tid] = (kn[tid] * sinv[MAX_G]) * k_norm[tid];
        __syncthreads();
        // RoPE (llama.zig:821-855) from the (cos, sin) table at the position
        const int hr = D.rope_dim / 2;
        const float *csp = rope_cs + (size_t)rp * hr * 2;
        for (int i = tid; i < G * hr; i += SC_THREADS) {
            const int g = i / hr, r = i % hr;
            const float cs = csp[2 * r], sn = csp[2 * r + 1];
            const int ia = D.rope_neox ? r : 2 * r, ib = D.rope_neox ? r + hr : 2 * r + 1;
            const float a = qs[g * HD + ia], b = qs[g * HD + ib];
            qs[g * HD + ia] = a * cs - b * sn;
            qs[g * HD + ib] = a * sn + b * cs;
        }
        if (own && tid >= SC_THREADS - 64 && tid - (SC_THREADS - 64) < hr) {
            const int r = tid - (SC_THREADS - 64);
            const float cs = csp[2 * r], sn = csp[2 * r + 1];
            const int ia = D.rope_neox ? r : 2 * r, ib = D.rope_neox ? r + hr : 2 * r + 1;
            const float a = kn[ia], b = kn[ib];
            kn[ia] = a * cs - b * sn;
            kn[ib] = a * sn + b * cs;
        }
        __syncthreads();
        if (own && tid < HD) { // the new row: to the cache and over its stale LDS copy
            const uint16_t kh = __half_raw(__float2half(kn[tid])).x, vh = __half_raw(__float2half(vnew)).x;
            const size_t crow = (((size_t)t * D.n_layers + li) * D.ctx + p_raw) * D.kvd + (size_t)kvh * HD;
            kc[crow + tid] = kh;
            vc[crow + tid] = vh;
            ks[(p_raw - t0) * KS + tid] = kh;
        }
        __syncthreads();
    }
    const uint16_t *krow = ks + min(ln, nt - 1) * KS;
    for (int g = wave; g < G; g += SC_THREADS / 64) {
        const float s = dot_f32_key<HD>(qs + g * HD, krow) * D.scale;
        if (ln < nt)
            S[((size_t)t * D.n_heads + (size_t)kvh * G + g) * s_stride + t0 + ln] = s;
    }
}

// ---- scores for many lanes ------------------------------------------------------------
// Work group (256 positions, KV head, lane), one thread per position: the
// thread loads its key row, converts it to f32 once, and scores it against
// each query head of the group in turn.  The query elements are wave-uniform
// and arrive as scalar operands (scalar loads of the rotated queries, which
// an earlier launch wrote), so the dot's only vector work is dotF32's own
// multiply and add per element, then its fixed tree.  The first product of
// each of the 32 accumulators is taken as the accumulator itself instead of
// 0 + x: the two differ only when x = -0 (0 + -0 = +0), and an accumulator
// that holds -0 where the reference holds +0 can only change the sign of a
// zero score -- s = +-0, which softmax reads only through s - m and max,
// where both zeros give the same e and p.  The new K/V rows were appended by
// qk_rope_kernel before this launch.
constexpr int SCM_THREADS = 256;

template <int HD>
__global__ __launch_bounds__(SCM_THREADS) void attn_scores_many_kernel(FrameDims D, const float *__restrict__ qrot,
                                                                     const uint16_t *__restrict__ kc,
                                                                     const int32_t *__restrict__ pos, int li,
                                                                     float *__restrict__ S, int s_stride) {
    static_assert(HD % 8 == 0 && HD <= 256, "whole 8-element chunks");
    constexpr int W32 = HD / 32 * 32; // elements in whole 32-steps; the rest go to accumulators 0..7
    const int kvh = blockIdx.y, t = blockIdx.z;
    const int G = D.n_heads / D.n_kv;
    const int P = min(pos[t], D.ctx - 1) + 1;
    const int j = blockIdx.x * SCM_THREADS + threadIdx.x;
    if (blockIdx.x * SCM_THREADS >= P)
        return;
    const uint16_t *krow =
        kc + (((size_t)t * D.n_layers + li) * D.ctx + min(j, P - 1)) * D.kvd + (size_t)kvh * HD;
    float k[HD];
#pragma unroll
    for (int i = 0; i < HD; i += 8) {
        const uint4 w = *(const uint4 *)(krow + i);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; e++)
            k[i + e] = half_bits_to_float(ww[e >> 1] >> (16 * (e & 1)));
    }
    const float *qg = qrot + (size_t)t * D.qd + (size_t)kvh * G * HD;
    float *srow = S + ((size_t)t * D.n_heads + (size_t)kvh * G) * s_stride + j;
    for (int g = 0; g < G; g++) {
        const float *q = qg + (size_t)g * HD; // uniform: scalar loads
        float acc[32];
#pragma unroll
        for (int i = 0; i < HD; i++) {
            const int u = i < W32 ? i % 32 : (i - W32) % 8;
            const float pr = q[i] * k[i];
            if (i < 32)
                acc[u] = pr;
            else
                acc[u] = acc[u] + pr;
        }
#pragma unroll
        for (int u = HD < 32 ? HD : 32; u < 32; u++)
            acc[u] = 0.0f;
        float s = -0.0f;
#pragma unroll
        for (int l = 0; l < 8; l++)
            s = s + (((acc[l] + acc[8 + l]) + acc[16 + l]) + acc[24 + l]);
        if (j < P)
            srow[(size_t)g * s_stride] = s * D.scale;
    }
}

// ---- softmax ------------------------------------------------------------------------
// Work group (query head, lane): the max, e_t, the position-ordered sum of e
// (the speculative composition), p_t.  The many-lane launch runs NT = 512:
// at 64 registers (eight waves per SIMD) four groups share a CU, so 32 lanes
// x 32 heads run in one round, and eight waves take the sum's chunk chains
// in one pass.

template <int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(8))) void attn_softmax_kernel(FrameDims D, const int32_t *__restrict__ pos,
                                                          float *__restrict__ S, int s_stride) {
    extern __shared__ __align__(16) float e[]; // e[s_stride]
    __shared__ float redf[NT / 64];
    __shared__ SeqSumLds seq;
    const int h = blockIdx.x, t = blockIdx.z;
    const int P = min(pos[t], D.ctx - 1) + 1;
    if (P <= 0) // a lane at a negative position has no scores (the whole group leaves)
        return;
    softmax_row_exact<NT>(S + ((size_t)t * D.n_heads + h) * s_stride, P, e, redf, seq);
}

// ---- P.V for many lanes ----------------------------------------------------------------
// Work group (64 value columns, up to NW query heads of one KV head, lane),
// one wave per head, lane = column.  A tile of PVM_TJ positions x 64 columns
// is staged in LDS once for the group's heads, as position quads: the two
// dwords of (quad q, column c) hold v[4q..4q+3][c] as f16 pairs, so one
// 8-byte read per lane brings four positions of its column (consecutive
// lanes: consecutive 8 bytes, conflict-free).  p of each wave's head is
// staged beside it and read four positions at a time by a broadcast read.
// Per position the wave issues the product (fma(p, v, +0) on the f16 value:
// v_fma_mix) and the dependent add, from a software pipeline whose order the
// fences keep: at step j the chain adds its product of position j and forms
// the product of position j + 4, and every fourth step reads the quad three
// ahead.  The tiles' global loads run PVM_SETS tiles ahead, and every
// iteration issues the same loads (tiles past the last are staged from
// clamped addresses and run no chain), so the in-order load counter waits
// for each set's own loads alone.  The chain stops at position P - 1 exactly
// (the last tile runs a bounded loop): nothing past the context enters a sum.
//
// Measured at 32 lanes x 4096 positions (Qwen3 shapes): 57 us.  The bound is
// the LDS (per CU and position: 8 waves x (128 B of values + 256 B of p))
// with the VALU close behind (v_fma_mix issues at about half the rate of an
// f32 multiply); p by v_readlane, p broadcast by the matrix cores
// (v_mfma_f32_32x32x1f32 against 1.0), two heads per lane, and the values as
// f32 with v_mul all measured slower, as did f32 values with p read once per
// 32 positions and turned into scalar operands by 32 v_readlane issued ahead
// of the group's products (76 us against 58: readlane + v_mul + add per
// position costs more than v_fma_mix + add, whatever it saves the LDS).
constexpr int PVM_TJ = 128;        // positions per tile
constexpr int PVM_Q = PVM_TJ / 4;  // position quads per tile
constexpr int PVM_RS = 2 * 64 + 4; // dwords per quad row (64 columns x 2, padded)
constexpr int PVM_SETS = 3;        // tiles of loads in flight (register sets)
constexpr int PVM_AH = 3;          // quads read ahead of the chain

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void attn_pv_many_kernel(FrameDims D, const uint16_t *__restrict__ vc,
                                                               const int32_t *__restrict__ pos, int li,
                                                               const float *__restrict__ Pm, int s_stride,
                                                               float *__restrict__ att) {
    constexpr int NT = 64 * NW;
    constexpr int ITEMS = PVM_Q * 8;           // (quad, column octet) items per tile
    constexpr int IPT = (ITEMS + NT - 1) / NT; // items per thread
    __shared__ __align__(16) uint32_t vt[2][PVM_Q * PVM_RS];
    __shared__ __align__(16) float pt[2][NW][PVM_TJ];
    const int G = D.n_heads / D.n_kv;
    const int n_hg = (G + NW - 1) / NW;
    const int sl = blockIdx.x, kvh = blockIdx.y / n_hg, hg = blockIdx.y % n_hg, t = blockIdx.z;
    const int tid = threadIdx.x, ln = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int P = min(pos[t], D.ctx - 1) + 1;
    const int ntile = (P + PVM_TJ - 1) / PVM_TJ;
    const int c0 = sl * 64, ncol = min(64, HD - c0);
    const int g = hg * NW + wave; // the wave's head within the KV group
    if (P <= 0) { // a lane at a negative position has no context: +0 out, no loads
        if (ln < ncol && g < G)
            att[(size_t)t * D.qd + ((size_t)kvh * G + g) * HD + c0 + ln] = 0.0f;
        return;
    }
    const char *vb = (const char *)(vc + (((size_t)t * D.n_layers + li) * D.ctx) * D.kvd + (size_t)kvh * HD + c0);
    const uint32_t rowb = (uint32_t)D.kvd * 2;
    // a wave past the group's last head runs on a clamped p row and stores nothing
    const float *prow = Pm + ((size_t)t * D.n_heads + (size_t)kvh * G + min(g, G - 1)) * s_stride;

    struct Set {
        uint4 v[IPT][4];
        float p[2];
    };
    // Every load is unconditional from a clamped address (rows to P - 1,
    // column octets to the head's last, p to the row's end).
    auto load = [&](int tile, Set &s) {
#pragma unroll
        for (int u = 0; u < IPT; u++) {
            const int i = min(tid + NT * u, ITEMS - 1), q = i >> 3, cg = min(i & 7, ncol / 8 - 1);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = min(tile * PVM_TJ + 4 * q + r, P - 1);
                s.v[u][r] = *(const uint4 *)(vb + (size_t)row * rowb + 16 * cg);
            }
        }
#pragma unroll
        for (int k = 0; k < 2; k++)
            s.p[k] = prow[min(tile * PVM_TJ + 64 * k + ln, s_stride - 1)];
    };
    auto stage = [&](int buf, const Set &s) {
#pragma unroll
        for (int k = 0; k < 2; k++)
            pt[buf][wave][64 * k + ln] = s.p[k];
#pragma unroll
        for (int u = 0; u < IPT; u++) {
            const int i = tid + NT * u;
            if (ITEMS % NT == 0 || i < ITEMS) {
                const int q = i >> 3, cg = i & 7;
                const uint32_t r0[4] = {s.v[u][0].x, s.v[u][0].y, s.v[u][0].z, s.v[u][0].w};
                const uint32_t r1[4] = {s.v[u][1].x, s.v[u][1].y, s.v[u][1].z, s.v[u][1].w};
                const uint32_t r2[4] = {s.v[u][2].x, s.v[u][2].y, s.v[u][2].z, s.v[u][2].w};
                const uint32_t r3[4] = {s.v[u][3].x, s.v[u][3].y, s.v[u][3].z, s.v[u][3].w};
#pragma unroll
                for (int m = 0; m < 4; m++) { // columns 8 cg + 2m (low halves) and + 1 (high halves)
                    uint4 w;
                    w.x = __builtin_amdgcn_perm(r1[m], r0[m], 0x05040100u);
                    w.y = __builtin_amdgcn_perm(r3[m], r2[m], 0x05040100u);
                    w.z = __builtin_amdgcn_perm(r1[m], r0[m], 0x07060302u);
                    w.w = __builtin_amdgcn_perm(r3[m], r2[m], 0x07060302u);
                    *(uint4 *)&vt[buf][q * PVM_RS + 16 * cg + 4 * m] = w;
                }
            }
        }
    };
    float o = 0.0f;
    auto compute = [&](int buf, int tile) {
        const uint32_t *src = &vt[buf][2 * ln];
        const float *pw = pt[buf][wave];
        const int nk = min(PVM_TJ, P - tile * PVM_TJ);
        if (nk == PVM_TJ) {
            uint2 w[PVM_AH + 1];
            float4 pq[PVM_AH + 1];
#pragma unroll
            for (int q = 0; q < PVM_AH; q++) {
                w[q] = *(const uint2 *)(src + q * PVM_RS);
                pq[q] = *(const float4 *)(pw + 4 * q);
            }
            auto vval = [&](int j) {
                const uint2 &x = w[(j >> 2) % (PVM_AH + 1)];
                return half_bits_to_float(((j & 2) ? x.y : x.x) >> (16 * (j & 1)));
            };
            auto pval = [&](int j) {
                const float4 &x = pq[(j >> 2) % (PVM_AH + 1)];
                return (j & 3) == 0 ? x.x : (j & 3) == 1 ? x.y : (j & 3) == 2 ? x.z : x.w;
            };
            float xp[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                xp[j] = __builtin_fmaf(pval(j), vval(j), 0.0f);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < PVM_TJ; j++) {
                if ((j & 3) == 0 && j / 4 + PVM_AH < PVM_Q) {
                    const int q = j / 4 + PVM_AH;
                    w[q % (PVM_AH + 1)] = *(const uint2 *)(src + q * PVM_RS);
                    pq[q % (PVM_AH + 1)] = *(const float4 *)(pw + 4 * q);
                }
                o = o + xp[j & 3];
                if (j + 4 < PVM_TJ)
                    xp[j & 3] = __builtin_fmaf(pval(j + 4), vval(j + 4), 0.0f);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            for (int j = 0; j < nk; j++) {
                const uint32_t w = src[(j >> 2) * PVM_RS + ((j >> 1) & 1)];
                const float x = __builtin_fmaf(pw[j], half_bits_to_float(w >> (16 * (j & 1))), 0.0f);
                o = o + x;
            }
        }
    };
    Set s[PVM_SETS];
    // the sets' loads are issued in set order (the fences keep them there),
    // so that each set's wait leaves the later sets' loads in flight
#pragma unroll
    for (int d = 0; d < PVM_SETS; d++) {
        load(d, s[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
    stage(0, s[0]);
    __builtin_amdgcn_sched_barrier(0);
    load(PVM_SETS, s[0]);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    // iteration k: tile k + 1 is staged from set (k + 1) % SETS into buffer
    // (k + 1) & 1 and that set reloaded with tile k + 1 + SETS; tile k's
    // chains run from buffer k & 1; one barrier per tile.  The loop runs
    // whole register sets.
    const int ntp = (ntile + PVM_SETS - 1) / PVM_SETS * PVM_SETS;
    for (int kb = 0; kb < ntp; kb += PVM_SETS) {
#pragma unroll
        for (int d = 0; d < PVM_SETS; d++) {
            const int k = kb + d, nxt = (d + 1) % PVM_SETS;
            stage((k + 1) & 1, s[nxt]);
            __builtin_amdgcn_sched_barrier(0);
            load(k + 1 + PVM_SETS, s[nxt]);
            __builtin_amdgcn_sched_barrier(0);
            if (k < ntile)
                compute(k & 1, k);
            lds_barrier();
        }
    }
    if (ln < ncol && g < G)
        att[(size_t)t * D.qd + ((size_t)kvh * G + g) * HD + c0 + ln] = o;
}

// ---- P.V for few lanes: the chain fed by producer waves ----------------------------
// With few lanes there are too few chains to fill the chip, and each chain's
// time is what counts: a wave that also multiplies, converts and stages
// spends two or more issue slots per position.  Here a work group (32 value
// columns, query head, lane) has one consumer wave, lane = column (lanes 32
// and up shadow 0..31 and store nothing), whose loop is only o = o + x_t
// over products x_t read from LDS four positions at a time, and PVS_NP
// producer waves that write x_t = p_t * v_t for the consumer two tiles
// ahead, 64 positions of each tile apiece.  The consumer's chain costs the
// same per position whatever its lane count; the narrower group halves
// each producer's share of the products per position.  The product
// is formed as fma(p, v, +0) on the f16 value directly (v_fma_mix_f32): the
// same rounding as p * v in f32,
// except that an exact zero comes out +0 -- and o, which starts at +0 and
// only ever receives sums, reads o + (+0) = o + (-0) = o either way.
// Each wave passes one barrier per tile; the consumer reads only positions
// below P, so what the producers write past the context is never used.  The
// consumer's barrier waits for none of its own reads: the ones in flight at
// a barrier read the next tile's buffer, which the producers only rewrite
// two barriers later; the producers' barrier waits for their stores.
constexpr int PVS_NP = 3;                // producer waves per work group
constexpr int PVS_COLS = 32;             // value columns per work group
constexpr int PVS_TJ = 64 * PVS_NP;      // positions per tile, 64 per producer
constexpr int PVS_SETS = 4;              // tiles of value loads in flight per producer
constexpr int PVS_STR = 4 * ((PVS_TJ / 4 + 15) / 16 * 16 + 1); // f32 stride of a column's products:
                                         // a whole number of 16-byte slots, 1 mod 16
constexpr int PVS_NBUF = 3;              // product tiles: the consumer's, and two ahead
constexpr int PVS_AHEAD = 8;             // consumer float4 reads in flight (divides a tile's groups, so
                                         // the ring carries the next tile's first reads in the slots
                                         // it starts from)
static_assert((PVS_TJ / 4) % PVS_AHEAD == 0, "the read ring must wrap at tile boundaries");

// Column c's products are LDS row c.  Rows are a whole number of 16-byte
// slots apart, 1 mod 16, so slot (c, g) -- position group g of column c --
// sits in bank group (c + g) mod 16.  The consumer reads one g across
// consecutive columns, a producer store one c across 16 consecutive g:
// every 8 and every 16 consecutive lanes of either access hit distinct bank
// groups.

// qwt >= 0: the output is also quantized for a weight of type qwt (the wo
// matvec's input, 256-column items): the last of an item's eight groups to
// store its columns quantizes the item (its data handed over through
// agent-scope stores and loads, counters in the sync buffer), in place of a
// quantizer launch.
//
// SM: the group computes its head's softmax itself (the scores in Pm,
// tensor.zig:18-28 in the reference's order, as attn_softmax_kernel) into
// LDS, and the producers form p_t = e_t * inv from there -- the same
// rounding as the softmax launch's p, with no launch, and the first value
// tiles' loads in flight while the softmax runs.  512 threads: waves 4..7
// help with the softmax, then only pass the tiles' barriers.
constexpr int PVS_SM_WAVES = 8;
constexpr int PVS_SM_VALS = (EXACT_MAX_CTX + 64 * PVS_SM_WAVES - 1) / (64 * PVS_SM_WAVES); // scores per thread
size_t pv_softmax_lds(int s_stride) { return (size_t)s_stride * 4; }

template <int HD, bool SM>
__global__ __launch_bounds__(SM ? 64 * PVS_SM_WAVES : 64 * (1 + PVS_NP)) void attn_pv_split_kernel(
    FrameDims D, const uint16_t *__restrict__ vc, const int32_t *__restrict__ pos, int li,
    const float *__restrict__ Pm, int s_stride, float *__restrict__ att, int qwt, QAct qa,
    int *__restrict__ sync) {
    constexpr int PP = PVS_TJ / PVS_NP; // positions per producer per tile
    constexpr int NW = SM ? PVS_SM_WAVES : 1 + PVS_NP;
    __shared__ __align__(16) float prod[PVS_NBUF][PVS_COLS * PVS_STR];
    extern __shared__ __align__(16) float e[]; // SM: e_t of the head, 64 * ceil(P / 64) values
    __shared__ float redf[NW];
    __shared__ SeqSumLds seq;
    const int ncb = (HD + PVS_COLS - 1) / PVS_COLS;
    // XCD-aware order: consecutive work items share an XCD (work groups are
    // dealt to the 8 XCDs round robin), so one KV head's values stay in few L2s
    const int nwg = ncb * D.n_heads, lin = blockIdx.x;
    const int wi = (nwg % 8 == 0) ? (lin % 8) * (nwg / 8) + lin / 8 : lin;
    const int sl = wi % ncb, h = wi / ncb, t = blockIdx.z;
    const int wave = threadIdx.x >> 6, ln = threadIdx.x & 63;
    const int G = D.n_heads / D.n_kv, kvh = h / G;
    const int P = min(pos[t], D.ctx - 1) + 1;
    const int ntile = (P + PVS_TJ - 1) / PVS_TJ;
    const int ntp = (ntile + PVS_SETS - 1) / PVS_SETS * PVS_SETS; // tiles the loops run (padded)
    const int c0 = sl * PVS_COLS, ncol = min(PVS_COLS, HD - c0);
    const float *prow = Pm + ((size_t)t * D.n_heads + h) * s_stride; // p (SM: the scores)
    // the consumer's end: its column's o out, and with a fused quantization
    // the item's arrival (the last of its eight groups quantizes it)
    auto finish = [&](float o) {
        float *dst = att + (size_t)t * D.qd + (size_t)h * HD + c0 + ln;
        if (qwt < 0) {
            if (ln < ncol)
                *dst = o;
        } else {
            if (ln < ncol)
                st_dev(dst, o);
            const int it = (h * HD + c0) / 256;
            if (last_arrival_wave(sync + SYNC_PV_QUANT + t * 64 + it, 256 / PVS_COLS))
                quant_item_wave<true>(qwt, att + (size_t)t * D.qd, D.qd, t, it, qa);
        }
    };
    if (P <= 0) { // a lane at a negative position has no context: +0 out, no
        if (wave == 0) // loads, no softmax; the arrival still counts
            finish(0.0f);
        return;      // (P is uniform over the group: every wave leaves here)
    }

    // ---- the producers' value tiles (declared here: SM issues the first
    // loads before the softmax) ----
    // lane (row group rg, column octet cq): eight columns of four positions,
    // 4 rg + [0, 4) of the producer's 64; a dwordx4 load per position brings
    // the eight values, so each load instruction reads 64 contiguous bytes
    // of 16 rows.  Offsets are 32-bit byte offsets from the layer's
    // (uniform) base, clamped to row P - 1.  p of the lane's four positions
    // is one float4, clamped to the last whole quad holding position P - 1
    // (inside the row: s_stride is a multiple of 64 and at least P).
    static_assert(PP == 64 && PVS_COLS == 32, "lane = (16 row groups of 4 positions, 4 column octets)");
    const bool producer = wave >= 1 && wave <= PVS_NP;
    const int pw = wave - 1, rg = ln & 15, cq = ln >> 4;
    const int cqc = min(cq, ncol / 8 - 1);
    const char *vb0 = (const char *)(vc + (((size_t)t * D.n_layers + li) * D.ctx) * D.kvd + (size_t)kvh * HD);
    const uint32_t rowb = (uint32_t)D.kvd * 2, colb = (uint32_t)(c0 + 8 * cqc) * 2;
    const uint32_t lim = (uint32_t)(P - 1) * rowb + colb;
    const int p4 = (P - 1) & ~3;
    const int r0 = PP * pw + 4 * rg; // first position of this lane within a tile
    uint4 hv[PVS_SETS][4];
    float4 pp[PVS_SETS];
    auto load_v = [&](int tile, uint4 (&v)[4]) {
        const uint32_t o = (uint32_t)(tile * PVS_TJ + r0) * rowb + colb;
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[j] = *(const uint4 *)(vb0 + min(o + (uint32_t)j * rowb, lim));
    };
    float inv = 0.0f;
    if constexpr (SM) {
        // the scores, their max, then the value loads: issued before the max,
        // the loads would be waited for with the scores (the compiler's wait
        // covers every load in flight), and the producers would reach the
        // softmax's first barrier only when their values had landed
        float sv[PVS_SM_VALS];
#pragma unroll
        for (int k = 0; k < PVS_SM_VALS; k++) {
            const int j = threadIdx.x + 64 * NW * k;
            sv[k] = j < P ? prow[j] : -INFINITY;
        }
        // softmax_row_exact's steps: the max (order-free), e_t = exp(s_t - m)
        // zero-filled to whole 64s, 1 / the position-ordered sum
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < PVS_SM_VALS; k++)
            m = fmaxf(m, sv[k]);
        m = wave_max(m);
        if (producer) {
#pragma unroll
            for (int d = 0; d < PVS_SETS; d++)
                load_v(d, hv[d]);
        }
        if (ln == 0)
            redf[wave] = m;
        lds_barrier();
        m = redf[0];
        for (int w = 1; w < NW; w++)
            m = fmaxf(m, redf[w]);
        softmax_exps<64 * NW>(sv, m, P, (P + 63) & ~63, e);
        lds_barrier();
        inv = 1.0f / seq_sum_nonneg<NW>(e, P, seq);
    }
    auto load = [&](int tile, uint4 (&v)[4], float4 &p) {
        load_v(tile, v);
        if constexpr (!SM)
            p = *(const float4 *)(prow + min(tile * PVS_TJ + r0, p4));
    };
    auto pget = [&](int tile, const float4 &p) {
        if constexpr (SM) { // p_t = e_t * inv, the softmax's own expression
            const float4 ev = *(const float4 *)&e[min(tile * PVS_TJ + r0, p4)];
            return make_float4(ev.x * inv, ev.y * inv, ev.z * inv, ev.w * inv);
        } else {
            return p;
        }
    };
    if (wave == 0) { // consumer
        float o = 0.0f;
        lds_barrier(); // tiles 0 and 1 are in
        const int crow = (ln % PVS_COLS) * PVS_STR;
        const float4 *src0 = (const float4 *)&prod[0][crow];
        float4 xr[PVS_AHEAD];
#pragma unroll
        for (int a = 0; a < PVS_AHEAD; a++)
            xr[a] = src0[a];
        for (int k = 0; k < ntp; k++) {
            const int nk = min(PVS_TJ, P - k * PVS_TJ);
            const float4 *nxt = (const float4 *)&prod[(k + 1) % PVS_NBUF][crow];
            if (nk == PVS_TJ) {
                const float4 *src = (const float4 *)&prod[k % PVS_NBUF][crow];
#pragma unroll
                for (int gj = 0; gj < PVS_TJ / 4; gj += 2) {
                    const int a = gj % PVS_AHEAD;
                    // one wait for two groups: the reads of both are the oldest in flight
                    __builtin_amdgcn_s_waitcnt(0xC07F & ~(0xF << 8) | ((PVS_AHEAD - 2) << 8));
                    const float4 x0 = xr[a], x1 = xr[a + 1];
                    __builtin_amdgcn_sched_barrier(0);
                    xr[a] = gj + PVS_AHEAD < PVS_TJ / 4 ? src[gj + PVS_AHEAD] : nxt[gj + PVS_AHEAD - PVS_TJ / 4];
                    __builtin_amdgcn_sched_barrier(0);
                    o = o + x0.x;
                    o = o + x0.y;
                    o = o + x0.z;
                    o = o + x0.w;
                    __builtin_amdgcn_sched_barrier(0);
                    xr[a + 1] = gj + 1 + PVS_AHEAD < PVS_TJ / 4 ? src[gj + 1 + PVS_AHEAD]
                                                                : nxt[gj + 1 + PVS_AHEAD - PVS_TJ / 4];
                    __builtin_amdgcn_sched_barrier(0);
                    o = o + x1.x;
                    o = o + x1.y;
                    o = o + x1.z;
                    o = o + x1.w;
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else if (nk > 0) { // the partial last tile
                const float *src = &prod[k % PVS_NBUF][crow];
                for (int j = 0; j < nk; j++)
                    o = o + src[j];
            }
            // no wait for the reads in flight (the next tile's); the memory
            // clobber keeps every LDS access on its side of the barrier
            __builtin_amdgcn_sched_barrier(0);
            __asm__ volatile("s_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        finish(o);
    } else if (producer) { // producer wave - 1: positions [PP (wave - 1), PP wave) of each tile
        int rw[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            rw[k] = (8 * cq + k) * PVS_STR + r0;
        auto produce = [&](int tile, const uint4 (&v)[4], const float4 &pv) {
            float *dst = prod[tile % PVS_NBUF];
            const float4 q = pget(tile, pv);
            const uint32_t w[4][4] = {{v[0].x, v[0].y, v[0].z, v[0].w},
                                      {v[1].x, v[1].y, v[1].z, v[1].w},
                                      {v[2].x, v[2].y, v[2].z, v[2].w},
                                      {v[3].x, v[3].y, v[3].z, v[3].w}};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int d = k >> 1, sh = 16 * (k & 1);
                float4 a;
                a.x = __builtin_fmaf(q.x, half_bits_to_float(w[0][d] >> sh), 0.0f);
                a.y = __builtin_fmaf(q.y, half_bits_to_float(w[1][d] >> sh), 0.0f);
                a.z = __builtin_fmaf(q.z, half_bits_to_float(w[2][d] >> sh), 0.0f);
                a.w = __builtin_fmaf(q.w, half_bits_to_float(w[3][d] >> sh), 0.0f);
                *(float4 *)&dst[rw[k]] = a;
            }
        };
        if constexpr (!SM) { // SM: the value loads went out before the softmax
#pragma unroll
            for (int d = 0; d < PVS_SETS; d++)
                load(d, hv[d], pp[d]);
        }
        produce(0, hv[0], pp[0]);
        load(PVS_SETS, hv[0], pp[0]);
        produce(1, hv[1], pp[1]);
        load(PVS_SETS + 1, hv[1], pp[1]);
        lds_barrier();
        // iteration k: tile k + 2 into buffer (k + 2) % NBUF from register set
        // (k + 2) % SETS, whose loads went out SETS - 1 tiles ago; then the
        // loads of tile k + 2 + SETS into the same set
        for (int kb = 0; kb < ntp; kb += PVS_SETS) {
#pragma unroll
            for (int d = 0; d < PVS_SETS; d++) {
                const int tile = kb + d + 2, set = (d + 2) % PVS_SETS;
                // pinned in place: products of later tiles hoisted above
                // this barrier would wait for loads meant to stay in flight
                __builtin_amdgcn_sched_barrier(0);
                produce(tile, hv[set], pp[set]);
                load(tile + PVS_SETS, hv[set], pp[set]);
                lds_barrier();
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else { // SM's helper waves: the same barriers as the consumer, nothing else
        lds_barrier();
        for (int k = 0; k < ntp; k++) {
            __builtin_amdgcn_sched_barrier(0);
            __asm__ volatile("s_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

size_t exact_softmax_lds(int s_stride) { return (size_t)s_stride * 4; }

template <int HD>
static void launch_hd(const FrameDims &D, const float *q, const float *k, const float *v, const float *q_norm,
                      const float *k_norm, const float *rope_cs, uint16_t *kc, uint16_t *vc, const int32_t *pos,
                      int li, bool fuse, float *S, int s_stride, float *att, size_t n, int qwt, QAct qa,
                      hipStream_t st) {
    const int n_chunks = (D.ctx + ATT_TC - 1) / ATT_TC;
    const int G = D.n_heads / D.n_kv;
    int ph = prof_begin(LOOMHIP_KT_ATTN_SCORES, st);
    if (!fuse) // the rotated queries and the appended rows come from qk_rope_kernel
        hipLaunchKernelGGL(attn_scores_many_kernel<HD>, dim3((D.ctx + SCM_THREADS - 1) / SCM_THREADS, D.n_kv, n),
                           dim3(SCM_THREADS), 0, st, D, q, kc, pos, li, S, s_stride);
    else
        hipLaunchKernelGGL(attn_scores_kernel<HD>, dim3(n_chunks, D.n_kv, n), dim3(SC_THREADS), 0, st, D, q, k, v,
                           q_norm, k_norm, rope_cs, kc, vc, pos, li, fuse ? 1 : 0, S, s_stride);
    prof_end(ph, st);
    if (n > 4) {
        ph = prof_begin(LOOMHIP_KT_ATTN_SOFTMAX, st);
        hipLaunchKernelGGL((attn_softmax_kernel<512>), dim3(D.n_heads, 1, n), dim3(512), exact_softmax_lds(s_stride),
                           st, D, pos, S, s_stride);
        prof_end(ph, st);
        note_launch();
    }
    ph = prof_begin(LOOMHIP_KT_ATTN_PV, st);
    if (n <= 4) { // the softmax inside the P.V groups
        const dim3 pg(((HD + PVS_COLS - 1) / PVS_COLS) * D.n_heads, 1, n);
        hipLaunchKernelGGL((attn_pv_split_kernel<HD, true>), pg, dim3(64 * PVS_SM_WAVES), pv_softmax_lds(s_stride),
                           st, D, vc, pos, li, S, s_stride, att, qwt, qa, g_ctx.sync);
    } else {
        // one wave per head of the KV group (up to 8 per group)
        const int nw = G >= 8 ? 8 : G >= 4 ? 4 : G >= 2 ? 2 : 1;
        const dim3 pg((HD + 63) / 64, D.n_kv * ((G + nw - 1) / nw), n);
        if (nw == 8)
            hipLaunchKernelGGL((attn_pv_many_kernel<HD, 8>), pg, dim3(512), 0, st, D, vc, pos, li, S, s_stride, att);
        else if (nw == 4)
            hipLaunchKernelGGL((attn_pv_many_kernel<HD, 4>), pg, dim3(256), 0, st, D, vc, pos, li, S, s_stride, att);
        else if (nw == 2)
            hipLaunchKernelGGL((attn_pv_many_kernel<HD, 2>), pg, dim3(128), 0, st, D, vc, pos, li, S, s_stride, att);
        else
            hipLaunchKernelGGL((attn_pv_many_kernel<HD, 1>), pg, dim3(64), 0, st, D, vc, pos, li, S, s_stride, att);
    }
    prof_end(ph, st);
    note_launch();
    note_launch();
}

bool attn_exact_quant_fusable(const FrameDims &D, size_t n) {
    return n <= 4 && (D.hd == 64 || D.hd == 128) && D.qd % 256 == 0 && D.qd / 256 <= 64;
}

bool launch_attn_exact(const FrameDims &D, const float *q, const float *k, const float *v, const float *q_norm,
                       const float *k_norm, const float *rope_cs, uint16_t *kc, uint16_t *vc, const int32_t *pos,
                       int li, bool fuse, float *S, int s_stride, float *att, size_t n, int qwt, const QAct &qa,
                       hipStream_t st) {
    if (D.ctx > EXACT_MAX_CTX || s_stride % 64 || s_stride < D.ctx)
        return false;
    if (qwt >= 0 && !attn_exact_quant_fusable(D, n))
        return false;
    switch (D.hd) {
    case 128:
        launch_hd<128>(D, q, k, v, q_norm, k_norm, rope_cs, kc, vc, pos, li, fuse, S, s_stride, att, n, qwt, qa, st);
        return true;
    case 64:
        launch_hd<64>(D, q, k, v, q_norm, k_norm, rope_cs, kc, vc, pos, li, fuse, S, s_stride, att, n, qwt, qa, st);
        return true;
    case 48:
        launch_hd<48>(D, q, k, v, q_norm, k_norm, rope_cs, kc, vc, pos, li, fuse, S, s_stride, att, n, qwt, qa, st);
        return true;
    default:
        return false;
    }
}

} // namespace lh
