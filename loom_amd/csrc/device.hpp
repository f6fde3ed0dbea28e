// device.hpp -- device-side helpers shared by the kernel files: the int8
// activation quantizers (one wave per item) and the completion counters that
// let the last workgroup of a set run an epilogue.
#pragma once

#include "kernels.hpp"

namespace lh {

constexpr int MAX_E = 256, MAX_K = 16, MAX_TOK = 256; // routing limits

// ---- exact dequant of one value from the device layout ------------------------
// f32 arithmetic in the reference's two-rounding form (src/gguf/ggml.zig:
// 1342-1374 Q4_K, 1420-1471 Q6_K, 1834-1849 Q4_0/Q8_0); value (r, c) of a
// rows x cols matrix.
// Every value of these formats is a * q - b with an integer q and one f32
// pair (a, b) per scale group of a block: Q4_K a = d*sc, b = dmin*m (32
// values per group), Q6_K a = d*sc, q = qv - 32, b = 0 (16 per group), Q8_0
// and Q4_0 a = d, b = 0 (the block).  a * q rounds once and - b once: the
// reference's two roundings ((d*sc)*q - dmin*m; s*(q-32); q*d), and - 0
// leaves every value (-0 included) as it is.

// Scale group of value e within its block.
__device__ inline int dq_group(int t, int e) {
    if (t == LH_Q4_K)
        return e / 32;
    if (t == LH_Q6_K)
        return 8 * (e / 128) + (e % 32) / 16 + 2 * ((e % 128) / 32);
    return 0;
}

// Groups per block.
__host__ __device__ inline constexpr int dq_groups(int t) { return t == LH_Q4_K ? 8 : t == LH_Q6_K ? 16 : 1; }

// The integer q of value e of block `unit` of a plane of U blocks (device layout).
__device__ inline int dq_q(int t, const uint8_t *__restrict__ w, size_t U, size_t unit, int e) {
    if (t == LH_Q4_K) {
        const int g = e / 32, l = e % 32;
        const uint8_t byte = w[unit * 144 + 16 + 32 * (g / 2) + l];
        return (g & 1) ? (byte >> 4) : (byte & 0xF);
    }
    if (t == LH_Q6_K) {
        const int h = e / 128, r128 = e % 128, quarter = r128 / 32, l = r128 % 32;
        const uint8_t qlb = w[unit * 128 + 64 * h + l + ((quarter & 1) ? 32 : 0)];
        const uint8_t qhb = w[U * 128 + unit * 64 + 32 * h + l];
        const int nib = (quarter < 2) ? (qlb & 0xF) : (qlb >> 4);
        return (nib | (((qhb >> (2 * quarter)) & 3) << 4)) - 32;
    }
    if (t == LH_Q8_0)
        return ((const int8_t *)w)[unit * 32 + e];
    if (t == LH_Q4_0) {
        const uint8_t *qs = w + unit * 16;
        return (e < 16 ? (qs[e] & 0xF) : (qs[e - 16] >> 4)) - 8;
    }
    return 0;
}

// The pair (a, b) of scale group g of block `unit`.
__device__ inline float2 dq_pair(int t, const uint8_t *__restrict__ w, size_t U, size_t unit, int g) {
    if (t == LH_Q4_K) {
        const uint8_t *blk = w + unit * 144;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
        const uint8_t *s = blk + 4;
        int sc, m;
        if (g < 4) {
            sc = s[g] & 63;
            m = s[g + 4] & 63;
        } else {
            sc = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4);
            m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
        }
        return make_float2(d * (float)sc, dmin * (float)m);
    }
    if (t == LH_Q6_K) {
        const int8_t *sc = (const int8_t *)(w + U * 192 + unit * 16);
        const float d = half_bits_to_float(((const uint16_t *)(w + U * 208))[unit]);
        return make_float2(d * (float)sc[g], 0.0f);
    }
    if (t == LH_Q8_0)
        return make_float2(half_bits_to_float(((const uint16_t *)(w + U * 32))[unit]), 0.0f);
    if (t == LH_Q4_0)
        return make_float2(half_bits_to_float(((const uint16_t *)(w + U * 16))[unit]), 0.0f);
    return make_float2(0.0f, 0.0f);
}

__device__ inline float dq_apply(float2 ab, int q) {
    const float v = ab.x * (float)q;
    return v - ab.y;
}

// Value e of block `unit` of a quantized plane of U blocks (device layout).
__device__ inline float dequant_unit(int t, const uint8_t *__restrict__ w, size_t U, size_t unit, int e) {
    return dq_apply(dq_pair(t, w, U, unit, dq_group(t, e)), dq_q(t, w, U, unit, e));
}

__device__ inline float dequant_value(int t, const uint8_t *__restrict__ w, size_t rows, size_t cols,
                                      size_t r, size_t c) {
    if (t == LH_F16)
        return half_bits_to_float(((const uint16_t *)w)[r * cols + c]);
    if (t == LH_F32)
        return ((const float *)w)[r * cols + c];
    const int be = block_elems(t);
    const size_t nb = cols / be;
    return dequant_unit(t, w, rows * nb, r * nb + c / be, (int)(c % be));
}

// ---- wave-level int8 activation quantizers ------------------------------------

// Four consecutive floats; COHERENT reads them through relaxed agent-scope
// atomic loads (values written by other work groups of the same launch).
template <bool COHERENT = false>
__device__ inline float4 load4(const float *x) {
    if constexpr (COHERENT) {
        float4 v;
        v.x = __hip_atomic_load(const_cast<float *>(x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v.y = __hip_atomic_load(const_cast<float *>(x + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v.z = __hip_atomic_load(const_cast<float *>(x + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v.w = __hip_atomic_load(const_cast<float *>(x + 3), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return v;
    } else {
        return *(const float4 *)x;
    }
}

// quantizeX256 (src/gguf/ggml.zig:776-800) of one 256-value block by one
// wave whose values 4l..4l+3 are already in lane l: amax is an exact max
// (order-free), the per-16 sums are integer.
__device__ inline void quant256_regs(const float4 xv, int8_t *__restrict__ q,
                                     float *__restrict__ d, int32_t *__restrict__ s) {
    const int lane = threadIdx.x & 63;
    float a = 0.0f;
    if (__builtin_isfinite(xv.x)) a = fmaxf(a, fabsf(xv.x));
    if (__builtin_isfinite(xv.y)) a = fmaxf(a, fabsf(xv.y));
    if (__builtin_isfinite(xv.z)) a = fmaxf(a, fabsf(xv.z));
    if (__builtin_isfinite(xv.w)) a = fmaxf(a, fabsf(xv.w));
    const float amax = wave_max(a);
    const float dd = amax / 127.0f;
    const float inv = (dd != 0.0f && __builtin_isfinite(dd)) ? 1.0f / dd : 0.0f;
    const int q0 = to_i8_sat(xv.x * inv), q1 = to_i8_sat(xv.y * inv);
    const int q2 = to_i8_sat(xv.z * inv), q3 = to_i8_sat(xv.w * inv);
    const uint32_t packed = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                            ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
    *(uint32_t *)(q + 4 * lane) = packed;
    const int sum16 = group_sum<4>(q0 + q1 + q2 + q3);
    if ((lane & 3) == 0)
        s[lane / 4] = sum16;
    if (lane == 0)
        *d = __builtin_isfinite(dd) ? dd : 0.0f;
}

template <bool COHERENT = false>
__device__ inline void quant_block256_wave(const float *__restrict__ x, int8_t *__restrict__ q,
                                           float *__restrict__ d, int32_t *__restrict__ s) {
    quant256_regs(load4<COHERENT>(x + 4 * (threadIdx.x & 63)), q, d, s);
}

// Lane l's four values of the quantizeX item starting at block b0.
__device__ inline const float *blocks32_src(const float *x, int nb, int b0) {
    const int lane = threadIdx.x & 63;
    const int blk = b0 + lane / 8;
    const int bc = blk < nb ? blk : nb - 1; // idle lanes read a valid block
    return x + bc * 32 + 4 * (lane & 7);
}

// quantizeX (src/gguf/ggml.zig:1077-1098) of up to eight 32-value blocks
// [b0, b0+8) of one vector by one wave, eight lanes per block, values
// already in the lanes (lane l holds values 4(l%8).. of block b0 + l/8).
__device__ inline void quant32x8_regs(const float4 xv, int nb, int b0, int8_t *__restrict__ q,
                                      float *__restrict__ d, int32_t *__restrict__ s) {
    const int lane = threadIdx.x & 63;
    const int blk = b0 + lane / 8;
    const bool live = blk < nb;
    float a = 0.0f;
    if (__builtin_isfinite(xv.x)) a = fmaxf(a, fabsf(xv.x));
    if (__builtin_isfinite(xv.y)) a = fmaxf(a, fabsf(xv.y));
    if (__builtin_isfinite(xv.z)) a = fmaxf(a, fabsf(xv.z));
    if (__builtin_isfinite(xv.w)) a = fmaxf(a, fabsf(xv.w));
    a = group8_max(a);
    const float dd = a / 127.0f;
    const float inv = (dd != 0.0f && __builtin_isfinite(dd)) ? 1.0f / dd : 0.0f;
    const int q0 = to_i8_sat(xv.x * inv), q1 = to_i8_sat(xv.y * inv);
    const int q2 = to_i8_sat(xv.z * inv), q3 = to_i8_sat(xv.w * inv);
    const int sum = group_sum<8>(q0 + q1 + q2 + q3);
    if (live) {
        const uint32_t packed = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
        *(uint32_t *)(q + blk * 32 + 4 * (lane & 7)) = packed;
        if ((lane & 7) == 0) {
            s[blk] = sum;
            d[blk] = __builtin_isfinite(dd) ? dd : 0.0f;
        }
    }
}

template <bool COHERENT = false>
__device__ inline void quant_blocks32_wave(const float *__restrict__ x, int nb, int b0,
                                           int8_t *__restrict__ q, float *__restrict__ d,
                                           int32_t *__restrict__ s) {
    quant32x8_regs(load4<COHERENT>(blocks32_src(x, nb, b0)), nb, b0, q, d, s);
}

// quantizeX (QB = 32, src/gguf/ggml.zig:1077-1098) or quantizeX256 (QB =
// 256, ggml.zig:776-800) with each lane owning one 32-value chunk c of a
// buffer of such chunks (v[0..8) its 32 values in order); for QB = 256 the
// eight lanes 8g..8g+7 hold one block's chunks and share its amax.  Writes q
// [32c, 32c+32), the per-16 sums (QB = 256: s[2c], s[2c+1]) or the block sum
// (QB = 32: s[c]) and the block scale d, for live lanes.  All lanes of the
// wave take part (QB = 256 reduces across lanes).
template <int QB>
__device__ inline void quant_chunk32(const float4 (&v)[8], bool live, int c, int8_t *__restrict__ q,
                                     float *__restrict__ d, int32_t *__restrict__ s) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        if (__builtin_isfinite(v[i].x)) a = fmaxf(a, fabsf(v[i].x));
        if (__builtin_isfinite(v[i].y)) a = fmaxf(a, fabsf(v[i].y));
        if (__builtin_isfinite(v[i].z)) a = fmaxf(a, fabsf(v[i].z));
        if (__builtin_isfinite(v[i].w)) a = fmaxf(a, fabsf(v[i].w));
    }
    if constexpr (QB == 256)
        a = group8_max(a);
    const float dd = a / 127.0f;
    const float inv = (dd != 0.0f && __builtin_isfinite(dd)) ? 1.0f / dd : 0.0f;
    uint32_t packed[8];
    int sum[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int q0 = to_i8_sat(v[i].x * inv), q1 = to_i8_sat(v[i].y * inv);
        const int q2 = to_i8_sat(v[i].z * inv), q3 = to_i8_sat(v[i].w * inv);
        packed[i] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                    ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
        sum[i >> 2] += q0 + q1 + q2 + q3;
    }
    if (!live)
        return;
    *(uint4 *)(q + 32 * c) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    *(uint4 *)(q + 32 * c + 16) = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    const float dv = __builtin_isfinite(dd) ? dd : 0.0f;
    if constexpr (QB == 256) {
        s[2 * c] = sum[0];
        s[2 * c + 1] = sum[1];
        if ((c & 7) == 0)
            d[c >> 3] = dv;
    } else {
        s[c] = sum[0] + sum[1];
        d[c] = dv;
    }
}

// Work items of quantizing one vector of `cols` values for weight type wt:
// one 256-block (K-quants) or eight 32-blocks per item.
__host__ __device__ inline int quant_items(int wt, int cols) {
    return act_block(wt) == 256 ? cols / 256 : (cols / 32 + 7) / 8;
}

// Quantize item `it` of vector v (x at x + v*x_stride) into qa.  COHERENT
// reads x through ld_dev (x was written by other workgroups of this launch).
template <bool COHERENT = false>
__device__ inline void quant_item_wave(int wt, const float *x, int cols, int v, int it, QAct qa) {
    if (act_block(wt) == 256) {
        const int nb = cols / 256;
        quant_block256_wave<COHERENT>(x + it * 256, qa.q + (size_t)v * cols + it * 256,
                            qa.d + (size_t)v * nb + it, qa.s + (size_t)v * (cols / 16) + it * 16);
    } else {
        const int nb = cols / 32;
        quant_blocks32_wave<COHERENT>(x, nb, it * 8, qa.q + (size_t)v * cols, qa.d + (size_t)v * nb,
                            qa.s + (size_t)v * nb);
    }
}

// LDS-only barrier: waits for this wave's LDS traffic, not for its global
// loads, so weight loads issued before it stay in flight.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0); vmcnt and expcnt left open
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- completion counters ----------------------------------------------------------
// Offsets (ints) inside the library's zero-initialised sync buffer.  Every
// counter is reset to zero by the arrival that completes it, so the buffer
// is all zeros between launches.
constexpr int SYNC_GATE_CHUNK = 0;   // [MAX_TOK / GT_TOK]: a counter per token chunk
constexpr int SYNC_GATE_FINAL = 128; // [1]
constexpr int SYNC_PV_QUANT = 256;   // [4 lanes][64 items]: P.V groups of one 256-column item
//
// Data handed from one workgroup to another inside a launch travels through
// relaxed agent-scope atomic stores and loads (st_dev / ld_dev), which are
// coherent per location across the chip's XCDs (each XCD has its own L2).
// An agent-scope fence would instead write back the whole L2 of the XCD,
// which costs far more than the data (about 0.7 us per workgroup, serialised
// per XCD).  Ordering: each arriving workgroup waits until all its stores
// are acknowledged (s_waitcnt 0) before the counter increment, and the last
// arrival issues its loads only after reading the counter.

__device__ inline void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_dev(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_dev(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld_dev(const uint32_t *p) {
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline bool last_arrival(int *counter, int target) {
    __shared__ int s_last;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0); // this thread's stores are acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == target - 1;
        if (s_last) // every arrival is in: reset for the next launch
            __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return s_last;
}

// The same for one wave: the calling wave alone has stored the data (all its
// lanes active); lane 0 counts, and every lane gets the verdict.
__device__ inline bool last_arrival_wave(int *counter, int target) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0); // this wave's stores are acknowledged
    int last = 0;
    if ((threadIdx.x & 63) == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == target - 1;
        if (last)
            __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return __builtin_amdgcn_readfirstlane(last) != 0;
}

// ---- routing ------------------------------------------------------------------------

// ---- routing (src/gguf/moe.zig:106-158) ----------------------------------------------
//
// The reference picks k experts by k rounds of argmax with strict '>' over
// the unused experts' selection values (scores + selection bias): lowest
// index wins ties, and a round that finds nothing above -inf picks expert 0.
// That is the order (value descending, index ascending) over values above
// -inf, so an expert's slot is its rank in that order.  With
// key = (ordered value << 31) | (0x7FFFFFFF - index) every key is distinct
// and rank = #{keys greater}.  Keys stay below 2^63, so "k_j > k_i" is the
// sign bit of k_i - k_j: the comparisons are 64-bit adds of negated keys
// and shifts, with no compare results to serialise on.
//
// For softmax gating without a selection bias the ranks are taken on the
// exp values e = exp(l - max) before the sequential sum: scores p = e * inv
// are a non-decreasing function of e, so the order can only differ where
// two different e round to the same p.  route_finish checks exactly that
// (adjacent ranks 0..k with equal p) once the sum is known, off the critical
// path, and asks for route_exact when it happens; ids stay bit-exact.

template <int NW>
struct __align__(16) RouteLds {
    unsigned long long nkey[NW][MAX_E]; // per-wave copy of the negated selection keys
    int prank[NW][MAX_E];               // partial ranks (NW > 1)
    float sc[MAX_E];                   // softmax exp values, for the sequential sum
    int id[MAX_K + 1];                 // slot -> expert (slot k: the next one)
    float val[MAX_K + 1];              // slot -> unbiased score (softmax: exp value)
    int n_valid;
    int redo; // set by the caller when route_finish asks for route_exact_wave
};

// Sequential f32 sum of lane s's value over s < K, uniform in every lane.
__device__ __forceinline__ float slot_sum(float v, int K) {
    float sum = 0.0f;
    for (int s = 0; s < K; s++)
        sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), s));
    return sum;
}

// Order-preserving map of an f32 onto u32 (larger value -> larger key).
__device__ __forceinline__ uint32_t ordered_u32(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// 63-bit key: the value's order in bits 62..31 (-0 folded into +0: the
// reference's '>' sees them equal), 0x7FFFFFFF - index below.  Valid keys
// are >= 2^54; invalid ones are 0.
__device__ __forceinline__ unsigned long long route_key(float c, int e, bool valid) {
    return valid ? ((unsigned long long)ordered_u32(c + 0.0f) << 31) | (0x7FFFFFFFu - (uint32_t)e) : 0ull;
}

// Sequential sum of v[0..E) in LDS (the reference's softmax sum order); the
// reads of each 32-value batch are issued before its adds.
__device__ __forceinline__ float lds_seq_sum(const float *v, int E) {
    // unconditional over whole batches of 32: the entries past E are +0
    // (exp(-inf - max)) and the running sum of exp values is never -0, so
    // adding them changes nothing
    float sum = 0.0f;
    for (int e0 = 0; e0 < E; e0 += 32) {
        float4 r[8];
#pragma unroll
        for (int q = 0; q < 8; q++)
            r[q] = *(const float4 *)(v + e0 + 4 * q);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            sum = sum + r[q].x;
            sum = sum + r[q].y;
            sum = sum + r[q].z;
            sum = sum + r[q].w;
        }
    }
    return sum;
}

// rank[i] = #{keys of [j0, j1) greater than key[i]} for i < ni, from the
// negated keys nk: each read once for all of the lane's experts; a key k_j
// counts when the sign bit of key[i] + nk_j = key[i] - k_j is set.
template <int NI>
__device__ __forceinline__ void count_greater(const unsigned long long *nk, int j0, int j1,
                                              const unsigned long long (&key)[NI], int ni,
                                              int (&rank)[NI]) {
    int r[NI];
#pragma unroll
    for (int i = 0; i < NI; i++)
        r[i] = 0;
    for (int j = j0; j < j1; j += 16) {
        ulonglong2 kk[8];
#pragma unroll
        for (int q = 0; q < 8; q++)
            kk[q] = *(const ulonglong2 *)(nk + j + 2 * q);
#pragma unroll
        for (int i = 0; i < NI; i++) {
            if (i < ni) {
#pragma unroll
                for (int q = 0; q < 8; q++)
                    r[i] += (int)((uint32_t)((key[i] + kk[q].x) >> 32) >> 31) +
                            (int)((uint32_t)((key[i] + kk[q].y) >> 32) >> 31);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NI; i++)
        rank[i] = r[i];
}

// Rank the experts' keys (key[i] for expert lane + 64i) and write the slot
// table.  SINGLE: one wave does it all (index 0 of L's per-wave arrays);
// otherwise NW waves split the comparisons, each holding every expert's key.
// Ends with the participating waves seeing L.id / L.val / L.n_valid.
template <int NW, bool SINGLE>
__device__ __forceinline__ void route_slots(const unsigned long long (&key)[MAX_E / 64],
                                   const float (&val)[MAX_E / 64], int valid_n, int E, int K,
                                   RouteLds<NW> &L) {
    constexpr int NI = MAX_E / 64;
    constexpr bool ONE = SINGLE || NW == 1;
    const int lane = threadIdx.x & 63, w = ONE ? 0 : threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < NI; i++)
        L.nkey[w][lane + 64 * i] = 0ull - key[i];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int Epad = (E + 15) & ~15; // keys past E are 0 and never count
    const int ch = ONE ? Epad : (((Epad / NW) + 15) & ~15);
    const int j0 = w * ch, j1 = min(Epad, j0 + ch);
    int rank[NI];
    count_greater<NI>(L.nkey[w], j0, j1, key, (E + 63) / 64, rank);
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            L.prank[w][lane + 64 * i] = rank[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NI; i++) {
            int r = 0;
#pragma unroll
            for (int v = 0; v < NW; v++)
                r += L.prank[v][lane + 64 * i];
            rank[i] = r;
        }
    }
    if (w == 0) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            if (key[i] != 0ull && rank[i] <= K) {
                L.id[rank[i]] = lane + 64 * i;
                L.val[rank[i]] = val[i];
            }
        // rounds that found nothing above -inf pick expert 0 (its unbiased score)
        const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val[0]), 0));
        if (lane >= valid_n && lane < K) {
            L.id[lane] = 0;
            L.val[lane] = v0;
        }
        if (lane == 0)
            L.n_valid = valid_n;
    }
    if constexpr (ONE) {
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    } else {
        __syncthreads();
    }
}

// Exact routing by one wave, in the reference's arithmetic: scores
// (sigmoid / softmax with the sequential sum / raw logits), selection values
// scores + bias, ranks.  Fills the slot table with the unbiased scores.
template <int NW, bool COHERENT>
__device__ __forceinline__ void route_exact_wave(const float *lg, const float *sel_bias, int E, int K,
                                        int gating, RouteLds<NW> &L) {
    constexpr int NI = MAX_E / 64;
    const int lane = threadIdx.x & 63;
    float sv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int e = lane + 64 * i;
        sv[i] = e < E ? (COHERENT ? ld_dev(lg + e) : lg[e]) : -INFINITY;
    }
    if (gating == 2) { // sigmoid (tensor.zig:34-36)
#pragma unroll
        for (int i = 0; i < NI; i++)
            sv[i] = 1.0f / (1.0f + exp_f32(-sv[i]));
    } else if (gating != 3) { // softmax (tensor.zig:18-28)
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NI; i++)
            m = fmaxf(m, sv[i]);
        m = wave_max(m);
#pragma unroll
        for (int i = 0; i < NI; i++) {
            sv[i] = exp_f32(sv[i] - m);
            L.sc[lane + 64 * i] = sv[i];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const float inv = 1.0f / lds_seq_sum(L.sc, E);
#pragma unroll
        for (int i = 0; i < NI; i++)
            sv[i] = sv[i] * inv;
    }
    unsigned long long key[NI];
    int valid_n = 0;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int e = lane + 64 * i;
        const float c = e < E ? (sel_bias ? sv[i] + sel_bias[e] : sv[i]) : -INFINITY;
        const bool valid = c > -INFINITY; // NaN and -inf never win a strict '>'
        key[i] = route_key(c, e, valid);
        valid_n += __popcll(__ballot(valid));
    }
    route_slots<NW, true>(key, sv, valid_n, E, K, L);
}

// Selection of one token by NW cooperating waves (threads [0, 64*NW)); the
// waves hold identical copies of every expert's values.  Returns with the
// slot table filled.  For softmax without a selection bias the table holds
// exp values and ranks on them (route_finish settles exactness); otherwise
// it is exact already.
__device__ __forceinline__ bool route_is_exact(int gating, const float *sel_bias) {
    return gating == 2 || gating == 3 || sel_bias != nullptr;
}

template <int NW, bool COHERENT>
__device__ __forceinline__ void route_rank(const float *lg, const float *sel_bias, int E, int K, int gating,
                                  RouteLds<NW> &L) {
    constexpr int NI = MAX_E / 64;
    const int lane = threadIdx.x & 63;
    if (gating != 2 && gating != 3 && sel_bias) { // softmax + selection bias: exact only
        if (NW == 1 || (int)threadIdx.x < 64)
            route_exact_wave<NW, COHERENT>(lg, sel_bias, E, K, gating, L);
        if constexpr (NW > 1)
            __syncthreads();
        return;
    }
    // logits and selection biases: unconditional loads (indices clamped) all
    // issued before the first use, then the entries past E masked
    float lv[NI], bv[NI], val[NI];
    const float *bsrc = sel_bias ? sel_bias : lg; // read either way, used with a bias only
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int e = min(lane + 64 * i, E - 1);
        lv[i] = COHERENT ? ld_dev(lg + e) : lg[e];
        bv[i] = bsrc[e];
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        lv[i] = lane + 64 * i < E ? lv[i] : -INFINITY;
        asm volatile("" ::"v"(bv[i])); // keeps the bias loads here, beside the logits
    }
    unsigned long long key[NI];
    int valid_n = 0;
    if (gating == 2 || gating == 3) { // sigmoid / softmax_topk: exact selection values
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int e = lane + 64 * i;
            val[i] = gating == 2 ? 1.0f / (1.0f + exp_f32(-lv[i])) : lv[i];
            const float c = e < E ? (sel_bias ? val[i] + bv[i] : val[i]) : -INFINITY;
            const bool valid = c > -INFINITY;
            key[i] = route_key(c, e, valid);
            valid_n += __popcll(__ballot(valid));
        }
    } else { // softmax: rank on e = exp(l - max)
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NI; i++)
            m = fmaxf(m, lv[i]);
        m = wave_max(m);
        bool any_nan = false;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            val[i] = exp_f32(lv[i] - m);
            if (lane + 64 * i < E)
                any_nan |= __builtin_isnan(val[i]);
            if (NW == 1 || (int)threadIdx.x < 64) // the copy route_finish sums
                L.sc[lane + 64 * i] = val[i];
        }
        // a NaN among the exp values makes the sum, and so every score, NaN:
        // nothing is selectable
        const bool none = __ballot(any_nan) != 0;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int e = lane + 64 * i;
            const bool valid = !none && e < E;
            key[i] = route_key(val[i], e, valid);
            valid_n += __popcll(__ballot(valid));
        }
    }
    route_slots<NW, false>(key, val, valid_n, E, K, L);
}

// Gate post-processing in slot order (moe.zig:143-157), lane s < K holding
// slot s's unbiased score: softmax over the k for softmax_topk, renorm with
// the f16-min clamp, scale.  Returns lane s's final gate.
// Routing for one (token, slot s) work group of the decode path (4 waves,
// NI = ceil(E/64)): every wave builds the token's keys, the waves split the
// rank counting, and slot s's expert is the one whose rank is s (a ballot;
// no slot table).  Softmax ranks on exp(l - max): two experts can come out
// in the other order only when their exp values round to the same final
// score, the near-tie case the reference's tests allow; the gates are
// computed exactly elsewhere.  Softmax with a selection bias goes through
// route_rank (exact scores).  ids, when given, receives the token's k ids
// (wave 0).  Rounds that find nothing above -inf pick expert 0.
template <int NI>
__device__ __forceinline__ int route_decode_slot(const float *lg, const float *sel_bias, int E, int K,
                                                 int gating, int s, RouteLds<4> &L, uint32_t *ids) {
    constexpr int NW = 4;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (gating != 2 && gating != 3 && sel_bias) {
        route_rank<NW, false>(lg, sel_bias, E, K, gating, L);
        if (ids && (int)threadIdx.x < K)
            ids[threadIdx.x] = (uint32_t)L.id[threadIdx.x];
        return L.id[s];
    }
    // logits and selection biases: unconditional loads (indices clamped)
    // all issued before the first use, then the entries past E masked
    float lv[NI], bv[NI];
    const float *bsrc = sel_bias ? sel_bias : lg; // read either way, used with a bias only
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int e = min(lane + 64 * i, E - 1);
        lv[i] = lg[e];
        bv[i] = bsrc[e];
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        lv[i] = lane + 64 * i < E ? lv[i] : -INFINITY;
        asm volatile("" ::"v"(bv[i])); // keeps the bias loads here, beside the logits
    }
    unsigned long long key[NI];
    int valid_n = 0;
    if (gating == 2 || gating == 3) { // sigmoid / softmax_topk: exact selection values
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int e = lane + 64 * i;
            const float val = gating == 2 ? 1.0f / (1.0f + exp_f32(-lv[i])) : lv[i];
            const float c = e < E ? (sel_bias ? val + bv[i] : val) : -INFINITY;
            const bool valid = c > -INFINITY;
            key[i] = route_key(c, e, valid);
            valid_n += __popcll(__ballot(valid));
        }
    } else { // softmax: rank on exp(l - max)
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NI; i++)
            m = fmaxf(m, lv[i]);
        m = wave_max(m);
        float val[NI];
        bool any_nan = false;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            val[i] = exp_f32(lv[i] - m);
            any_nan |= lane + 64 * i < E && __builtin_isnan(val[i]);
        }
        // a NaN among the exp values makes the sum, and so every score, NaN:
        // nothing is selectable
        const bool none = __ballot(any_nan) != 0;
#pragma unroll
        for (int i = 0; i < NI; i++)
            key[i] = route_key(val[i], lane + 64 * i, !none && lane + 64 * i < E);
        valid_n = none ? 0 : E;
    }
#pragma unroll
    for (int i = 0; i < NI; i++)
        L.nkey[w][lane + 64 * i] = 0ull - key[i];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int Epad = (E + 15) & ~15; // keys past E are 0 and never count
    const int ch = ((Epad / NW) + 15) & ~15;
    const int j0 = w * ch, j1 = min(Epad, j0 + ch);
    int rank[NI];
    count_greater<NI>(L.nkey[w], j0, j1, key, NI, rank);
#pragma unroll
    for (int i = 0; i < NI; i++)
        L.prank[w][lane + 64 * i] = rank[i];
    __syncthreads();
    int e = 0;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        int r = 0;
#pragma unroll
        for (int v = 0; v < NW; v++)
            r += L.prank[v][lane + 64 * i];
        rank[i] = r;
        const unsigned long long hit = __ballot(key[i] != 0ull && r == s);
        if (hit)
            e = 64 * i + (int)__builtin_ctzll(hit);
    }
    if (s >= valid_n)
        e = 0;
    if (ids && w == 0) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            if (key[i] != 0ull && rank[i] < K)
                ids[rank[i]] = (uint32_t)(lane + 64 * i);
        if (lane >= valid_n && lane < K)
            ids[lane] = 0;
    }
    return e;
}

__device__ __forceinline__ float gates_post(float g, int K, int gating, int weights_norm,
                                            float weights_scale) {
    if (gating == 3) {
        float m = -INFINITY;
        for (int s = 0; s < K; s++)
            m = fmaxf(m, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), s)));
        g = exp_f32(g - m);
        const float inv = 1.0f / slot_sum(g, K);
        g = g * inv;
    }
    if (weights_norm) {
        const float denom = fmaxf(slot_sum(g, K), 6.103515625e-5f);
        g = g / denom;
    }
    if (weights_scale != 1.0f)
        g = g * weights_scale;
    return g;
}

// Gates of the slots (moe.zig:143-157) by one wave after route_rank: softmax
// scores p = e / sum (redo = true, uniformly, when two adjacent ranks 0..k
// have equal p from different e: the caller then reroutes with
// route_exact_wave and calls this again with exact = true), softmax over the
// k for softmax_topk, renorm with the f16-min clamp, scale.  Lane s < K
// returns slot s's gate.  exact: the slot table holds final scores.
template <int NW>
__device__ __forceinline__ float route_finish(RouteLds<NW> &L, int E, int K, int gating, bool exact,
                                     int weights_norm, float weights_scale, bool &redo) {
    const int lane = threadIdx.x & 63;
    float g = lane < K ? L.val[lane] : 0.0f;
    redo = false;
    if (!exact && gating != 2 && gating != 3) {
        const float inv = 1.0f / lds_seq_sum(L.sc, E);
        const float pl = lane <= K ? L.val[lane] * inv : 0.0f;
        // adjacent ranks s, s+1 (both selectable) with equal p from different e
        const float pn = __shfl_down(pl, 1, 64);
        const float en = __shfl_down(lane <= K ? L.val[lane] : 0.0f, 1, 64);
        const float el = lane <= K ? L.val[lane] : 0.0f;
        const bool tie = lane < K && lane + 1 < L.n_valid && pl == pn && el != en;
        redo = __ballot(tie) != 0;
        g = lane < K ? pl : 0.0f;
    }
    return gates_post(g, K, gating, weights_norm, weights_scale);
}

} // namespace lh
