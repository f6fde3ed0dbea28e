// mmq.hip -- grouped int8 matrix-core matmul for Q4_K / Q6_K (and, from the
// 32-value-block section below, Q8_0 / Q4_0) weights against int8
// activations, bit-identical to the reference CPU kernels
// (src/gguf/ggml.zig:1002-1059 kBlockDot / matvecK256 / matmulK256,
// 1196-1222 matvecQ40Int, 1277-1294 matvecQ80Int) and so to dmmv.hip.
//
// The integer part of every block dot runs on the int8 MFMAs: the activations
// of 16 tokens are the A rows, 16 weight rows the B columns (Q4_K:
// v_mfma_i32_16x16x64_i8 over a 64-value quant span; Q6_K: the same MFMA
// over four 16-value runs, one run per MFMA).  Integer dots are exact in
// any order, so isum = sum sc * dot and msum = sum mn * bsum are the
// reference's integers; the f32 tail per (token, row, super-block) is the
// reference's expression, and each output sums its blocks in block order
// from LDS.
//
// Lane l of a wave: weight row l % 16 of its 16-row tile, k-quarter l / 16;
// the result lane l holds tokens 4*(l/16) .. +3 of that row.
#include <type_traits>

#include "device.hpp"
#include "fmt.hpp"
#include "kernels.hpp"

namespace lh {

typedef int mmq_i4 __attribute__((ext_vector_type(4)));

constexpr uint64_t NIB = 0x0F0F0F0F0F0F0F0Full;

// One wave computes one (16-row tile, super-block) for 16*MT tokens.  Every
// global load of the wave (weights, activation rows, activation scales) is
// issued before its first MFMA, so a wave costs one memory round trip.
//
// Q4_K: isum = sum_g sc[g] * dot(q_g, x_g) from one MFMA per 32-value group;
// the mins' integer sum_g mn[g] * sum(x_g) is one chained MFMA per group
// against mn[g] replicated over the group's bytes (mn <= 63 fits int8).
// Q6_K: the weights enter the MFMA as q - 32 (-32..31 fits int8), so
// isum = sum_run sc[run] * dot(q - 32, x) -- the reference's
// sum sc * (dot(q, x) - 32 * sum(x)) as one exact integer.  A 32-value group
// spans two 16-value runs with their own scales: one MFMA per run, the other
// run's lanes zeroed.

// Q4_K on v_mfma_i32_16x16x64_i8: one MFMA spans the 64 values of a 32-byte
// quant span p (groups 2p and 2p+1).  Lane quarter q4 holds 16 contiguous
// values, [64p + 16*q4, +16): quarters 0-1 lie in group 2p (low nibbles of
// the span's bytes), 2-3 in group 2p+1 (high nibbles), so both the
// activation and the weight loads are 16 contiguous bytes per lane.  The
// group sums come from two MFMAs, each with the other group's quarters of
// the weights zeroed; the mins' sum is one chained MFMA per span against
// each quarter's group min replicated.
struct Q4kTile {
    uint4 hdr;
    uint4 qs[4]; // span p's 16 bytes for this lane's quarter
};

__device__ __forceinline__ Q4kTile q4k_load(const uint8_t *blk, int q4) {
    Q4kTile w;
    w.hdr = *(const uint4 *)blk;
#pragma unroll
    for (int p = 0; p < 4; p++)
        w.qs[p] = *(const uint4 *)(blk + 16 + 32 * p + 16 * (q4 & 1));
    return w;
}

template <int MT>
__device__ __forceinline__ void q4k_tile(const Q4kTile &w, int q4, const mmq_i4 (&xa)[MT][4],
                                         const float (&xd)[MT][4], float (&r)[MT][4]) {
    int sc[8], mn[8];
#pragma unroll
    for (int p = 0; p < 4; p++)
        Fmt<LH_Q4_K>::scales(w.hdr, 2 * p, sc[2 * p], mn[2 * p], sc[2 * p + 1], mn[2 * p + 1]);
    const float d = half_bits_to_float(w.hdr.x & 0xffff);
    const float dmin = half_bits_to_float(w.hdr.x >> 16);
    const mmq_i4 z = {0, 0, 0, 0};
    const bool lo = q4 < 2;
    int isum[MT][4];
    mmq_i4 msum[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        msum[mt] = z;
#pragma unroll
        for (int i = 0; i < 4; i++)
            isum[mt][i] = 0;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint4 v = w.qs[p];
        const int sh = lo ? 0 : 4;
        const mmq_i4 wv = {(int)((v.x >> sh) & 0x0F0F0F0Fu), (int)((v.y >> sh) & 0x0F0F0F0Fu),
                           (int)((v.z >> sh) & 0x0F0F0F0Fu), (int)((v.w >> sh) & 0x0F0F0F0Fu)};
        const mmq_i4 wa = lo ? wv : z, wb = lo ? z : wv;
        const int m32 = (int)((uint32_t)(lo ? mn[2 * p] : mn[2 * p + 1]) * 0x01010101u);
        const mmq_i4 mrep = {m32, m32, m32, m32};
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const mmq_i4 da = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[mt][p], wa, z, 0, 0, 0);
            const mmq_i4 db = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[mt][p], wb, z, 0, 0, 0);
            msum[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[mt][p], mrep, msum[mt], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) // 24-bit products (|dot| < 2^16, sc <= 63): full rate, exact
                isum[mt][i] += __mul24(sc[2 * p], da[i]) + __mul24(sc[2 * p + 1], db[i]);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // xb.d * (d * f32(isum) - dmin * f32(min_isum))  (ggml.zig:1016-1017)
            const float a = d * (float)isum[mt][i];
            const float bb = dmin * (float)msum[mt][i];
            r[mt][i] = xd[mt][i] * (a - bb);
        }
}

// Q6_K (device SoA ql[U][128] | qh[U][64] | sc[U][16] | d[U]) on
// v_mfma_i32_16x16x64_i8: MFMA h spans values [64h, 64h + 64) and lane
// quarter q4 holds the 16 values [64h + 16*q4, +16) -- exactly the 16-value
// run 4h + q4 -- so activation and weight loads are 16 contiguous bytes per
// lane.  Each run has its own scale: one MFMA per run, the other quarters'
// weights zeroed.  The weights enter as q - 32 (-32..31 fits int8), so isum =
// sum_run sc[run] * dot(q - 32, x), the reference's sum sc * (dot(q, x) - 32 *
// sum(x)) as one exact integer.
struct Q6kTile {
    uint4 ql[2], qh[2]; // half n's 16 bytes of low bits / high bits for this lane's quarter
    uint4 sc;
    uint16_t d;
};

__device__ __forceinline__ Q6kTile q6k_load(const uint8_t *base, size_t U, size_t unit, int q4) {
    Q6kTile w;
#pragma unroll
    for (int n = 0; n < 2; n++) {
        w.ql[n] = *(const uint4 *)(base + unit * 128 + 64 * n + 16 * q4);
        w.qh[n] = *(const uint4 *)(base + U * 128 + unit * 64 + 32 * n + 16 * (q4 & 1));
    }
    w.sc = *(const uint4 *)(base + U * 192 + unit * 16);
    w.d = *(const uint16_t *)(base + U * 208 + unit * 2);
    return w;
}

// 4 bytes of 6-bit quants (low nibble at shift ls, two high bits at shift hs)
// -> q - 32 as int8: flip bit 5, then sign-extend it into bits 6 and 7
// where it is set (the values below 32)
__device__ __forceinline__ int q6_minus32(uint32_t ql, uint32_t qh, int ls, int hs) {
    const uint32_t v = ((ql >> ls) & 0x0F0F0F0Fu) | (((qh >> hs) & 0x03030303u) << 4);
    const uint32_t y = v ^ 0x20202020u;
    const uint32_t m = y & 0x20202020u;
    return (int)(y | (m << 1) | (m << 2));
}

template <int MT>
__device__ __forceinline__ void q6k_tile(const Q6kTile &w, int q4, const mmq_i4 (&xa)[MT][4],
                                         const float (&xd)[MT][4], float (&r)[MT][4]) {
    const float dw = half_bits_to_float(w.d);
    const mmq_i4 z = {0, 0, 0, 0};
    int isum[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            isum[mt][i] = 0;
#pragma unroll
    for (int h = 0; h < 4; h++) {
        const int n = h >> 1, ls = 4 * (h & 1), hs = 4 * (h & 1) + 2 * (q4 >> 1);
        const mmq_i4 vs = {q6_minus32(w.ql[n].x, w.qh[n].x, ls, hs), q6_minus32(w.ql[n].y, w.qh[n].y, ls, hs),
                           q6_minus32(w.ql[n].z, w.qh[n].z, ls, hs), q6_minus32(w.ql[n].w, w.qh[n].w, ls, hs)};
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int sc = (int)(int8_t)byte_of(w.sc, 4 * h + qq);
            const mmq_i4 bq = q4 == qq ? vs : z;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const mmq_i4 dq = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[mt][h], bq, z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) // 24-bit products (|dot| < 2^16, |sc| <= 128): full rate, exact
                    isum[mt][i] += __mul24(sc, dq[i]);
            }
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // xb.d * dec.d * f32(isum)  (ggml.zig:1019)
            const float s = xd[mt][i] * dw;
            r[mt][i] = s * (float)isum[mt][i];
        }
}

// ---- Q4_K with (token, group) rows: up to 16 tokens against unmasked weights -------
// A 64-deep MFMA span holds two Q4_K groups, each with its own scale.
// q4k_tile zeroes the weights outside one group and runs one MFMA per group:
// a masked copy of every weight tile, and a quarter-rate integer multiply
// per scale.  Here the A rows of an MFMA are (token, group) pairs instead:
// row m = (t, g) carries token t's activations on the k slots of group part g
// and zeros elsewhere -- arranged once per token as it loads -- so one MFMA
// over the unmasked weights returns both groups' integer dots for 8 tokens,
// and the scales multiply those dots with full-rate 24-bit multiply-adds
// (|dot| < 2^16, scale <= 63).  The mins are one chained MFMA per span
// against the part's group min replicated over its k slots: sum_g mn_g *
// sum(x_g).  Integer dots are exact in any order, so every block's integers
// -- and the f32 tail after them -- are the reference's.
//
// k slots.  MFMA (P, half) covers quant spans 2P and 2P + 1: lane
// quarter q4 holds the 16 bytes 64P + 16*q4 of the block's 128 (span
// 2P + q4/2, bytes 16*(q4&1) + [0, 16)), their low nibbles for half 0 and
// high nibbles for half 1 -- group 4P + 2*(q4/2) + half.  A lane loads each
// weight byte once.  A row r16 = (token r16/2, part r16&1) is nonzero on the
// quarters with q4/2 == r16&1.
struct Q4kTileV {
    uint4 hdr;
    uint4 qs[2]; // quant bytes 64P + 16*q4, P = 0, 1
};

__device__ __forceinline__ Q4kTileV q4kv_load(const uint8_t *blk, int q4) {
    Q4kTileV w;
    w.hdr = *(const uint4 *)blk;
    w.qs[0] = *(const uint4 *)(blk + 16 + 16 * q4);
    w.qs[1] = *(const uint4 *)(blk + 80 + 16 * q4);
    return w;
}

// Offset in the block's 256 activations of lane quarter q4's 16 k slots in
// MFMA j = 2P + half.
__device__ __forceinline__ int q4kv_xoff(int j, int q4) {
    return 128 * (j >> 1) + 64 * (q4 >> 1) + 32 * (j & 1) + 16 * (q4 & 1);
}

// Result lane (row r16, quarter q4) holds A rows 4*q4 + i: tokens 2*q4 + i/2
// of the set (part i&1), whose two values r[s][0..1] it returns.
template <int NS>
__device__ __forceinline__ void q4kv_tile(const Q4kTileV &w, int q4, int ns, const mmq_i4 (&xa)[NS][4],
                                          const float (&xd)[NS][2], float (&r)[NS][2]) {
    const uint32_t a = w.hdr.y, b = w.hdr.z, c = w.hdr.w;
    // Fmt<LH_Q4_K>::scales four groups at a time: bytes 0-3 are groups 0-3 (P = 0), 4-7 (P = 1)
    const uint32_t scv[2] = {a & 0x3F3F3F3Fu, (c & 0x0F0F0F0Fu) | ((a >> 2) & 0x30303030u)};
    const uint32_t mnv[2] = {b & 0x3F3F3F3Fu, ((c >> 4) & 0x0F0F0F0Fu) | ((b >> 2) & 0x30303030u)};
    const float d = half_bits_to_float(w.hdr.x & 0xffff);
    const float dmin = half_bits_to_float(w.hdr.x >> 16);
    const mmq_i4 z = {0, 0, 0, 0};
    // MFMA j = 2P + half: the nibbles (they replace the packed bytes), this
    // lane's group min replicated (its k slots are group 4P + 2*(q4/2) +
    // half), and the scales of parts 0 and 1 (groups 4P + half, 4P + 2 + half)
    mmq_i4 wv[4];
    int mr[4], s0[4], s1[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int P = j >> 1, half = j & 1;
        const uint4 v = w.qs[P];
        const uint32_t sh = 4 * half;
        wv[j] = mmq_i4{(int)((v.x >> sh) & 0x0F0F0F0Fu), (int)((v.y >> sh) & 0x0F0F0F0Fu),
                       (int)((v.z >> sh) & 0x0F0F0F0Fu), (int)((v.w >> sh) & 0x0F0F0F0Fu)};
        mr[j] = (int)__builtin_amdgcn_perm(mnv[P], mnv[P], (uint32_t)(2 * (q4 >> 1) + half) * 0x01010101u);
        s0[j] = (int)((scv[P] >> (8 * half)) & 0xFF);
        s1[j] = (int)((scv[P] >> (8 * (2 + half))) & 0xFF);
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
        if (s >= ns)
            break;
        mmq_i4 dq[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            dq[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[s][j], wv[j], z, 0, 0, 0);
        mmq_i4 msum = z;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const mmq_i4 mrep = {mr[j], mr[j], mr[j], mr[j]};
            msum = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[s][j], mrep, msum, 0, 0, 0);
        }
        int isum[2] = {0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            isum[0] += __mul24(s0[j], dq[j][0]) + __mul24(s1[j], dq[j][1]);
            isum[1] += __mul24(s0[j], dq[j][2]) + __mul24(s1[j], dq[j][3]);
        }
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            // xb.d * (d * f32(isum) - dmin * f32(min_isum))  (ggml.zig:1016-1017)
            const int ms = msum[2 * jj] + msum[2 * jj + 1];
            const float aa = d * (float)isum[jj];
            const float bb = dmin * (float)ms;
            r[s][jj] = xd[s][jj] * (aa - bb);
        }
    }
}

// LDS row stride of the (token, group) values: a result lane stores tokens
// 2*q4 + jj of row r16, so the quarters' stores land 2*RS floats apart --
// 16 or 48 mod 64 (RS = R + 8, R a multiple of 16) puts them in distinct banks.
__host__ __device__ constexpr int q4kv_rs(int R) { return R + 8; }

// LDS of one work group: the per-block values [FUSED + 1][nb][16*MT][16*RG + 1]
// (the +1 staggers the four token quarters a wave writes across banks).
static size_t mmq_lds_bytes(int cols, int mt, int rg, bool fused) {
    return (size_t)4 * (fused ? 2 : 1) * (cols / 256) * 16 * mt * (16 * rg + 1);
}

constexpr int MMQ_MAX_SBW = 4; // super-blocks per wave (at most): cols <= 8192 (4096 at 32 tokens)

// Waves per work group (at most).  Eight: with sixteen the waves of a group
// finish microseconds apart at the barrier (four per SIMD share its issue).
constexpr int MMQ_WAVES = 8;

// One wave's operands for one super-block: the activations as the MFMA A
// operands (16 bytes per 64-value span and lane quarter).
template <int T, int MT, bool FUSED>
struct MmqOps {
    typename std::conditional<T == LH_Q4_K, Q4kTile, Q6kTile>::type w, w2;
    mmq_i4 xa[MT][4];
    float xd[MT][4];
};

// Work group: RG row tiles of 16 rows x KS super-block slices, one wave per
// (tile, slice); wave (rg, ks) computes super-blocks ks + j*KS (j < SBW) of
// its 16 rows for the group's tokens.  All of a wave's loads are issued,
// weights first, before its first MFMA.  The values meet in LDS; every output
// sums its blocks in block order (the reference's `acc += r`), SwiGLU(gate,
// up) when FUSED, and is stored or added.
// The work group's part of mmq_kernel: row tile bx, group by.
template <int T, int MT, bool FUSED, int SBW>
__device__ __forceinline__ void mmq_body(const DmmvParams &p, int bx, int by, int RG, int KS, float *part) {
    constexpr int TOK = 16 * MT;
    const bool ident = p.ident_n > 0;
    DmmvGroup grp;
    if (ident) {
        grp.plane = 0;
        grp.first = by * TOK;
        grp.n = min(TOK, p.ident_n - grp.first);
    } else {
        const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
        if (by >= ng)
            return;
        grp = p.groups[by];
    }
    const int n = grp.n, cols = p.cols, nb = cols / 256;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
    const int r16 = ln & 15, q4 = ln >> 4;
    const int rg = wave % RG, ks = wave / RG;
    const int R = 16 * RG, RS = R + 1;
    const int row0 = bx * R;
    const int rl = 16 * rg + r16;
    const int row = min(row0 + rl, p.rows - 1);
    const size_t U = (size_t)p.rows * nb;
    const size_t mat = (size_t)nb * TOK * RS; // floats per matrix in LDS
    const uint8_t *wb = p.w + (size_t)grp.plane * p.plane_bytes;
    const uint8_t *wb2 = FUSED ? p.w2 + (size_t)grp.plane * p.plane_bytes : nullptr;
    MmqOps<T, MT, FUSED> op[SBW];
    int bj[SBW];
    // 1. weights (they depend on the group only)
#pragma unroll
    for (int j = 0; j < SBW; j++) {
        bj[j] = min(ks + j * KS, nb - 1); // past nb: a real block, never stored
        const size_t unit = (size_t)row * nb + bj[j];
        if constexpr (T == LH_Q4_K) {
            op[j].w = q4k_load(wb + unit * 144, q4);
            if constexpr (FUSED)
                op[j].w2 = q4k_load(wb2 + unit * 144, q4);
        } else {
            op[j].w = q6k_load(wb, U, unit, q4);
        }
    }
    // 2. activations: the row of A-row r16 in each token tile (tokens past n
    // repeat the last one; their outputs are never stored), then every
    // super-block's 8-value pieces and the output tokens' block scales
    int vrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        vrow[mt] = ident ? grp.first + min(16 * mt + r16, n - 1) : p.pair_src[grp.first + min(16 * mt + r16, n - 1)];
    int vout[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            vout[mt][i] = __shfl(vrow[mt], 4 * q4 + i);
#pragma unroll
    for (int j = 0; j < SBW; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int8_t *xr = p.xq + (size_t)vrow[mt] * cols + 256 * bj[j] + 16 * q4;
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++)
                op[j].xa[mt][s4] = *(const mmq_i4 *)(xr + 64 * s4);
#pragma unroll
            for (int i = 0; i < 4; i++)
                op[j].xd[mt][i] = p.xd[(size_t)vout[mt][i] * nb + bj[j]];
        }
    // 3. the first output of this thread (the common case is one per thread):
    // its destination and, for a residual add, the value it adds to
    const int idx0 = threadIdx.x, tk0 = idx0 / R, rr0 = idx0 % R;
    const bool out0 = idx0 < n * R && row0 + rr0 < p.rows;
    const int dst0 = ident ? grp.first + tk0 : p.pair_dst[grp.first + min(tk0, n - 1)];
    const float old0 = out0 && p.accumulate ? p.out[(size_t)dst0 * p.out_stride + row0 + rr0] : 0.0f;
    __builtin_amdgcn_sched_barrier(0); // every load above is in flight before the first MFMA
    // 4. the tiles
#pragma unroll
    for (int j = 0; j < SBW; j++) {
        float r[MT][4], r2[MT][4];
        if constexpr (T == LH_Q4_K) {
            q4k_tile<MT>(op[j].w, q4, op[j].xa, op[j].xd, r);
            if constexpr (FUSED)
                q4k_tile<MT>(op[j].w2, q4, op[j].xa, op[j].xd, r2);
        } else {
            q6k_tile<MT>(op[j].w, q4, op[j].xa, op[j].xd, r);
        }
        if (ks + j * KS < nb) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const size_t o = ((size_t)bj[j] * TOK + 16 * mt + 4 * q4 + i) * RS + rl;
                    part[o] = r[mt][i];
                    if constexpr (FUSED)
                        part[mat + o] = r2[mt][i];
                }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < n * R; idx += blockDim.x) {
        const int tk = idx / R, rr = idx % R;
        if (row0 + rr >= p.rows)
            continue;
        const float *pv = part + (size_t)tk * RS + rr;
        float acc = 0.0f;
        for (int b = 0; b < nb; b++)
            acc = acc + pv[(size_t)b * TOK * RS];
        float v = acc;
        if constexpr (FUSED) {
            float acc2 = 0.0f;
            for (int b = 0; b < nb; b++)
                acc2 = acc2 + pv[mat + (size_t)b * TOK * RS];
            v = swiglu1(acc, acc2);
        }
        const bool first = idx == idx0;
        const int dst = first ? dst0 : ident ? grp.first + tk : p.pair_dst[grp.first + tk];
        float *o = p.out + (size_t)dst * p.out_stride + row0 + rr;
        if (p.accumulate)
            v = (first ? old0 : *o) + v;
        *o = v;
    }
}

template <int T, int MT, bool FUSED, int SBW>
__global__ __launch_bounds__(64 * MMQ_WAVES) void mmq_kernel(DmmvParams p, int RG, int KS) {
    extern __shared__ __align__(16) float part[];
    mmq_body<T, MT, FUSED, SBW>(p, blockIdx.x, blockIdx.y, RG, KS, part);
}

// Up to DMMV_MAX_SEG matrices (Q4_K or Q6_K, same columns, same lane groups)
// in one launch: the row tiles of the segments one after another along x.
template <int MT, int SBW>
__global__ __launch_bounds__(64 * MMQ_WAVES) void mmq_seg_kernel(DmmvSegParams sp, int RG, int KS) {
    extern __shared__ __align__(16) float part[];
    int tile = blockIdx.x, s = 0;
    while (s + 1 < sp.n_seg && tile >= sp.seg[s].tiles) {
        tile -= sp.seg[s].tiles;
        s++;
    }
    DmmvParams p = sp.base;
    p.w = sp.seg[s].w;
    p.rows = sp.seg[s].rows;
    p.out = sp.seg[s].out;
    p.out_stride = sp.seg[s].rows;
    if (sp.seg[s].t == LH_Q4_K)
        mmq_body<LH_Q4_K, MT, false, SBW>(p, tile, blockIdx.y, RG, KS, part);
    else
        mmq_body<LH_Q6_K, MT, false, SBW>(p, tile, blockIdx.y, RG, KS, part);
}

// Streaming variant for one super-block per wave (nb <= MMQ_WAVES): a work
// group walks NTILE consecutive row tiles of its group (each RG x 16 rows).  The activations are loaded once; each
// tile's weights are requested while the previous tile computes, in two
// register sets, and the values meet in two LDS buffers, one barrier per
// tile.  Same arithmetic and order as mmq_kernel.
template <int T, int MT, bool FUSED>
__global__ __launch_bounds__(64 * MMQ_WAVES) void mmq_stream_kernel(DmmvParams p, int RG, int NTILE) {
    extern __shared__ __align__(16) float part[];
    constexpr int TOK = 16 * MT;
    using Tile = typename std::conditional<T == LH_Q4_K, Q4kTile, Q6kTile>::type;
    const bool ident = p.ident_n > 0;
    DmmvGroup grp;
    if (ident) {
        grp.plane = 0;
        grp.first = (int)blockIdx.y * TOK;
        grp.n = min(TOK, p.ident_n - grp.first);
    } else {
        const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
        if ((int)blockIdx.y >= ng)
            return;
        grp = p.groups[blockIdx.y];
    }
    const int n = grp.n, cols = p.cols, nb = cols / 256;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
    const int r16 = ln & 15, q4 = ln >> 4;
    const int rg = wave % RG, b = wave / RG; // this wave's super-block
    const int R = 16 * RG, RS = R + 1;
    const int rl = 16 * rg + r16;
    const int tile0 = blockIdx.x * NTILE;
    const int nti = min(NTILE, (p.rows + R - 1) / R - tile0);
    const size_t U = (size_t)p.rows * nb;
    const size_t mat = (size_t)nb * TOK * RS;
    const size_t buf = (size_t)(FUSED ? 2 : 1) * mat;
    const uint8_t *wb = p.w + (size_t)grp.plane * p.plane_bytes;
    const uint8_t *wb2 = FUSED ? p.w2 + (size_t)grp.plane * p.plane_bytes : nullptr;
    auto load_tile = [&](int tile, Tile &a, Tile &a2) {
        const size_t unit = (size_t)min(tile * R + rl, p.rows - 1) * nb + b;
        if constexpr (T == LH_Q4_K) {
            a = q4k_load(wb + unit * 144, q4);
            if constexpr (FUSED)
                a2 = q4k_load(wb2 + unit * 144, q4);
        } else {
            a = q6k_load(wb, U, unit, q4);
        }
    };
    Tile wa, wa2, wbt, wbt2;
    load_tile(tile0, wa, wa2);
    int vrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        vrow[mt] = ident ? grp.first + min(16 * mt + r16, n - 1) : p.pair_src[grp.first + min(16 * mt + r16, n - 1)];
    mmq_i4 xa[MT][4];
    float xd[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int8_t *xr = p.xq + (size_t)vrow[mt] * cols + 256 * b + 16 * q4;
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++)
            xa[mt][s4] = *(const mmq_i4 *)(xr + 64 * s4);
#pragma unroll
        for (int i = 0; i < 4; i++)
            xd[mt][i] = p.xd[(size_t)__shfl(vrow[mt], 4 * q4 + i) * nb + b];
    }
    // one tile: its values into LDS buffer pb, the barrier, then the outputs
    auto run_tile = [&](int it, const Tile &w, const Tile &w2) {
        float *pb = part + (size_t)(it & 1) * buf;
        float r[MT][4], r2[MT][4];
        if constexpr (T == LH_Q4_K) {
            q4k_tile<MT>(w, q4, xa, xd, r);
            if constexpr (FUSED)
                q4k_tile<MT>(w2, q4, xa, xd, r2);
        } else {
            q6k_tile<MT>(w, q4, xa, xd, r);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const size_t o = ((size_t)b * TOK + 16 * mt + 4 * q4 + i) * RS + rl;
                pb[o] = r[mt][i];
                if constexpr (FUSED)
                    pb[mat + o] = r2[mt][i];
            }
        // a buffer is written again two tiles on, after every thread has
        // passed the next tile's barrier
        __syncthreads();
        const int row0 = (tile0 + it) * R;
        for (int idx = threadIdx.x; idx < n * R; idx += blockDim.x) {
            const int tk = idx / R, rr = idx % R;
            if (row0 + rr >= p.rows)
                continue;
            const float *pv = pb + (size_t)tk * RS + rr;
            float acc = 0.0f;
            for (int bb = 0; bb < nb; bb++)
                acc = acc + pv[(size_t)bb * TOK * RS];
            float v = acc;
            if constexpr (FUSED) {
                float acc2 = 0.0f;
                for (int bb = 0; bb < nb; bb++)
                    acc2 = acc2 + pv[mat + (size_t)bb * TOK * RS];
                v = swiglu1(acc, acc2);
            }
            const int dst = ident ? grp.first + tk : p.pair_dst[grp.first + tk];
            float *o = p.out + (size_t)dst * p.out_stride + row0 + rr;
            *o = p.accumulate ? *o + v : v;
        }
    };
    for (int it = 0; it < nti; it += 2) {
        if (it + 1 < nti)
            load_tile(tile0 + it + 1, wbt, wbt2);
        __builtin_amdgcn_sched_barrier(0);
        run_tile(it, wa, wa2);
        if (it + 1 >= nti)
            break;
        if (it + 2 < nti)
            load_tile(tile0 + it + 2, wa, wa2);
        __builtin_amdgcn_sched_barrier(0);
        run_tile(it + 1, wbt, wbt2);
    }
}

// ---- grouped Q4_K expert matmuls streamed through LDS ------------------------------
// The one-shot work groups of mmq_kernel hold their weights in registers from
// the first load to the last MFMA: two of them fit a CU, each waits ~2.5 us
// on its loads, and a grouped launch also queues a work group per group the
// routing could make (at 32 tokens x top-8 over 128 experts: 144 possible,
// ~45 made).  Here one work group per CU walks (group, run of row tiles)
// items, sized on the device from the groups actually made, and streams each
// tile's weights through a ring of three LDS stages with direct
// global->LDS loads (16 bytes per lane, 1 KB of LDS per wave instruction):
// the next tiles load while one computes, and the registers hold only the
// group's activations.
//
// Geometry: a tile is TR = 16*RG rows x all NB super-blocks of one matrix
// (both for the fused gate/up); wave (rg, b) computes block b of rows
// 16*rg .. +16, RG = 8 / NB.  LDS slot j of a matrix is (block, 16-byte chunk
// c, row r), r fastest, so a wave's operand read is 1 KB of consecutive
// slots and a row header a broadcast; chunk 0 of a (row, block) is its
// header, 1..8 its quants.
template <bool FUSED, int NB>
struct Mmqs {
    static constexpr int RG = 8 / NB, W = RG * NB, TR = 16 * RG;
    static constexpr int MAT = TR * NB * 9; // 16-byte chunks per matrix
    static constexpr int MATS = FUSED ? 2 : 1;
    static constexpr int CH = MATS * MAT;
    static constexpr int INS = (CH + 63) / 64; // 1 KB wave loads per tile, dealt round robin:
    static constexpr int K = (INS + W - 1) / W; // waves below KW issue K, the rest K - 1
    static constexpr int KW = INS % W == 0 ? W : INS % W;
    static constexpr int STAGE = INS * 1024;    // bytes per stage
    static constexpr int RS = q4kv_rs(TR);
    static constexpr int PART = MATS * NB * 16 * RS; // floats
    static constexpr size_t LDS = 3 * (size_t)STAGE + 2 * 4 * (size_t)PART;
    static_assert(LDS <= 160 * 1024, "three stages and two sums buffers fit a CU's LDS");
};

// Global address of chunk j of a tile (rows row0 .. +TR, clamped to the
// matrix) of the Q4_K matrix at mb.
template <int NB, int TR>
__device__ __forceinline__ const uint8_t *mmqs_chunk(const uint8_t *mb, int rows, int row0, int j) {
    const int bb = j / (9 * TR), c = (j / TR) % 9, r = j % TR;
    const int row = min(row0 + r, rows - 1);
    return mb + ((size_t)row * NB + bb) * 144 + c * 16;
}

// A work-group barrier that waits for this wave's LDS stores only: the
// workgroup fence of lds_barrier also waits for the direct-to-LDS loads in
// flight (they are LDS stores), which would drain the ring at every tile.
// The loads a barrier must cover are waited for explicitly (wait_vm) before
// it; the asm's memory clobber keeps the compiler from moving LDS accesses
// across it.
__device__ __forceinline__ void ring_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0); vmcnt and expcnt left open
    asm volatile("s_barrier" ::: "memory");
}

// Reads of a stage.  The compiler cannot tell the three stages apart, so
// before any LDS read it would wait for every direct-to-LDS load in flight;
// the reads are issued as one asm block instead, ending in its own lgkmcnt
// wait, after the explicit vmcnt wait and barrier that order them behind
// their own tile's loads.
typedef unsigned mmqs_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t lds_off(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ void lds_read3(uint32_t a0, uint32_t a1, uint32_t a2, uint4 &r0, uint4 &r1, uint4 &r2) {
    mmqs_u4 x0, x1, x2;
    asm volatile("ds_read_b128 %0, %3\n\tds_read_b128 %1, %4\n\tds_read_b128 %2, %5\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(x0), "=&v"(x1), "=&v"(x2)
                 : "v"(a0), "v"(a1), "v"(a2)
                 : "memory");
    r0 = make_uint4(x0.x, x0.y, x0.z, x0.w);
    r1 = make_uint4(x1.x, x1.y, x1.z, x1.w);
    r2 = make_uint4(x2.x, x2.y, x2.z, x2.w);
}

template <int N>
__device__ __forceinline__ void wait_vm() { // s_waitcnt vmcnt(N) alone
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

template <bool FUSED, int NB>
__global__ __launch_bounds__(64 * MMQ_WAVES) void mmqs_kernel(DmmvParams p) {
    using G = Mmqs<FUSED, NB>;
    constexpr int TOK = 16, TR = G::TR, RS = G::RS, K = G::K;
    constexpr int TPS = 8, NS = TOK / TPS; // tokens per MFMA set (x 2 groups = 16 A rows), sets
    __shared__ __align__(16) uint8_t st0[G::STAGE], st1[G::STAGE], st2[G::STAGE];
    __shared__ __align__(16) float part0[G::PART], part1[G::PART];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
    const int r16 = ln & 15, q4 = ln >> 4;
    const int rg = wave % G::RG, b = wave / G::RG;
    const int rl = 16 * rg + r16;
    const int tiles = (p.rows + TR - 1) / TR;
    const size_t mat = (size_t)NB * TOK * RS;
    const mmq_i4 z = {0, 0, 0, 0};
    const bool live = (q4 >> 1) == (r16 & 1); // A row r16 = (token r16/2, group part r16&1)
    // items: each group's tiles in cpg runs, so that the items about fill the grid
    const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
    const int nwg = gridDim.x;
    const int cpg = ng > 0 ? max(1, min(tiles, nwg / ng)) : 1;
    const int run = (tiles + cpg - 1) / cpg;
    const int items = ng * cpg;
    for (int item = blockIdx.x; item < items; item += nwg) {
        const int gi = item / cpg, t0 = (item % cpg) * run;
        const int nt = min(run, tiles - t0);
        if (nt <= 0)
            continue;
        const DmmvGroup grp = p.groups[gi];
        const int n = grp.n, ns = (n + TPS - 1) / TPS;
        const uint8_t *pb = p.w + (size_t)grp.plane * p.plane_bytes;
        const uint8_t *pb2 = FUSED ? p.w2 + (size_t)grp.plane * p.plane_bytes : pb;
        // the group's activations as A rows, and the block scales of this
        // lane's result tokens 2*q4 + jj of each set
        auto vec_of = [&](int t) {
            if (p.group_src)
                return p.group_src[(size_t)gi * p.group_stride + t];
            t = min(t, n - 1);
            return p.pos_ident ? grp.first + t : p.pair_src[grp.first + t];
        };
        mmq_i4 xa[NS][4];
        float xd[NS][2];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int8_t *xr = p.xq + (size_t)vec_of(TPS * s + r16 / 2) * p.cols + 256 * b;
#pragma unroll
            for (int j = 0; j < 4; j++)
                xa[s][j] = live && s < ns ? *(const mmq_i4 *)(xr + q4kv_xoff(j, q4)) : z;
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
                xd[s][jj] = s < ns ? p.xd[(size_t)vec_of(TPS * s + 2 * q4 + jj) * NB + b] : 0.0f;
        }
        // one tile's weights into a stage: this wave's 1 KB pieces I = wave + W*i
        auto issue = [&](int tile, uint8_t *stg) {
            const int row0 = tile * TR;
#pragma unroll
            for (int i = 0; i < K; i++) {
                const int I = wave + G::W * i;
                if (I >= G::INS)
                    break; // (uniform)
                int j = I * 64 + ln;
                const uint8_t *src = pb; // past the tile's chunks: a valid address, never read back
                if (j < G::CH) {
                    const uint8_t *mb = pb;
                    if (FUSED && j >= G::MAT) {
                        mb = pb2;
                        j -= G::MAT;
                    }
                    src = mmqs_chunk<NB, TR>(mb, p.rows, row0, j);
                }
                __builtin_amdgcn_global_load_lds((const void *)src,
                                                 (__attribute__((address_space(3))) void *)(stg + I * 1024), 16, 0, 0);
            }
        };
        // tile k's loads have landed once only the next tile's (this wave's
        // K or K - 1 pieces, issued after it) may be outstanding
        auto wait_tile = [&](int k) {
            if (k + 1 >= nt)
                wait_vm<0>();
            else if (wave < G::KW)
                wait_vm<K>();
            else
                wait_vm<K - 1>();
        };
        // a tile's MFMAs from its stage, its per-block values into pbuf
        auto compute = [&](const uint8_t *stg, float *pbuf) {
            auto frag = [&](int m) {
                const uint32_t mbase = lds_off(stg) + (uint32_t)m * G::MAT * 16;
                Q4kTileV w;
                lds_read3(mbase + ((b * 9 + 0) * TR + rl) * 16, mbase + ((b * 9 + 1 + q4) * TR + rl) * 16,
                          mbase + ((b * 9 + 5 + q4) * TR + rl) * 16, w.hdr, w.qs[0], w.qs[1]);
                return w;
            };
            float r[NS][2], r2[NS][2];
            q4kv_tile<NS>(frag(0), q4, ns, xa, xd, r);
            if constexpr (FUSED)
                q4kv_tile<NS>(frag(1), q4, ns, xa, xd, r2);
#pragma unroll
            for (int s = 0; s < NS; s++)
                if (s < ns)
#pragma unroll
                    for (int jj = 0; jj < 2; jj++) {
                        const size_t o = ((size_t)b * TOK + TPS * s + 2 * q4 + jj) * RS + rl;
                        pbuf[o] = r[s][jj];
                        if constexpr (FUSED)
                            pbuf[mat + o] = r2[s][jj];
                    }
        };
        // tile k's outputs: every (token, row) summed over its blocks in block
        // order from pbuf (all the block values read first), SwiGLU(gate, up)
        // when fused, stored -- pos_ident, no residual add (launch_mmqs), so
        // no global load here, which would wait (vmcnt counts in order) for
        // the tiles in flight
        auto reduce = [&](int k, const float *pbuf) {
            const int row0 = (t0 + k) * TR;
            for (int idx = threadIdx.x; idx < n * TR; idx += blockDim.x) {
                const int tk = idx / TR, rr = idx % TR;
                if (row0 + rr >= p.rows)
                    continue;
                const float *pv = pbuf + (size_t)tk * RS + rr;
                float v1[NB], v2[NB];
#pragma unroll
                for (int bb = 0; bb < NB; bb++) {
                    v1[bb] = pv[(size_t)bb * TOK * RS];
                    if constexpr (FUSED)
                        v2[bb] = pv[mat + (size_t)bb * TOK * RS];
                }
                float acc = 0.0f;
#pragma unroll
                for (int bb = 0; bb < NB; bb++)
                    acc = acc + v1[bb];
                float v = acc;
                if constexpr (FUSED) {
                    float acc2 = 0.0f;
#pragma unroll
                    for (int bb = 0; bb < NB; bb++)
                        acc2 = acc2 + v2[bb];
                    v = swiglu1(acc, acc2);
                }
                p.out[(size_t)(grp.first + tk) * p.out_stride + row0 + rr] = v;
            }
        };
        // Step k: wait for tile k, one barrier, then tile k - 1's sums out (its
        // values were written before this barrier), tile k + 2's loads into
        // the stage tile k - 1 computed from (every wave has passed its reads),
        // and tile k's MFMAs.  The sums buffers alternate, so tile k's values
        // are written while tile k - 1's are read.  The stores precede the next
        // loads, so the next wait (vmcnt counts in order) covers them too.
        auto step = [&](int k, const uint8_t *cur, uint8_t *refill) {
            wait_tile(k);
            ring_barrier();
            if (k > 0)
                reduce(k - 1, (k - 1) & 1 ? part1 : part0);
            if (k + 2 < nt)
                issue(t0 + k + 2, refill);
            compute(cur, k & 1 ? part1 : part0);
        };
        issue(t0, st0);
        if (nt > 1)
            issue(t0 + 1, st1);
        for (int k = 0; k < nt; k += 3) {
            step(k, st0, st2);
            if (k + 1 >= nt)
                break;
            step(k + 1, st1, st0);
            if (k + 2 >= nt)
                break;
            step(k + 2, st2, st1);
        }
        ring_barrier();
        reduce(nt - 1, (nt - 1) & 1 ? part1 : part0);
        ring_barrier(); // the next item's stages and sums reuse this one's LDS
    }
}

// The streamed launch: the fused gate/up of grouped experts (not lane
// groups), Q4_K over 2048 columns, up to 16 tokens per group, outputs at the
// pair positions with no residual add; false = not served.
static bool launch_mmqs(int t, bool fused, const DmmvParams &p, hipStream_t st) {
    if (t != LH_Q4_K || !fused || p.ident_n > 0 || !p.groups || !p.pos_ident || p.accumulate || p.rows < 1 ||
        p.cols != 8 * 256)
        return false;
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
            cus = c;
        else
            cus = 256;
    }
    // one work group per CU (its LDS fills one)
    hipLaunchKernelGGL((mmqs_kernel<true, 8>), dim3(cus), dim3(64 * Mmqs<true, 8>::W), 0, st, p);
    return true;
}


// Shape of a launch: KS = min(nb, MMQ_WAVES) slices of SBW super-blocks per
// wave, as many row tiles beside them as fit the wave count and 64 KB of LDS,
// but no more than the matrix has.
static bool mmq_shape(int rows, int cols, int mt, bool fused, int &rg, int &ks, int &sbw) {
    const int nb = cols / 256;
    ks = nb < MMQ_WAVES ? nb : MMQ_WAVES;
    sbw = (nb + ks - 1) / ks;
    if (sbw == 3)
        sbw = 4;
    if (sbw > MMQ_MAX_SBW || (mt == 2 && sbw > 2)) // 4 x 32 tokens would not fit the registers
        return false;
    rg = MMQ_WAVES / ks;
    const int tiles = (rows + 15) / 16;
    if (rg > tiles)
        rg = tiles;
    while (rg > 1 && mmq_lds_bytes(cols, mt, rg, fused) > 64 * 1024)
        rg--;
    return mmq_lds_bytes(cols, mt, rg, fused) <= 64 * 1024;
}

// ---- Q8_0 / Q4_0 (32-value blocks) on the int8 matrix cores ----------------------
// A work group of MQ32_W waves per (16-row tile, 16 tokens of a group: a group
// of up to 32 takes two, along z); wave w takes the w-th share of the rows'
// 64-value spans.  Per span
// (blocks 2s and 2s + 1) lane quarter q4 holds 16 values of block 2s + q4/2
// -- A: token r16's activations, B: row r16's quants (Q4_0 as nibble - 8) --
// and two MFMAs over the span, each with the other block's quarters of the
// weights zeroed, give each block's integer dot for the 16 tokens: Q8_0
// sum w*x; Q4_0 sum (q - 8)*x, which is the reference's sum q*x - 8*sum x as
// one exact integer.  Each block's f32 tail (d * xd) * f32(isum)
// (ggml.zig:1212-1218, 1289-1290) goes to LDS; then every output sums its
// blocks in block order from +0 -- the reference's acc += r -- one thread
// per output.  A wave's loads run MQ32_AHEAD spans ahead; the tokens' block
// scales are staged in LDS once.
constexpr int MQ32_AHEAD = 4;
constexpr int MQ32_W = 8;         // waves per work group (span shares)
constexpr int MQ32_MAXS = 8;      // spans per wave: cols <= 4096
constexpr int MQ32_PART = 32768;  // LDS floats of block values: nb * 256

template <int T>
__global__ __launch_bounds__(64 * MQ32_W) void mmq32_kernel(DmmvParams p) {
    constexpr int MT = 1;
    static_assert(T == LH_Q8_0 || T == LH_Q4_0, "32-value blocks");
    constexpr int QB = T == LH_Q8_0 ? 32 : 16; // quant bytes per block
    constexpr int NO = 256 * MT;               // outputs per work group: (token, row)
    constexpr int MAXNB = 64 * MQ32_W * MQ32_MAXS / 32;
    __shared__ __align__(16) float part[MQ32_PART];      // [block][token * 16 + row]
    __shared__ __align__(16) float xds[16 * MT][MAXNB];  // the tokens' block scales
    const int ln = threadIdx.x & 63, r16 = ln & 15, q4 = ln >> 4;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const bool ident = p.ident_n > 0;
    DmmvGroup grp;
    if (ident) {
        grp.plane = 0;
        grp.first = (int)blockIdx.y * 16;
        grp.n = min(16, p.ident_n - grp.first);
    } else {
        const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
        if ((int)blockIdx.y >= ng)
            return;
        grp = p.groups[blockIdx.y];
        // tokens 16 z .. of the group (pairs first + 16 z ..)
        grp.first += 16 * (int)blockIdx.z;
        grp.n = min(16, grp.n - 16 * (int)blockIdx.z);
        if (grp.n <= 0)
            return;
    }
    const int n = grp.n, cols = p.cols, nb = cols / 32, ns = cols / 64;
    const int s_lo = wave * ns / MQ32_W, cnt = (wave + 1) * ns / MQ32_W - s_lo; // this wave's spans
    const int row0 = (int)blockIdx.x * 16;
    const int row = min(row0 + r16, p.rows - 1);
    const size_t U = (size_t)p.rows * nb;
    const uint8_t *wb = p.w + (size_t)grp.plane * p.plane_bytes;
    // A row r16 of token tile mt carries a vector (tokens past n repeat the
    // last; their outputs are never stored); this lane's outputs are tokens
    // 16 mt + 4 q4 + i of row r16
    const int8_t *xr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int tk = min(16 * mt + r16, n - 1);
        const int vrow = ident ? grp.first + tk : p.pair_src[grp.first + tk];
        xr[mt] = p.xq + (size_t)vrow * cols + 16 * q4;
    }
    // the group's block scales, bound for LDS (row tk of xds: token tk's nb
    // scales; tokens past n repeat the last): thread (tk, part) loads blocks
    // xpart + TPT u of token tk, unconditionally from clamped indices, first;
    // they are stored after the first spans' loads are out, so that store
    // waits for these loads alone
    constexpr int TPT = 64 * MQ32_W / (16 * MT); // threads per token
    constexpr int XU = (MAXNB + TPT - 1) / TPT;  // scales per thread (at most)
    const int xtk = (int)threadIdx.x / TPT, xpart = (int)threadIdx.x % TPT;
    const float *xdr;
    {
        const int tc = min(xtk, n - 1);
        xdr = p.xd + (size_t)(ident ? grp.first + tc : p.pair_src[grp.first + tc]) * nb;
    }
    float xe[XU];
#pragma unroll
    for (int u = 0; u < XU; u++)
        xe[u] = xdr[min(xpart + TPT * u, nb - 1)];
    __builtin_amdgcn_sched_barrier(0);
    // block 2s + q4/2 of the lane's row: its 16 quant bytes (Q8_0: half q4 & 1;
    // Q4_0: all 16, the nibble half picked below) and the (d, d) pair of blocks 2s, 2s + 1
    const uint8_t *wq = wb + ((size_t)row * nb + (q4 >> 1)) * QB + (T == LH_Q8_0 ? 16 * (q4 & 1) : 0);
    const uint32_t *wd = (const uint32_t *)(wb + U * QB + (size_t)row * nb * 2);
    struct Span {
        mmq_i4 a[MT], w;
        uint32_t d;
    };
    // span j of this wave (past its last: the last, loaded and not used)
    auto load = [&](int j, Span &o) {
        const int sc = s_lo + min(j, cnt - 1);
        o.w = *(const mmq_i4 *)(wq + (size_t)2 * sc * QB);
        o.d = wd[sc];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            o.a[mt] = *(const mmq_i4 *)(xr[mt] + 64 * sc);
    };
    const mmq_i4 z = {0, 0, 0, 0};
    const bool lo = q4 < 2;
    auto span = [&](const Span &o, int sc) {
        mmq_i4 wv = o.w;
        if constexpr (T == LH_Q4_0) {
            // the lane's nibble half, then q - 8 per byte: (q + 0x78) ^ 0x80
            const uint32_t sh = 4 * (q4 & 1);
#pragma unroll
            for (int e = 0; e < 4; e++)
                wv[e] = (int)((((uint32_t)wv[e] >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ (int)0x80808080u;
        }
        const mmq_i4 wa = lo ? wv : z, wbk = lo ? z : wv;
        const float dwa = half_bits_to_float(o.d & 0xffffu), dwb = half_bits_to_float(o.d >> 16);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const mmq_i4 da = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[mt], wa, z, 0, 0, 0);
            const mmq_i4 db = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[mt], wbk, z, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tk = 16 * mt + 4 * q4 + i;
                const float2 xd = *(const float2 *)&xds[tk][2 * sc];
                const float sa = dwa * xd.x;
                part[(size_t)(2 * sc) * NO + tk * 16 + r16] = sa * (float)da[i];
                const float sb = dwb * xd.y;
                part[(size_t)(2 * sc + 1) * NO + tk * 16 + r16] = sb * (float)db[i];
            }
        }
    };
    // each span's loads are issued as a unit, in span order (the fences keep
    // them there), so a span's wait leaves the later spans' loads in flight
    Span ring[MQ32_AHEAD];
#pragma unroll
    for (int j = 0; j < MQ32_AHEAD; j++) {
        load(j, ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < XU; u++)
        if (xpart + TPT * u < nb)
            xds[xtk][xpart + TPT * u] = xe[u];
    lds_barrier(); // the scales
#pragma unroll
    for (int j = 0; j < MQ32_MAXS; j++) {
        if (j < cnt)
            span(ring[j % MQ32_AHEAD], s_lo + j);
        __builtin_amdgcn_sched_barrier(0);
        if (j + MQ32_AHEAD < MQ32_MAXS)
            load(j + MQ32_AHEAD, ring[j % MQ32_AHEAD]);
        __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier(); // every block's values
    // output o = (token o / 16, row o % 16): its blocks in order from +0
    for (int o = (int)threadIdx.x; o < NO; o += 64 * MQ32_W) {
        const int tk = o >> 4, rr = o & 15;
        float acc = 0.0f;
#pragma unroll 8
        for (int bl = 0; bl < nb; bl++)
            acc = acc + part[(size_t)bl * NO + o];
        if (tk < n && row0 + rr < p.rows) {
            const int dst = ident ? grp.first + tk : p.pair_dst[grp.first + tk];
            float *out = p.out + (size_t)dst * p.out_stride + row0 + rr;
            *out = p.accumulate ? *out + acc : acc;
        }
    }
}

static bool mmq32_supported(int t, int cols, int max_tok, bool fused) {
    // the block values of a work group fill (cols / 32) * 256 floats of LDS
    return (t == LH_Q8_0 || t == LH_Q4_0) && !fused && cols % 64 == 0 && cols >= 64 * MQ32_W &&
           cols <= 64 * MQ32_W * MQ32_MAXS && max_tok >= 1 && max_tok <= 32 &&
           (size_t)(cols / 32) * 256 <= (size_t)MQ32_PART;
}

// Identity pairs go in groups of 16 tokens; a caller's groups of up to 32
// take two work groups each (z).
static bool launch_mmq32(int t, int max_tok, const DmmvParams &p, hipStream_t st) {
    const bool ident = p.ident_n > 0;
    const int groups = ident ? (p.ident_n + 15) / 16 : p.n_groups;
    const dim3 grid((p.rows + 15) / 16, groups, ident || max_tok <= 16 ? 1 : 2), block(64 * MQ32_W);
    if (t == LH_Q8_0)
        hipLaunchKernelGGL(mmq32_kernel<LH_Q8_0>, grid, block, 0, st, p);
    else
        hipLaunchKernelGGL(mmq32_kernel<LH_Q4_0>, grid, block, 0, st, p);
    return true;
}

bool mmq_supported(int t, int cols, int max_tok, bool fused) {
    if (t == LH_Q8_0 || t == LH_Q4_0)
        return mmq32_supported(t, cols, max_tok, fused);
    if ((t != LH_Q4_K && t != LH_Q6_K) || cols % 256 || cols < 256 || max_tok < 1 || max_tok > 32)
        return false;
    if (fused && t != LH_Q4_K) // a fused pair is gate/up: Q4_K only here
        return false;
    int rg, ks, sbw;
    return mmq_shape(16, cols, (max_tok + 15) / 16, fused, rg, ks, sbw);
}

// Streaming serves the lane-group (identity) launches with at least
// MMQ_STREAM_MIN (row tile, group) pairs (the head): for the grouped expert
// launches the one-shot kernel measured faster (its groups already give
// thousands of short work groups).  Its two register sets hold one work
// group per CU, so the pairs are split over about MMQ_STREAM_WGS work groups
// (one per CU, no partial second round), at most MMQ_MAX_NTILE tiles each.
constexpr int MMQ_STREAM_MIN = 1024;
constexpr int MMQ_STREAM_WGS = 256;
constexpr int MMQ_MAX_NTILE = 64;

template <int T, int MT, bool FUSED>
static void mmq_launch_t(const DmmvParams &p, int rg, int ks, int sbw, hipStream_t st) {
    const size_t lds = mmq_lds_bytes(p.cols, MT, rg, FUSED);
    const int groups = p.ident_n > 0 ? (p.ident_n + 16 * MT - 1) / (16 * MT) : p.n_groups;
    const int tiles = (p.rows + 16 * rg - 1) / (16 * rg);
    if (sbw == 1 && p.ident_n > 0 && 2 * lds <= 64 * 1024) {
        const long pairs = (long)tiles * groups;
        int ntile = pairs < MMQ_STREAM_MIN ? 1 : (int)((pairs + MMQ_STREAM_WGS - 1) / MMQ_STREAM_WGS);
        ntile = ntile > MMQ_MAX_NTILE ? MMQ_MAX_NTILE : ntile;
        if (ntile > 1) {
            const dim3 grid((tiles + ntile - 1) / ntile, groups), block(64 * rg * ks);
            hipLaunchKernelGGL((mmq_stream_kernel<T, MT, FUSED>), grid, block, 2 * lds, st, p, rg, ntile);
            return;
        }
    }
    const dim3 grid(tiles, groups), block(64 * rg * ks);
    if (sbw == 1)
        hipLaunchKernelGGL((mmq_kernel<T, MT, FUSED, 1>), grid, block, lds, st, p, rg, ks);
    else if (sbw == 2)
        hipLaunchKernelGGL((mmq_kernel<T, MT, FUSED, 2>), grid, block, lds, st, p, rg, ks);
    else if constexpr (MT == 1)
        hipLaunchKernelGGL((mmq_kernel<T, MT, FUSED, 4>), grid, block, lds, st, p, rg, ks);
}

// Segments of Q4_K / Q6_K matrices over the same columns, lanes in groups of
// 16 (identity pairs, sp.base.ident_n set: twice the work groups of 32-lane
// groups measured faster for these small matrices at 32 lanes); declined
// (false) when a segment's type or the shape is not served.
bool launch_mmq_seg(DmmvSegParams sp, hipStream_t st) {
    const DmmvParams &p = sp.base;
    if (p.ident_n < 1 || sp.n_seg < 1 || sp.n_seg > DMMV_MAX_SEG)
        return false;
    constexpr int mt = 1;
    int rg = MMQ_WAVES, ks = 0, sbw = 0, tiles = 0;
    for (int i = 0; i < sp.n_seg; i++) {
        if ((sp.seg[i].t != LH_Q4_K && sp.seg[i].t != LH_Q6_K) || !mmq_supported(sp.seg[i].t, p.cols, 16 * mt, false))
            return false;
        int r, k, b;
        if (!mmq_shape(sp.seg[i].rows, p.cols, mt, false, r, k, b))
            return false;
        if (r < rg)
            rg = r;
        ks = k;
        sbw = b;
    }
    if (sbw > 2)
        return false;
    for (int i = 0; i < sp.n_seg; i++) {
        sp.seg[i].tiles = (sp.seg[i].rows + 16 * rg - 1) / (16 * rg);
        tiles += sp.seg[i].tiles;
    }
    const size_t lds = mmq_lds_bytes(p.cols, mt, rg, false);
    const dim3 grid(tiles, (p.ident_n + 16 * mt - 1) / (16 * mt)), block(64 * rg * ks);
    auto kern = sbw == 1 ? mmq_seg_kernel<mt, 1> : mmq_seg_kernel<mt, 2>;
    hipLaunchKernelGGL(kern, grid, block, lds, st, sp, rg, ks);
    note_launch();
    return true;
}

// Groups of at most max_tok (<= 32) tokens (with p.ident_n: max_tok sets
// the group size); p.rpw is unused.
bool launch_mmq(int t, int max_tok, bool fused, const DmmvParams &p, hipStream_t st) {
    if (!mmq_supported(t, p.cols, max_tok, fused) || p.rows < 1)
        return false;
    if (t == LH_Q8_0 || t == LH_Q4_0) {
        launch_mmq32(t, max_tok, p, st);
        note_launch();
        return true;
    }
    const int mt = max_tok > 16 ? 2 : 1;
    int rg, ks, sbw;
    if (!mmq_shape(p.rows, p.cols, mt, fused, rg, ks, sbw))
        return false;
    if (mt == 1 && launch_mmqs(t, fused, p, st)) {
        note_launch();
        return true;
    }
    if (t == LH_Q4_K) {
        if (mt == 1)
            fused ? mmq_launch_t<LH_Q4_K, 1, true>(p, rg, ks, sbw, st)
                  : mmq_launch_t<LH_Q4_K, 1, false>(p, rg, ks, sbw, st);
        else
            fused ? mmq_launch_t<LH_Q4_K, 2, true>(p, rg, ks, sbw, st)
                  : mmq_launch_t<LH_Q4_K, 2, false>(p, rg, ks, sbw, st);
    } else if (mt == 1) {
        mmq_launch_t<LH_Q6_K, 1, false>(p, rg, ks, sbw, st);
    } else {
        mmq_launch_t<LH_Q6_K, 2, false>(p, rg, ks, sbw, st);
    }
    note_launch();
    return true;
}

} // namespace lh
