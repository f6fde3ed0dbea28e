// mmq.hip -- grouped int8 matrix-core matmul for Q4_K / Q6_K weights against
// int8 activations, bit-identical to the reference CPU kernels
// (src/gguf/ggml.zig:1002-1059 kBlockDot / matvecK256 / matmulK256) and so
// to dmmv.hip.
//
// The integer part of every block dot runs on v_mfma_i32_16x16x32_i8: the
// activations of 16 tokens are the A rows, 16 weight rows the B columns, K a
// 32-value sub-block (Q4_K: one scale group; Q6_K: two 16-value runs, one
// MFMA each with the other run's lanes zeroed).  Integer dots are exact in any
// order, so isum = sum sc * dot and msum = sum mn * bsum are the reference's
// integers; the f32 tail per (token, row, super-block) is the reference's
// expression, and each output sums its blocks in block order from LDS.
//
// Lane l of a wave: weight row l % 16 of its 16-row tile, k-quarter l / 16
// (8 values); the result lane l holds tokens 4*(l/16) .. +3 of that row.
#include "fmt.hpp"
#include "kernels.hpp"

namespace lh {

typedef int mmq_i4 __attribute__((ext_vector_type(4)));

constexpr uint64_t NIB = 0x0F0F0F0F0F0F0F0Full;

// Activation sums a tile keeps in LDS per token: per 32 values for Q4_K's
// mins, per 16 for Q6_K's -32 offsets.
template <int T> constexpr int sum_span() { return T == LH_Q4_K ? 32 : 16; }

// Token rows of sums are padded by 4 ints: the four tokens a lane reads sit
// in different banks.
static size_t mmq_lds_bytes(int t, int cols, int mt, int rg, bool fused) {
    const int nb = cols / 256, tok = 16 * mt, ks = 4 / rg;
    const size_t sums = (size_t)tok * (cols / (t == LH_Q4_K ? 32 : 16) + 4);
    const size_t part = ks > 1 ? (size_t)(fused ? 2 : 1) * rg * 16 * tok * nb : 0;
    return 4 * (sums + (size_t)tok * nb + part);
}

// Q4_K: one super-block's tail values r[mt][i] (token 16*mt + 4*q4 + i,
// weight row of this lane's column).
template <int MT>
__device__ __forceinline__ void q4k_block(const uint8_t *blk, const int8_t *const xrow[MT], int b, int q4,
                                          const int32_t *xs, const float *xdl, int nb, int nsum, float r[MT][4]) {
    const uint4 hdr = *(const uint4 *)blk;
    uint64_t nib[4];
#pragma unroll
    for (int p = 0; p < 4; p++)
        nib[p] = *(const uint64_t *)(blk + 16 + 32 * p + 8 * q4);
    int sc[8], mn[8];
#pragma unroll
    for (int p = 0; p < 4; p++)
        Fmt<LH_Q4_K>::scales(hdr, 2 * p, sc[2 * p], mn[2 * p], sc[2 * p + 1], mn[2 * p + 1]);
    const float d = half_bits_to_float(hdr.x & 0xffff);
    const float dmin = half_bits_to_float(hdr.x >> 16);
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const uint64_t wv = g & 1 ? (nib[g >> 1] >> 4) & NIB : nib[g >> 1] & NIB;
            const long xa = *(const long *)(xrow[mt] + 256 * b + 32 * g + 8 * q4);
            const mmq_i4 z = {0, 0, 0, 0};
            const mmq_i4 dd = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, (long)wv, z, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
                isum[i] += sc[g] * dd[i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tk = 16 * mt + 4 * q4 + i;
            const int4 s0 = *(const int4 *)(xs + tk * nsum + 8 * b);
            const int4 s1 = *(const int4 *)(xs + tk * nsum + 8 * b + 4);
            const int msum = mn[0] * s0.x + mn[1] * s0.y + mn[2] * s0.z + mn[3] * s0.w + mn[4] * s1.x +
                             mn[5] * s1.y + mn[6] * s1.z + mn[7] * s1.w;
            // xb.d * (d * f32(isum) - dmin * f32(min_isum))  (ggml.zig:1016-1017)
            const float a = d * (float)isum[i];
            const float bb = dmin * (float)msum;
            r[mt][i] = xdl[tk * nb + b] * (a - bb);
        }
    }
}

// Q6_K (device SoA ql[U][128] | qh[U][64] | sc[U][16] | d[U]).
template <int MT>
__device__ __forceinline__ void q6k_block(const uint8_t *base, size_t U, size_t unit, const int8_t *const xrow[MT],
                                          int b, int q4, const int32_t *xs, const float *xdl, int nb, int nsum,
                                          float r[MT][4]) {
    uint64_t ql[2][2], qh[2];
#pragma unroll
    for (int n = 0; n < 2; n++) {
#pragma unroll
        for (int o = 0; o < 2; o++)
            ql[n][o] = *(const uint64_t *)(base + unit * 128 + 64 * n + 32 * o + 8 * q4);
        qh[n] = *(const uint64_t *)(base + U * 128 + unit * 64 + 32 * n + 8 * q4);
    }
    const uint4 scv = *(const uint4 *)(base + U * 192 + unit * 16);
    const float dw = half_bits_to_float(*(const uint16_t *)(base + U * 208 + unit * 2));
    int sc[16];
#pragma unroll
    for (int k = 0; k < 16; k++)
        sc[k] = (int)(int8_t)byte_of(scv, k);
    const bool lo_run = q4 < 2; // values 32g + 8*q4 .. +7 lie in run 2g (q4 < 2) or 2g+1
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int n = g >> 2, qd = g & 3;
            const uint64_t l4 = qd >= 2 ? (ql[n][qd & 1] >> 4) & NIB : ql[n][qd & 1] & NIB;
            const uint64_t v = l4 | (((qh[n] >> (2 * qd)) & 0x0303030303030303ull) << 4);
            const long xa = *(const long *)(xrow[mt] + 256 * b + 32 * g + 8 * q4);
            const mmq_i4 z = {0, 0, 0, 0};
            const mmq_i4 d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, lo_run ? (long)v : 0l, z, 0, 0, 0);
            const mmq_i4 d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, lo_run ? 0l : (long)v, z, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
                isum[i] += sc[2 * g] * d0[i] + sc[2 * g + 1] * d1[i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tk = 16 * mt + 4 * q4 + i;
            // weights are q-32: dot(q-32, x) = dot(q, x) - 32*sum(x) per run
            int corr = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int4 sv = *(const int4 *)(xs + tk * nsum + 16 * b + 4 * c);
                corr += sc[4 * c] * sv.x + sc[4 * c + 1] * sv.y + sc[4 * c + 2] * sv.z + sc[4 * c + 3] * sv.w;
            }
            // xb.d * dec.d * f32(isum)  (ggml.zig:1019)
            const float s = xdl[tk * nb + b] * dw;
            r[mt][i] = s * (float)(isum[i] - 32 * corr);
        }
    }
}

template <int T, int MT>
__device__ __forceinline__ void mmq_block(const uint8_t *wb, size_t U, int row, int b, const int8_t *const xrow[MT],
                                          int q4, const int32_t *xs, const float *xdl, int nb, int nsum,
                                          float r[MT][4]) {
    const size_t unit = (size_t)row * nb + b;
    if constexpr (T == LH_Q4_K)
        q4k_block<MT>(wb + unit * 144, xrow, b, q4, xs, xdl, nb, nsum, r);
    else
        q6k_block<MT>(wb, U, unit, xrow, b, q4, xs, xdl, nb, nsum, r);
}

// Work group: 16*RG weight rows x 16*MT tokens of one group; wave w takes
// row group w % RG and, with KS = 4/RG waves per row group, super-blocks
// w/RG, w/RG + KS, ...  With KS == 1 a wave owns whole rows and sums their
// blocks in order in registers; otherwise the per-block values meet in LDS
// and are summed in block order there.
template <int T, int MT, int RG, bool FUSED>
__global__ __launch_bounds__(256) void mmq_kernel(DmmvParams p) {
    extern __shared__ __align__(16) int32_t mlds[];
    __shared__ int vec[16 * MT];
    constexpr int TOK = 16 * MT, KS = 4 / RG, SPAN = sum_span<T>();
    const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
    if ((int)blockIdx.y >= ng)
        return;
    const DmmvGroup grp = p.groups[blockIdx.y];
    const int n = grp.n, cols = p.cols, nb = cols / 256, nsr = cols / SPAN, nsum = nsr + 4, n16 = cols / 16;
    const int tid = threadIdx.x, wave = tid >> 6, ln = tid & 63, r16 = ln & 15, q4 = ln >> 4;
    const int rg = wave % RG, ks = wave / RG;
    const int row0 = blockIdx.x * 16 * RG;
    int32_t *xs = mlds;                          // [TOK][nsum] (nsr used)
    float *xdl = (float *)(xs + TOK * nsum);     // [TOK][nb]
    float *part = xdl + TOK * nb;                // [FUSED + 1][RG * 16][TOK][nb] (KS > 1)
    if (tid < TOK)
        vec[tid] = p.pair_src[grp.first + (tid < n ? tid : n - 1)];
    __syncthreads();
    // per-SPAN sums from the per-16 sums (exact integers)
    for (int i = tid; i < TOK * nsr; i += 256) {
        const int tk = i / nsr, k = i % nsr;
        const int32_t *sv = p.xs + (size_t)vec[tk] * n16 + k * (SPAN / 16);
        xs[tk * nsum + k] = SPAN == 32 ? sv[0] + sv[1] : sv[0];
    }
    for (int i = tid; i < TOK * nb; i += 256)
        xdl[i] = p.xd[(size_t)vec[i / nb] * nb + i % nb];
    __syncthreads();
    const int8_t *xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        xrow[mt] = p.xq + (size_t)vec[16 * mt + r16] * cols;
    const int rl = 16 * rg + r16; // row within the tile
    const int row = min(row0 + rl, p.rows - 1);
    const size_t U = (size_t)p.rows * nb;
    const uint8_t *wb = p.w + (size_t)grp.plane * p.plane_bytes;
    const uint8_t *wb2 = FUSED ? p.w2 + (size_t)grp.plane * p.plane_bytes : nullptr;
    if constexpr (KS == 1) {
        float acc[MT][4], acc2[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                acc[mt][i] = acc2[mt][i] = 0.0f;
        for (int b = 0; b < nb; b++) { // block order: the reference's acc += r
            float r[MT][4];
            mmq_block<T, MT>(wb, U, row, b, xrow, q4, xs, xdl, nb, nsum, r);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[mt][i] = acc[mt][i] + r[mt][i];
            if constexpr (FUSED) {
                mmq_block<T, MT>(wb2, U, row, b, xrow, q4, xs, xdl, nb, nsum, r);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc2[mt][i] = acc2[mt][i] + r[mt][i];
            }
        }
        if (row0 + rl >= p.rows)
            return;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tk = 16 * mt + 4 * q4 + i;
                if (tk >= n)
                    continue;
                const float v = FUSED ? swiglu1(acc[mt][i], acc2[mt][i]) : acc[mt][i];
                float *o = p.out + (size_t)p.pair_dst[grp.first + tk] * p.out_stride + row0 + rl;
                *o = p.accumulate ? *o + v : v;
            }
    } else {
        constexpr int R = RG * 16;
        for (int b = ks; b < nb; b += KS) {
            float r[MT][4];
            mmq_block<T, MT>(wb, U, row, b, xrow, q4, xs, xdl, nb, nsum, r);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    part[((size_t)rl * TOK + 16 * mt + 4 * q4 + i) * nb + b] = r[mt][i];
            if constexpr (FUSED) {
                mmq_block<T, MT>(wb2, U, row, b, xrow, q4, xs, xdl, nb, nsum, r);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        part[(size_t)R * TOK * nb + ((size_t)rl * TOK + 16 * mt + 4 * q4 + i) * nb + b] =
                            r[mt][i];
            }
        }
        __syncthreads();
        for (int idx = tid; idx < n * R; idx += 256) {
            const int tk = idx / R, rr = idx % R;
            if (row0 + rr >= p.rows)
                continue;
            float *o = p.out + (size_t)p.pair_dst[grp.first + tk] * p.out_stride + row0 + rr;
            const float v = row_value<FUSED>(part, (size_t)R * TOK * nb, (size_t)rr * TOK + tk, nb);
            *o = p.accumulate ? *o + v : v;
        }
    }
}

// Row groups per work group: whole rows per wave (RG = 4) when that still
// gives >= 512 work groups, else the super-blocks split over the waves.
static int mmq_pick_rg(int rows, int groups, int nb) {
    if ((long)((rows + 63) / 64) * groups >= 512 || nb < 2)
        return 4;
    if ((long)((rows + 31) / 32) * groups >= 512 || nb < 4)
        return 2;
    return 1;
}

bool mmq_supported(int t, int cols, int max_tok, bool fused) {
    if ((t != LH_Q4_K && t != LH_Q6_K) || cols % 256 || max_tok < 1 || max_tok > 32)
        return false;
    if (fused && t != LH_Q4_K) // a fused pair is gate/up: Q4_K only here
        return false;
    return mmq_lds_bytes(t, cols, (max_tok + 15) / 16, 1, fused) <= 64 * 1024;
}

template <int T, int MT, bool FUSED>
static void mmq_launch_rg(int rg, const DmmvParams &p, hipStream_t st) {
    const size_t lds = mmq_lds_bytes(T, p.cols, MT, rg, FUSED);
    const dim3 grid((p.rows + 16 * rg - 1) / (16 * rg), p.n_groups);
    if (rg == 4)
        hipLaunchKernelGGL((mmq_kernel<T, MT, 4, FUSED>), grid, dim3(256), lds, st, p);
    else if (rg == 2)
        hipLaunchKernelGGL((mmq_kernel<T, MT, 2, FUSED>), grid, dim3(256), lds, st, p);
    else
        hipLaunchKernelGGL((mmq_kernel<T, MT, 1, FUSED>), grid, dim3(256), lds, st, p);
}

// Groups of at most max_tok (<= 32) tokens; p.rpw is unused.
bool launch_mmq(int t, int max_tok, bool fused, const DmmvParams &p, hipStream_t st) {
    if (!mmq_supported(t, p.cols, max_tok, fused))
        return false;
    const int mt = max_tok > 16 ? 2 : 1;
    const int rg = mmq_pick_rg(p.rows, p.n_groups, p.cols / 256);
    if (mmq_lds_bytes(t, p.cols, mt, rg, fused) > 64 * 1024)
        return false;
    if (t == LH_Q4_K) {
        if (mt == 1)
            fused ? mmq_launch_rg<LH_Q4_K, 1, true>(rg, p, st) : mmq_launch_rg<LH_Q4_K, 1, false>(rg, p, st);
        else
            fused ? mmq_launch_rg<LH_Q4_K, 2, true>(rg, p, st) : mmq_launch_rg<LH_Q4_K, 2, false>(rg, p, st);
    } else if (mt == 1) {
        mmq_launch_rg<LH_Q6_K, 1, false>(rg, p, st);
    } else {
        mmq_launch_rg<LH_Q6_K, 2, false>(rg, p, st);
    }
    note_launch();
    return true;
}

} // namespace lh
