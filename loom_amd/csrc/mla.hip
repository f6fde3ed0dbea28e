// mla.hip -- Multi-head Latent Attention over the compressed cache, the
// seam's mlaInit / mlaAppend / mlaReadCache / mlaSetWk / mlaAttnHeads
// (src/compute/backend.zig:162-169,193-197), in the reference's own
// evaluation order (the host head loop, src/gguf/deepseek.zig:988-1047):
//
//   qa   = 0;  qa = qa + q_nope[r] * W_k[r], r = 0 .. nope-1   (axpy, ggml.zig:222-231)
//   s_t  = (dotF32(qa, c_t) + dotF32(q_rope, kr_t)) * scale     (ggml.zig:198-217)
//   p    = softmax(s): the position-ordered sum                 (tensor.zig:18-28)
//   o    = 0;  o = o + p_t * c_t, t = 0 .. seq-1                (axpy)
//   out  = W_v . o, int8 activations                            (ggml.zig:602)
//
// so the compressed output o and the head outputs are bit-identical to
// Loom's CPU path at every context length.  kv_b (rows h*(nope+vd) ..
// +nope: head h's W_k, the next vd rows its W_v, each kvr long) is split per
// head into W_k and W_v planes of the device layout once; the absorb reads
// the quantized W_k and dequantizes in the kernel (the f32 copy the seam's
// mlaSetWk offers holds the same values at 7x the bytes).  Five launches:
//
//   mla_absorb_kernel   one lane per (head, latent column): the chain over r
//   mla_scores_kernel   a (32 heads x 16 positions) tile per work group; each
//                       half-wave owns 8 heads x 8 positions and its 32 lanes
//                       are dotF32's 32 accumulators (lane j: k = j mod 32),
//                       combined per output through LDS in dotF32's order
//   mla_softmax_kernel  one work group per head: max, exp, the ordered sum
//   mla_wsum_kernel     one lane per (head, latent column): the chain over t
//   W_v                 quant_act + the grouped matvec, plane = head
#include "frame.hpp"
#include "runtime.hpp"

#include <mutex>
#include <string>
#include <vector>

namespace lh {

constexpr int MLA_MAX_CTX = EXACT_MAX_CTX; // the softmax row's LDS
constexpr int MLA_MAX_KVR = 4096;
constexpr int MLA_MAX_ROPE = 512;

// ---- absorb -----------------------------------------------------------------
// qa[h][c] = chain over r of q_nope[h][r] * W_k[h][r][c] (product rounded,
// then added), from +0.  Work group (256 latent columns, head h), rows in
// chunks of MA_ROWS: the chunk's blocks of the head's W_k over those columns
// are copied into LDS with 16-byte loads as a compact plane of the same
// device layout (U' = rows x blocks), the scale-group pairs (a, b) of every
// row are decoded from it once, then each thread runs its column's chain with
// value = a * q - b (the dequant's own rounding).
constexpr int MA_THREADS = 256;
constexpr int MA_SLOTS = 16;     // scale groups in 256 columns, at most (Q6_K)
constexpr int MA_ROWS = 128;     // rows per LDS chunk
constexpr int MA_MAX_NOPE = 256;
constexpr int MA_STAGE = MA_ROWS * 8 * 34 + 64; // bytes of the largest chunk (Q8_0: 8 blocks of 34 bytes a row)

// The arrays of a block in the device layout: (offset of the array in units
// of U, bytes per block).  The d arrays (2 bytes a block) come last.
template <int T>
__device__ constexpr int ma_arrays() { return T == LH_Q4_K ? 1 : T == LH_Q6_K ? 4 : 2; }
template <int T>
__device__ constexpr int ma_off(int a) {
    return T == LH_Q4_K ? 0 : T == LH_Q6_K ? (a == 0 ? 0 : a == 1 ? 128 : a == 2 ? 192 : 208)
                                          : (a == 0 ? 0 : T == LH_Q8_0 ? 32 : 16);
}
template <int T>
__device__ constexpr int ma_bytes(int a) {
    return T == LH_Q4_K ? 144 : T == LH_Q6_K ? (a == 0 ? 128 : a == 1 ? 64 : a == 2 ? 16 : 2)
                                            : (a == 0 ? (T == LH_Q8_0 ? 32 : 16) : 2);
}

template <int T>
__global__ __launch_bounds__(MA_THREADS) void mla_absorb_kernel(const uint8_t *__restrict__ wk, size_t plane,
                                                                const float *__restrict__ q_nope, int nope, int kvr,
                                                                float *__restrict__ qa) {
    constexpr int BE = block_elems(T), GPB = dq_groups(T);
    __shared__ __align__(16) uint8_t stage[MA_STAGE];
    __shared__ float2 pairs[MA_ROWS * MA_SLOTS];
    __shared__ float qn[MA_MAX_NOPE];
    const int h = blockIdx.y, c0 = blockIdx.x * MA_THREADS, tid = threadIdx.x;
    const int nb = kvr / BE;
    const uint8_t *w = wk + (size_t)h * plane;
    const size_t U = (size_t)nope * nb;
    const int b0 = c0 / BE, nblk = (min(MA_THREADS, kvr - c0) + BE - 1) / BE, nslots = nblk * GPB;
    for (int i = tid; i < nope; i += MA_THREADS)
        qn[i] = q_nope[(size_t)h * nope + i];
    const int c = min(c0 + tid, kvr - 1), cb = c / BE - b0, e = c % BE;
    const int slot = cb * GPB + dq_group(T, e);
    float acc = 0.0f;
    for (int r0 = 0; r0 < nope; r0 += MA_ROWS) {
        const int rows = min(MA_ROWS, nope - r0);
        const int Uc = rows * nblk; // blocks of the compact plane
        __syncthreads();            // the previous chunk's reads are done
#pragma unroll
        for (int a = 0; a < ma_arrays<T>(); a++) {
            const int bb = ma_bytes<T>(a);
            const uint8_t *src = w + (size_t)ma_off<T>(a) * U;
            uint8_t *dst = stage + ma_off<T>(a) * Uc;
            if (bb >= 16) {
                const int per_row = nblk * bb / 16; // 16-byte pieces of a row's blocks
                for (int i = tid; i < rows * per_row; i += MA_THREADS) {
                    const int r = i / per_row, k = i % per_row;
                    *(uint4 *)(dst + (size_t)r * nblk * bb + 16 * k) =
                        *(const uint4 *)(src + ((size_t)(r0 + r) * nb + b0) * bb + 16 * k);
                }
            } else {
                for (int i = tid; i < rows * nblk; i += MA_THREADS) {
                    const int r = i / nblk, k = i % nblk;
                    ((uint16_t *)dst)[i] = ((const uint16_t *)src)[(size_t)(r0 + r) * nb + b0 + k];
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < rows * nslots; i += MA_THREADS) {
            const int r = i / nslots, sl = i % nslots;
            pairs[r * MA_SLOTS + sl] = dq_pair(T, stage, (size_t)Uc, (size_t)r * nblk + sl / GPB, sl % GPB);
        }
        __syncthreads();
#pragma unroll 16
        for (int r = 0; r < rows; r++) {
            const int q = dq_q(T, stage, (size_t)Uc, (size_t)r * nblk + cb, e);
            const float p = qn[r0 + r] * dq_apply(pairs[r * MA_SLOTS + slot], q);
            acc = acc + p;
        }
    }
    if (c0 + tid < kvr)
        qa[(size_t)h * kvr + c0 + tid] = acc;
}

// ---- scores -----------------------------------------------------------------
constexpr int MS_THREADS = 256; // 4 waves
constexpr int MS_HPW = 8;       // heads per wave (both half-waves)
constexpr int MS_TPH = 8;       // positions per half-wave
constexpr int MS_HEADS = (MS_THREADS / 64) * MS_HPW;
constexpr int MS_POS = 2 * MS_TPH;
constexpr int MS_PST = 36; // f32 stride of one output's 32 partials (16-byte reads hit 16 distinct slots)
constexpr int MS_ROUND = MS_HPW / 2 * MS_TPH; // outputs combined per round and half-wave (one per lane)

// dotF32's 32 accumulators spread over a half-wave: lane j adds A[i][k] *
// B[m][k] for k = j, j + 32, ... over the whole 32-steps, then (lanes 0..7)
// the leftover 8-chunks, for the 8 rows arow[] of A and the 8 rows brow[] of B.
__device__ __forceinline__ void mla_partials(const float *A, const int (&arow)[MS_HPW], const float *B,
                                             const int (&brow)[MS_TPH], int n, int j,
                                             float (&acc)[MS_HPW][MS_TPH]) {
#pragma unroll
    for (int i = 0; i < MS_HPW; i++)
#pragma unroll
        for (int m = 0; m < MS_TPH; m++)
            acc[i][m] = 0.0f;
    const int n32 = n / 32 * 32, n8 = n / 8 * 8;
    auto step = [&](int k) {
        float a[MS_HPW], b[MS_TPH];
#pragma unroll
        for (int i = 0; i < MS_HPW; i++)
            a[i] = A[(size_t)arow[i] * n + k];
#pragma unroll
        for (int m = 0; m < MS_TPH; m++)
            b[m] = B[(size_t)brow[m] * n + k];
#pragma unroll
        for (int i = 0; i < MS_HPW; i++)
#pragma unroll
            for (int m = 0; m < MS_TPH; m++) {
                const float p = a[i] * b[m];
                acc[i][m] = acc[i][m] + p;
            }
    };
    for (int k = j; k < n32; k += 32)
        step(k);
    if (j < 8)
        for (int k = n32 + j; k < n8; k += 8)
            step(k);
}

// One output's dotF32 from its 32 partials (LDS): per vector lane l,
// ((p[l] + p[8+l]) + p[16+l]) + p[24+l]; the 8 lanes summed in order from -0
// (@reduce, as dot_f32_key); then the elements past the last 8-chunk.
__device__ __forceinline__ float mla_finish(const float *part, const float *a, const float *b, int n) {
    float p[32];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const float4 v = *(const float4 *)(part + 4 * q);
        p[4 * q] = v.x;
        p[4 * q + 1] = v.y;
        p[4 * q + 2] = v.z;
        p[4 * q + 3] = v.w;
    }
    float s = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++)
        s = s + (((p[l] + p[8 + l]) + p[16 + l]) + p[24 + l]);
    for (int i = n / 8 * 8; i < n; i++) {
        const float q = a[i] * b[i];
        s = s + q;
    }
    return s;
}

// One dot per (A row, B row) of the tile: acc -> LDS -> the lane's output of
// each round (round r: A rows 4r .. 4r+3; lane j: A row 4r + j/8, B row j%8),
// into res[r].  A and B rows are n long.
__device__ __forceinline__ void mla_dot_tile(const float *A, const int (&arow)[MS_HPW], const float *B,
                                             const int (&brow)[MS_TPH], int n, int j, float *part,
                                             float (&res)[2]) {
    float acc[MS_HPW][MS_TPH];
    mla_partials(A, arow, B, brow, n, j, acc);
#pragma unroll
    for (int r = 0; r < 2; r++) {
        __syncthreads(); // the previous round's reads are done
#pragma unroll
        for (int i = 0; i < MS_HPW / 2; i++)
#pragma unroll
            for (int m = 0; m < MS_TPH; m++)
                part[(i * MS_TPH + m) * MS_PST + j] = acc[4 * r + i][m];
        __syncthreads();
        const int i = 4 * r + (j >> 3), m = j & 7;
        res[r] = mla_finish(part + j * MS_PST, A + (size_t)arow[i] * n, B + (size_t)brow[m] * n, n);
    }
}

// Work group: heads hb .. (wave w: blockIdx.y * 32 + 8w ..), positions
// (half-wave hw: blockIdx.x * 16 + 8hw ..).  Rows past the heads or the
// context read the last row; their outputs are not stored.
__global__ __launch_bounds__(MS_THREADS) void mla_scores_kernel(
    const float *__restrict__ qa, const float *__restrict__ q_rope, const float *__restrict__ c_kv,
    const float *__restrict__ k_rope, int seq, int H, int kvr, int rope, float scale, float *__restrict__ S,
    int s_stride) {
    __shared__ __align__(16) float lds[MS_THREADS / 64][2][MS_ROUND * MS_PST];
    const int wave = threadIdx.x >> 6, ln = threadIdx.x & 63, hw = ln >> 5, j = ln & 31;
    const int hb = blockIdx.y * MS_HEADS + wave * MS_HPW, tb = blockIdx.x * MS_POS + hw * MS_TPH;
    int arow[MS_HPW], brow[MS_TPH];
#pragma unroll
    for (int i = 0; i < MS_HPW; i++)
        arow[i] = min(hb + i, H - 1);
#pragma unroll
    for (int m = 0; m < MS_TPH; m++)
        brow[m] = min(tb + m, seq - 1);
    float *part = lds[wave][hw];
    float dc[2], dr[2];
    mla_dot_tile(qa, arow, c_kv, brow, kvr, j, part, dc);
    mla_dot_tile(q_rope, arow, k_rope, brow, rope, j, part, dr);
    const int t = tb + (j & 7);
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int h = hb + 4 * r + (j >> 3);
        if (h < H && t < seq)
            S[(size_t)h * s_stride + t] = (dc[r] + dr[r]) * scale;
    }
}

// ---- softmax ----------------------------------------------------------------
template <int NT>
__global__ __launch_bounds__(NT) void mla_softmax_kernel(float *__restrict__ S, int s_stride, int seq) {
    extern __shared__ __align__(16) float e[]; // e[s_stride]
    __shared__ float redf[NT / 64];
    __shared__ SeqSumLds sq;
    float *row = S + (size_t)blockIdx.x * s_stride;
    softmax_row_exact<NT>(row, seq, e, redf, sq);
    for (int j = seq + threadIdx.x; j < s_stride; j += NT) // the weighted sum's padding
        row[j] = 0.0f;
}

// ---- weighted sum of the cached rows ------------------------------------------
// o[h][c] = chain over t of p[h][t] * c_kv[t][c] (product rounded, then
// added), from +0.  Wave = head, lane = latent column: a work group's four
// waves take four heads over the same 64 columns, and the work groups of one
// column tile are ntile apart in launch order (with kvr 512 each tile's rows
// stay in one XCD's L2: work groups go round-robin over the 8 XCDs).  The
// rows come through LDS in tiles of MW_TP positions: loaded MW_AHEAD tiles
// ahead with 16-byte loads, stored transposed (row = column, each 4-position
// chunk at chunk q ^ (column >> 4), which keeps the stores and the 16-byte
// reads free of bank conflicts) into one of 3 buffers.  Each tile begins with
// one wait for its own values (read the tile before) and then issues the next
// tile's LDS reads and its p loads (scalar: p is uniform over the wave), so
// they are in flight while this tile's products and adds run.  The last tile
// runs whole: past seq both p (the softmax writes +0 up to the row's end) and
// the rows (loaded as +0) are zero, and o + (+-0) is o (o starts at +0 and a
// sum of products never reaches -0 from there), so the padding is exact.
constexpr int MW_TP = 32;
constexpr int MW_AHEAD = 2;
constexpr int MW_NB = 3;
constexpr int MW_RS = MW_TP + 4;          // f32 row stride of a transposed tile
constexpr int MW_NF = MW_TP * 16 / 256;   // 16-byte loads per thread per tile
static_assert(MW_AHEAD % 2 == 0, "the value registers alternate with the tile's parity");
typedef const __attribute__((address_space(4))) float const_f32;
__global__ __launch_bounds__(256) void mla_wsum_kernel(const float *__restrict__ S, int s_stride,
                                                       const float *__restrict__ c_kv, int seq, int H, int kvr,
                                                       int ntile, float *__restrict__ o_lat) {
    __shared__ __align__(16) float tl[MW_NB][64 * MW_RS];
    const int id = blockIdx.x, tile = id % ntile, hg = id / ntile;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), ln = tid & 63;
    const int h = hg * 4 + wave, hc = min(h, H - 1);
    const int c = tile * 64 + ln;
    const_f32 *pr = (const_f32 *)(S + (size_t)hc * s_stride);
    const int ntl = (seq + MW_TP - 1) / MW_TP;
    // rows past seq read row seq - 1, columns past kvr read columns kvr - 4 ..
    // (their results are not stored)
    auto gload = [&](int k, float4 (&r)[MW_NF]) {
#pragma unroll
        for (int j = 0; j < MW_NF; j++) {
            const int f = tid + 256 * j, pos = f / 16, c4 = f % 16;
            const int tt = k * MW_TP + pos;
            const int cc = min(tile * 64 + 4 * c4, kvr - 4);
            const float4 v = *(const float4 *)(c_kv + (size_t)min(tt, seq - 1) * kvr + cc);
            r[j] = tt < seq ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto lstore = [&](int buf, const float4 (&r)[MW_NF]) {
#pragma unroll
        for (int j = 0; j < MW_NF; j++) {
            const int f = tid + 256 * j, pos = f / 16, c4 = f % 16;
            const int q = pos >> 2, w = pos & 3;
            const float vals[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int row = 4 * c4 + e;
                tl[buf][row * MW_RS + 4 * (q ^ (row >> 4)) + w] = vals[e];
            }
        }
    };
    auto lread = [&](int k, float4 (&x)[MW_TP / 4]) {
        const float *src = tl[k % MW_NB] + ln * MW_RS;
#pragma unroll
        for (int q = 0; q < MW_TP / 4; q++)
            x[q] = *(const float4 *)(src + 4 * (q ^ (ln >> 4)));
    };
    // p of tile k (a tile starting past the row also starts past seq: its
    // values are never used)
    auto pload = [&](float (&p)[MW_TP], int k) {
        const int base = min(k * MW_TP, s_stride - MW_TP);
#pragma unroll
        for (int u = 0; u < MW_TP; u++)
            p[u] = pr[base + u];
    };
    float acc = 0.0f;
    auto tilek = [&](int k, const float4 (&xc)[MW_TP / 4], const float (&pc)[MW_TP], float4 (&xn)[MW_TP / 4],
                     float (&pn)[MW_TP], float4 (&r)[MW_NF]) {
        __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): this tile's values and p
        __builtin_amdgcn_sched_barrier(0);
        if (k + 1 < ntl)
            lread(k + 1, xn);
        pload(pn, k + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < MW_TP / 4; q++) {
            const float xs[4] = {xc[q].x, xc[q].y, xc[q].z, xc[q].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float m = pc[4 * q + e] * xs[e];
                acc = acc + m;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // tile k + 2 (in r) into the buffer tile k - 1 left; tile k + 2 + AHEAD's loads go out
        lstore((k + 2) % MW_NB, r);
        gload(k + 2 + MW_AHEAD, r);
        __syncthreads();
    };
    float4 rg[MW_AHEAD][MW_NF];
    float4 xa[MW_TP / 4], xb[MW_TP / 4];
    float pa[MW_TP], pb[MW_TP];
    gload(0, rg[0]);
    lstore(0, rg[0]);
    gload(1, rg[0]);
    lstore(1, rg[0]);
#pragma unroll
    for (int a = 0; a < MW_AHEAD; a++)
        gload(2 + a, rg[a]);
    __syncthreads();
    lread(0, xa);
    pload(pa, 0);
    for (int k0 = 0; k0 < ntl; k0 += MW_AHEAD) {
#pragma unroll
        for (int a = 0; a < MW_AHEAD; a++) {
            const int k = k0 + a;
            if (k < ntl) {
                if (a & 1)
                    tilek(k, xb, pb, xa, pa, rg[a]);
                else
                    tilek(k, xa, pa, xb, pb, rg[a]);
            }
        }
    }
    if (h < H && c < kvr)
        o_lat[(size_t)h * kvr + c] = acc;
}

// ---- host ---------------------------------------------------------------------

struct KvbSplit {
    int t = -1;
    size_t len = 0, H = 0, nope = 0, vd = 0, kvr = 0;
    void *wk = nullptr, *wv = nullptr;
};

struct Mla {
    std::mutex mu;
    // the seam's device cache: c rows [layers][ctx][kvr], then rope rows [layers][ctx][rope]
    float *cache = nullptr;
    size_t layers = 0, ctx = 0, kvr = 0, rope = 0;
    bool want = false;
    size_t wk_layers = 0;
    Scratch qa, S, olat, act, kvb_stage, tail, act2, frame;
    std::unordered_map<std::string, float *> yarn; // rope (cos, sin) tables per shape
    std::unordered_map<size_t, void *> vgroups; // per head count: groups {h, h, 1}
    std::unordered_map<const void *, KvbSplit> kvb;
};
static Mla g_mla;

static int reserve_on(Scratch &s, size_t bytes, hipStream_t st) {
    if (bytes > s.cap)
        (void)hipStreamSynchronize(st);
    return s.reserve(bytes);
}

static const DmmvGroup *head_groups(size_t H) {
    auto it = g_mla.vgroups.find(H);
    if (it != g_mla.vgroups.end())
        return (const DmmvGroup *)it->second;
    std::vector<DmmvGroup> g(H);
    for (size_t h = 0; h < H; h++)
        g[h] = DmmvGroup{(int)h, (int)h, 1};
    void *d = nullptr;
    if (hipMalloc(&d, sizeof(DmmvGroup) * H) != hipSuccess)
        return nullptr;
    if (hipMemcpy(d, g.data(), sizeof(DmmvGroup) * H, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return nullptr;
    }
    g_mla.vgroups[H] = d;
    return (const DmmvGroup *)d;
}

static int mla_check(const loomhip_mla_attn *a, size_t seq) {
    if (!a || !a->wk || !a->wv)
        return fail(LOOMHIP_ERR_ARG, "mla: null weights");
    if (a->n_heads == 0 || a->nope == 0 || a->vd == 0 || a->kvr == 0 || a->rope == 0)
        return fail(LOOMHIP_ERR_ARG, "mla: empty shape");
    if (a->nope > (size_t)MA_MAX_NOPE)
        return fail(LOOMHIP_DECLINED, "mla: nope %zu over %d", a->nope, MA_MAX_NOPE);
    if (seq == 0 || seq > (size_t)MLA_MAX_CTX)
        return fail(LOOMHIP_DECLINED, "mla: context %zu outside 1..%d", seq, MLA_MAX_CTX);
    if (a->kvr > (size_t)MLA_MAX_KVR || a->rope > (size_t)MLA_MAX_ROPE || a->n_heads > (size_t)IOTA_LEN)
        return fail(LOOMHIP_DECLINED, "mla: kvr %zu / rope %zu / heads %zu not served", a->kvr, a->rope, a->n_heads);
    if (a->kvb_type == LH_F32 || a->kvb_type == LH_F16 || !dmmv_supported(a->kvb_type, (int)a->kvr))
        return fail(LOOMHIP_DECLINED, "mla: kv_b type %d with %zu columns not served", a->kvb_type, a->kvr);
    return LOOMHIP_OK;
}

static int mla_attn_impl(const loomhip_mla_attn *a, const float *c_kv, const float *k_rope, size_t seq,
                         const float *q_nope, const float *q_rope, float *out, float *o_lat, hipStream_t st) {
    if (int rc = mla_check(a, seq))
        return rc;
    const int t = a->kvb_type;
    const size_t H = a->n_heads, kvr = a->kvr, s_stride = (seq + 63) / 64 * 64;
    const size_t qbytes = align16(H * kvr) + align16(H * kvr / 32 * 4) + align16(H * kvr / 16 * 4);
    int rc;
    if ((rc = reserve_on(g_mla.qa, H * kvr * 4, st)) || (rc = reserve_on(g_mla.S, H * s_stride * 4, st)) ||
        (rc = reserve_on(g_mla.act, qbytes, st)) || (!o_lat && (rc = reserve_on(g_mla.olat, H * kvr * 4, st))))
        return rc;
    const DmmvGroup *groups = head_groups(H);
    if (!groups)
        return fail(LOOMHIP_ERR_HIP, "mla: head group table");
    float *qa = (float *)g_mla.qa.ptr, *S = (float *)g_mla.S.ptr;
    float *ol = o_lat ? o_lat : (float *)g_mla.olat.ptr;
    // 1. absorb
    int ph = prof_begin(LOOMHIP_KT_MLA_ABSORB, st);
    {
        const dim3 g((unsigned)((kvr + MA_THREADS - 1) / MA_THREADS), (unsigned)H);
        const size_t pl = plane_bytes(t, a->nope, kvr);
        const uint8_t *wk = (const uint8_t *)a->wk;
        const int nope = (int)a->nope;
        switch (t) {
        case LH_Q4_K:
            hipLaunchKernelGGL((mla_absorb_kernel<LH_Q4_K>), g, dim3(MA_THREADS), 0, st, wk, pl, q_nope, nope, (int)kvr, qa);
            break;
        case LH_Q6_K:
            hipLaunchKernelGGL((mla_absorb_kernel<LH_Q6_K>), g, dim3(MA_THREADS), 0, st, wk, pl, q_nope, nope, (int)kvr, qa);
            break;
        case LH_Q8_0:
            hipLaunchKernelGGL((mla_absorb_kernel<LH_Q8_0>), g, dim3(MA_THREADS), 0, st, wk, pl, q_nope, nope, (int)kvr, qa);
            break;
        default:
            hipLaunchKernelGGL((mla_absorb_kernel<LH_Q4_0>), g, dim3(MA_THREADS), 0, st, wk, pl, q_nope, nope, (int)kvr, qa);
            break;
        }
    }
    note_launch();
    prof_end(ph, st);
    // 2. scores
    ph = prof_begin(LOOMHIP_KT_MLA_SCORES, st);
    hipLaunchKernelGGL(mla_scores_kernel, dim3((unsigned)((seq + MS_POS - 1) / MS_POS), (unsigned)((H + MS_HEADS - 1) / MS_HEADS)),
                       dim3(MS_THREADS), 0, st, qa, q_rope, c_kv, k_rope, (int)seq, (int)H, (int)kvr, (int)a->rope,
                       a->scale, S, (int)s_stride);
    note_launch();
    prof_end(ph, st);
    // 3. softmax
    ph = prof_begin(LOOMHIP_KT_MLA_SOFTMAX, st);
    hipLaunchKernelGGL((mla_softmax_kernel<1024>), dim3((unsigned)H), dim3(1024), s_stride * 4, st, S, (int)s_stride,
                       (int)seq);
    note_launch();
    prof_end(ph, st);
    // 4. weighted sum
    ph = prof_begin(LOOMHIP_KT_MLA_WSUM, st);
    {
        const int ntile = (int)((kvr + 63) / 64);
        hipLaunchKernelGGL(mla_wsum_kernel, dim3((unsigned)(ntile * ((H + 3) / 4))), dim3(256), 0, st, S,
                           (int)s_stride, c_kv, (int)seq, (int)H, (int)kvr, ntile, ol);
    }
    note_launch();
    prof_end(ph, st);
    // 5. W_v: quantize every head's o and run the grouped matvec, plane = head
    QAct q;
    q.q = (int8_t *)g_mla.act.ptr;
    q.d = (float *)((char *)g_mla.act.ptr + align16(H * kvr));
    q.s = (int32_t *)((char *)q.d + align16(H * kvr / 32 * 4));
    ph = prof_begin(LOOMHIP_KT_MLA_WV, st);
    launch_quant_act(t, ol, (int)kvr, (int)kvr, (int)H, q, st);
    DmmvParams p{};
    p.w = (const uint8_t *)a->wv;
    p.w2 = nullptr;
    p.plane_bytes = plane_bytes(t, a->vd, kvr);
    p.rows = (int)a->vd;
    p.cols = (int)kvr;
    p.xq = q.q;
    p.xd = q.d;
    p.xs = q.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = groups;
    p.n_groups_dev = nullptr;
    p.n_groups = (int)H;
    p.out = out;
    p.out_stride = (int)a->vd;
    p.rpw = dmmv_pick_rpw(t, (int)kvr, (int)a->vd, (int)H, 1, false);
    p.accumulate = 0;
    p.ident_n = 0;
    const bool launched = launch_dmmv(t, 1, false, p, st);
    prof_end(ph, st);
    if (!launched)
        return fail(LOOMHIP_DECLINED, "mla: W_v partials exceed LDS for %zu columns", kvr);
    return LOOMHIP_OK;
}

static int mla_split(int t, const void *src, size_t H, size_t nope, size_t vd, size_t kvr, void *wk, void *wv,
                     hipStream_t st) {
    const size_t rb = ggml_bytes(t, 1, kvr), stride = (nope + vd) * rb;
    launch_repack_strided(t, src, stride, wk, nope, kvr, H, st);
    launch_repack_strided(t, (const uint8_t *)src + nope * rb, stride, wv, vd, kvr, H, st);
    return LOOMHIP_OK;
}

// x[i] = x[i] + y[i] (tensor.zig:50-52)
__global__ void mla_add_kernel(float *__restrict__ x, const float *__restrict__ y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        x[i] = x[i] + y[i];
}

// out = out + W . x for one vector: the matvec (int8 activations, ggml.zig:
// 602) with the residual add as its epilogue (tensor.zig:50-52).
static int matvec_add(int t, const void *w, const float *x, int rows, int cols, float *out, hipStream_t st) {
    const size_t qbytes = align16(cols) + align16((size_t)cols / 32 * 4) + align16((size_t)cols / 16 * 4);
    if (int rc = reserve_on(g_mla.act2, qbytes, st))
        return rc;
    QAct q;
    q.q = (int8_t *)g_mla.act2.ptr;
    q.d = (float *)((char *)g_mla.act2.ptr + align16(cols));
    q.s = (int32_t *)((char *)q.d + align16((size_t)cols / 32 * 4));
    launch_quant_act(t, x, cols, cols, 1, q, st);
    int ng = 0;
    const DmmvGroup *g = dense_groups(1, 1, &ng);
    if (!g)
        return fail(LOOMHIP_ERR_HIP, "mla: dense group table");
    DmmvParams p{};
    p.w = (const uint8_t *)w;
    p.w2 = nullptr;
    p.plane_bytes = plane_bytes(t, rows, cols);
    p.rows = rows;
    p.cols = cols;
    p.xq = q.q;
    p.xd = q.d;
    p.xs = q.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = g;
    p.n_groups_dev = nullptr;
    p.n_groups = ng;
    p.out = out;
    p.out_stride = rows;
    p.rpw = dmmv_pick_rpw(t, cols, rows, ng, 1, false);
    p.accumulate = 1;
    p.ident_n = 0;
    if (!launch_dmmv(t, 1, false, p, st))
        return fail(LOOMHIP_DECLINED, "mla: attn_output partials exceed LDS for %d columns", cols);
    return LOOMHIP_OK;
}

// The whole layer after the attention head (the seam's mlaLayerTail,
// cpu.zig:63; the engine's own sequence, deepseek.zig:1044-1046 and
// 1325-1387): attention with W_v, x = x + attn_output . heads, normed =
// rmsnorm(x) * ffn_norm, acc = the routed experts in selection order plus
// the shared expert, x = x + acc.  Every check runs before the first launch.
static int mla_tail_impl(const loomhip_mla_attn *a, const float *c_kv, const float *k_rope, size_t seq,
                         const float *q_nope, const float *q_rope, int out_t, const void *attn_out,
                         const float *ffn_norm, float eps, const loomhip_moe_layer *moe, float *x, hipStream_t st) {
    if (int rc = mla_check(a, seq))
        return rc;
    if (!moe || !attn_out || !ffn_norm || !x)
        return fail(LOOMHIP_ERR_ARG, "mla_layer_tail: null pointer");
    const size_t hv = a->n_heads * a->vd, dim = moe->dim;
    if (out_t == LH_F32 || out_t == LH_F16 || !dmmv_supported(out_t, (int)hv))
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: attn_output type %d with %zu columns not served", out_t, hv);
    if (dim == 0 || dim % 32 || dim > 7936)
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: dim %zu not served", dim);
    if (int rc = moe_layer_check(moe, 1, true))
        return rc;
    if (int rc = reserve_on(g_mla.tail, align16(hv * 4) + 2 * align16(dim * 4), st))
        return rc;
    float *head = (float *)g_mla.tail.ptr;
    float *normed = (float *)((char *)g_mla.tail.ptr + align16(hv * 4));
    float *acc = (float *)((char *)normed + align16(dim * 4));
    int rc;
    if ((rc = mla_attn_impl(a, c_kv, k_rope, seq, q_nope, q_rope, head, nullptr, st)) ||
        (rc = matvec_add(out_t, attn_out, head, (int)dim, (int)hv, x, st)) ||
        (rc = rmsnorm_exact_dev(x, (int)dim, ffn_norm, eps, normed, 1, st)) ||
        (rc = loomhip_moe_layer_dev(moe, normed, 1, LOOMHIP_COMBINE_SELECTION, acc, nullptr, nullptr, st)))
        return rc;
    hipLaunchKernelGGL(mla_add_kernel, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, st, x, acc, (int)dim);
    note_launch();
    return LOOMHIP_OK;
}

// kv_b split per head into the device layout once per host tensor (keyed by
// its pointer, re-split when the tensor behind it changes).
static int kvb_cached(int t, const uint8_t *kv_b, size_t kvb_len, size_t n_heads, size_t nope, size_t vd, size_t kvr,
                      hipStream_t st, KvbSplit **out) {
    KvbSplit &ks = g_mla.kvb[kv_b];
    if (ks.t == t && ks.len == kvb_len && ks.H == n_heads && ks.nope == nope && ks.vd == vd && ks.kvr == kvr) {
        *out = &ks;
        return LOOMHIP_OK;
    }
    (void)hipStreamSynchronize(st);
    if (ks.wk)
        (void)hipFree(ks.wk);
    if (ks.wv)
        (void)hipFree(ks.wv);
    ks = KvbSplit{};
    void *wk = nullptr, *wv = nullptr;
    hipError_t e = hipMalloc(&wk, plane_bytes(t, nope, kvr) * n_heads);
    if (e == hipSuccess)
        e = hipMalloc(&wv, plane_bytes(t, vd, kvr) * n_heads);
    int rc = e == hipSuccess ? reserve_on(g_mla.kvb_stage, kvb_len, st) : hip_fail(e, "hipMalloc kv_b split");
    if (rc == LOOMHIP_OK) {
        e = hipMemcpy(g_mla.kvb_stage.ptr, kv_b, kvb_len, hipMemcpyHostToDevice);
        rc = e == hipSuccess ? mla_split(t, g_mla.kvb_stage.ptr, n_heads, nope, vd, kvr, wk, wv, st)
                             : hip_fail(e, "kv_b upload");
    }
    if (rc == LOOMHIP_OK && (e = hipStreamSynchronize(st)) != hipSuccess)
        rc = hip_fail(e, "kv_b split");
    if (rc != LOOMHIP_OK) {
        if (wk)
            (void)hipFree(wk);
        if (wv)
            (void)hipFree(wv);
        g_mla.kvb.erase(kv_b);
        return rc;
    }
    ks = KvbSplit{t, kvb_len, n_heads, nope, vd, kvr, wk, wv};
    *out = &ks;
    return LOOMHIP_OK;
}

static int ensure_cache() {
    if (!g_mla.want) // as the Vulkan arm: a declined mlaInit leaves no usable cache
        return fail(LOOMHIP_DECLINED, "mla: no cache shape (mlaInit)");
    if (g_mla.cache)
        return LOOMHIP_OK;
    const size_t n = g_mla.layers * g_mla.ctx * (g_mla.kvr + g_mla.rope);
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, n * 4);
    if (e != hipSuccess)
        return hip_fail(e, "hipMalloc mla cache");
    if ((e = hipMemset(d, 0, n * 4)) != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "hipMemset mla cache");
    }
    g_mla.cache = (float *)d;
    return LOOMHIP_OK;
}

static float *cache_c(size_t li, size_t pos) { return g_mla.cache + (li * g_mla.ctx + pos) * g_mla.kvr; }
static float *cache_r(size_t li, size_t pos) {
    return g_mla.cache + g_mla.layers * g_mla.ctx * g_mla.kvr + (li * g_mla.ctx + pos) * g_mla.rope;
}

void mla_release() {
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (g_mla.cache)
        (void)hipFree(g_mla.cache);
    g_mla.cache = nullptr;
    g_mla.want = false;
    g_mla.wk_layers = 0;
    for (auto &kv : g_mla.kvb) {
        (void)hipFree(kv.second.wk);
        (void)hipFree(kv.second.wv);
    }
    g_mla.kvb.clear();
    for (auto &kv : g_mla.vgroups)
        (void)hipFree(kv.second);
    g_mla.vgroups.clear();
    g_mla.qa.release();
    g_mla.S.release();
    g_mla.olat.release();
    g_mla.act.release();
    g_mla.kvb_stage.release();
    g_mla.tail.release();
    g_mla.act2.release();
    g_mla.frame.release();
    for (auto &kv : g_mla.yarn)
        (void)hipFree(kv.second);
    g_mla.yarn.clear();
}

// ---- the whole MLA token (mlaTokenFrame) ------------------------------------------

// deepseek.zig:581-629 ropeApply's angles for vectors of `rope` values, as
// (cos, sin) per (position, pair) [ctx][rope / 2][2]: the YaRN ramp between
// the interpolated (theta / factor) and extrapolated angle over the
// corrected dimension range (beta_fast 32, beta_slow 1) when factor > 1,
// else the plain NORM angle; f32 throughout with the C library's logf,
// powf, cosf and sinf, in the reference's expressions.  Kept per shape.
static const float *yarn_table(size_t ctx, size_t rope, float base, float factor, float orig) {
    char key[128];
    snprintf(key, sizeof key, "%zu/%zu/%a/%a/%a", ctx, rope, base, factor, orig);
    auto it = g_mla.yarn.find(key);
    if (it != g_mla.yarn.end())
        return it->second;
    const size_t half = rope / 2;
    const float d = (float)rope;
    const bool yarn = factor > 1.0f;
    float low = 0.0f, high = 0.0f;
    if (yarn) {
        const float two_pi = (float)(2.0 * 3.14159265358979323846); // comptime 2*pi as f32
        auto corr = [&](float beta) { return d * logf(orig / (beta * two_pi)) / (2.0f * logf(base)); };
        low = fmaxf(0.0f, floorf(corr(32.0f)));
        high = fminf(d - 1.0f, ceilf(corr(1.0f)));
    }
    std::vector<float> h(ctx * half * 2);
    for (size_t p = 0; p < ctx; p++)
        for (size_t i = 0; i < half; i++) {
            const float exponent = (float)(2 * i) / d;
            const float freq = powf(base, -exponent);
            const float theta_extrap = (float)p * freq;
            float theta = theta_extrap;
            if (yarn) {
                const float theta_interp = theta_extrap / factor;
                const float y = ((float)i - low) / fmaxf(0.001f, high - low);
                const float ramp_mix = 1.0f - fminf(fmaxf(y, 0.0f), 1.0f); // 1 = extrapolate
                theta = theta_interp * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
            }
            h[(p * half + i) * 2] = cosf(theta);
            h[(p * half + i) * 2 + 1] = sinf(theta);
        }
    float *dev = nullptr;
    if (hipMalloc(&dev, h.size() * 4) != hipSuccess)
        return nullptr;
    if (hipMemcpy(dev, h.data(), h.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(dev);
        return nullptr;
    }
    g_mla.yarn[key] = dev;
    return dev;
}

// Work group h < H: head h's nope slice of q copied out and its rope slice
// rotated at this position; work group H: the new k_rope row (kv_a's tail)
// rotated into the cache.  NORM pairs: (a, b) -> (a c - b s, a s + b c),
// each product rounded before its add (deepseek.zig:606-611).
__global__ __launch_bounds__(64) void mla_rope_kernel(const float *__restrict__ q, int H, int nope, int rope,
                                                      const float *__restrict__ kr_src, const float *__restrict__ cs,
                                                      float *__restrict__ q_nope, float *__restrict__ q_rope,
                                                      float *__restrict__ kr_row) {
    const int h = blockIdx.x, kd = nope + rope;
    const float *src = h < H ? q + (size_t)h * kd + nope : kr_src;
    float *dst = h < H ? q_rope + (size_t)h * rope : kr_row;
    if (h < H)
        for (int i = threadIdx.x; i < nope; i += 64)
            q_nope[(size_t)h * nope + i] = q[(size_t)h * kd + i];
    for (int i = threadIdx.x; 2 * i + 1 < rope; i += 64) {
        const float c = cs[2 * i], sn = cs[2 * i + 1];
        const float a = src[2 * i], b = src[2 * i + 1];
        dst[2 * i] = a * c - b * sn;
        dst[2 * i + 1] = a * sn + b * c;
    }
}

} // namespace lh

using namespace lh;

extern "C" {

int loomhip_mla_init(size_t layers, size_t ctx_len, size_t kvr, size_t rope) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (layers == 0 || ctx_len == 0 || kvr == 0 || rope == 0)
        return fail(LOOMHIP_ERR_ARG, "mla_init: empty shape");
    if (ctx_len > (size_t)MLA_MAX_CTX || kvr > (size_t)MLA_MAX_KVR || rope > (size_t)MLA_MAX_ROPE) {
        g_mla.want = false;
        return fail(LOOMHIP_DECLINED, "mla_init: context %zu (max %d) / kvr %zu / rope %zu not served", ctx_len,
                    MLA_MAX_CTX, kvr, rope);
    }
    if (g_mla.cache && (g_mla.layers != layers || g_mla.ctx != ctx_len || g_mla.kvr != kvr || g_mla.rope != rope)) {
        (void)hipDeviceSynchronize();
        (void)hipFree(g_mla.cache);
        g_mla.cache = nullptr;
    }
    g_mla.layers = layers;
    g_mla.ctx = ctx_len;
    g_mla.kvr = kvr;
    g_mla.rope = rope;
    g_mla.want = true;
    return LOOMHIP_OK;
}

int loomhip_has_mla_cache(void) {
    if (require_ready())
        return 0;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    return ensure_cache() == LOOMHIP_OK;
}

int loomhip_mla_append(size_t li, size_t pos, const float *c_kv, size_t c_len, const float *k_rope, size_t r_len) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (int rc = ensure_cache())
        return rc;
    if (li >= g_mla.layers || pos >= g_mla.ctx || c_len != g_mla.kvr || r_len != g_mla.rope || !c_kv || !k_rope)
        return fail(LOOMHIP_DECLINED, "mla_append: layer %zu pos %zu lengths %zu/%zu outside the cache", li, pos,
                    c_len, r_len);
    hipError_t e = hipMemcpy(cache_c(li, pos), c_kv, c_len * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(cache_r(li, pos), k_rope, r_len * 4, hipMemcpyHostToDevice);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_append");
}

int loomhip_mla_read_cache(size_t li, size_t pos, float *c_kv, size_t c_len, float *k_rope, size_t r_len) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (int rc = ensure_cache())
        return rc;
    if (li >= g_mla.layers || pos >= g_mla.ctx || c_len != g_mla.kvr || r_len != g_mla.rope || !c_kv || !k_rope)
        return fail(LOOMHIP_DECLINED, "mla_read_cache: layer %zu pos %zu lengths %zu/%zu outside the cache", li,
                    pos, c_len, r_len);
    hipError_t e = hipStreamSynchronize(g_ctx.compute);
    if (e == hipSuccess)
        e = hipMemcpy(c_kv, cache_c(li, pos), c_len * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess)
        e = hipMemcpy(k_rope, cache_r(li, pos), r_len * 4, hipMemcpyDeviceToHost);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_read_cache");
}

int loomhip_mla_set_wk(size_t li, const float *wk_f32, size_t n) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (li != g_mla.wk_layers || !wk_f32 || n == 0)
        return fail(LOOMHIP_DECLINED, "mla_set_wk: layer %zu out of order (expected %zu)", li, g_mla.wk_layers);
    g_mla.wk_layers++;
    return LOOMHIP_OK;
}

int loomhip_mla_split_kvb_dev(int t, const void *kv_b, size_t n_heads, size_t nope, size_t vd, size_t kvr, void *wk,
                              void *wv, void *stream) {
    if (int rc = require_ready())
        return rc;
    if (!kv_b || !wk || !wv || n_heads == 0 || nope == 0 || vd == 0 || kvr % 32)
        return fail(LOOMHIP_ERR_ARG, "mla_split_kvb: bad arguments");
    if (t == LH_F32 || t == LH_F16 || !dmmv_supported(t, (int)kvr))
        return fail(LOOMHIP_DECLINED, "mla_split_kvb: type %d with %zu columns not served", t, kvr);
    return mla_split(t, kv_b, n_heads, nope, vd, kvr, wk, wv, stream_of(stream));
}

int loomhip_mla_attn_dev(const loomhip_mla_attn *a, const float *c_kv, const float *k_rope, size_t seq,
                         const float *q_nope, const float *q_rope, float *out, float *o_lat, void *stream) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (!c_kv || !k_rope || !q_nope || !q_rope || !out)
        return fail(LOOMHIP_ERR_ARG, "mla_attn_dev: null pointer");
    return mla_attn_impl(a, c_kv, k_rope, seq, q_nope, q_rope, out, o_lat, stream_of(stream));
}

int loomhip_mla_attn_heads(size_t li, size_t pos, const float *q_nope, size_t qn_len, const float *q_rope,
                           size_t qr_len, int kvb_type, const uint8_t *kv_b, size_t kvb_len, float *out,
                           size_t out_len, size_t n_heads, size_t nope, size_t vd, float scale) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (int rc = ensure_cache())
        return rc;
    const size_t kvr = g_mla.kvr, rope = g_mla.rope, seq = pos + 1;
    if (li >= g_mla.layers || seq > g_mla.ctx)
        return fail(LOOMHIP_DECLINED, "mla_attn_heads: layer %zu / position %zu outside the cache", li, pos);
    if (!q_nope || !q_rope || !kv_b || !out || qn_len != n_heads * nope || qr_len != n_heads * rope ||
        out_len != n_heads * vd)
        return fail(LOOMHIP_DECLINED, "mla_attn_heads: slice lengths do not match %zu heads", n_heads);
    if (kvb_type == LH_F32 || kvb_type == LH_F16 || !dmmv_supported(kvb_type, (int)kvr) ||
        kvb_len != n_heads * (nope + vd) * ggml_bytes(kvb_type, 1, kvr))
        return fail(LOOMHIP_DECLINED, "mla_attn_heads: kv_b type %d / %zu bytes not served", kvb_type, kvb_len);
    hipStream_t st = g_ctx.compute;
    KvbSplit *ks = nullptr;
    if (int rc = kvb_cached(kvb_type, kv_b, kvb_len, n_heads, nope, vd, kvr, st, &ks))
        return rc;
    const size_t qn = n_heads * nope, qr = n_heads * rope;
    int rc = g_ctx.xstage.reserve((qn + qr) * 4);
    if (rc || (rc = g_ctx.ostage.reserve(out_len * 4)))
        return rc;
    float *dq = (float *)g_ctx.xstage.ptr;
    hipError_t e = hipMemcpyAsync(dq, q_nope, qn * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dq + qn, q_rope, qr * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "mla_attn_heads upload");
    const loomhip_mla_attn a{kvb_type, ks->wk, ks->wv, n_heads, nope, vd, kvr, rope, scale};
    rc = mla_attn_impl(&a, cache_c(li, 0), cache_r(li, 0), seq, dq, dq + qn, (float *)g_ctx.ostage.ptr, nullptr, st);
    if (rc)
        return rc;
    e = hipMemcpyAsync(out, g_ctx.ostage.ptr, out_len * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_attn_heads");
}

int loomhip_mla_layer_tail_dev(const loomhip_mla_attn *a, const float *c_kv, const float *k_rope, size_t seq,
                               const float *q_nope, const float *q_rope, int attn_out_type, const void *attn_out,
                               const float *ffn_norm, float eps, const loomhip_moe_layer *moe, float *x,
                               void *stream) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (!c_kv || !k_rope || !q_nope || !q_rope)
        return fail(LOOMHIP_ERR_ARG, "mla_layer_tail_dev: null pointer");
    return mla_tail_impl(a, c_kv, k_rope, seq, q_nope, q_rope, attn_out_type, attn_out, ffn_norm, eps, moe, x,
                         stream_of(stream));
}

int loomhip_mla_token_frame(const loomhip_mla_layer_desc *descs, size_t n_layers, const loomhip_mla_frame_cfg *fc,
                            float *x, size_t pos, const float *out_norm, loomhip_weight_ref lm_head, float *logits,
                            size_t vocab) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (!descs || !fc || !x || !out_norm || !logits || n_layers == 0 || vocab == 0)
        return fail(LOOMHIP_ERR_ARG, "mla_token_frame: null argument");
    if (int rc = ensure_cache())
        return rc;
    const size_t dim = fc->dim, H = fc->n_heads, nope = fc->nope, rope = fc->rope, kvr = fc->kvr, vd = fc->v_head_dim;
    const size_t kd = nope + rope, hv = H * vd;
    if (n_layers > g_mla.layers || pos >= g_mla.ctx || kvr != g_mla.kvr || rope != g_mla.rope)
        return fail(LOOMHIP_DECLINED, "mla_token_frame: %zu layers / position %zu / kvr %zu / rope %zu outside the cache",
                    n_layers, pos, kvr, rope);
    if (dim == 0 || dim % 32 || dim > 7936 || kvr % 32 || kvr > 7936 || rope % 2 || H == 0)
        return fail(LOOMHIP_DECLINED, "mla_token_frame: dim %zu / kvr %zu / rope %zu not served", dim, kvr, rope);
    auto ref_ok = [](const loomhip_weight_ref &r, size_t rows, size_t cols, size_t planes = 1) {
        return r.data && r.len == ggml_bytes(r.type, rows, cols) * planes;
    };
    auto quant_ok = [](int t, size_t cols) { return t != LH_F32 && t != LH_F16 && dmmv_supported(t, (int)cols); };
    if (!ref_ok(lm_head, vocab, dim) || !quant_ok(lm_head.type, dim))
        return fail(LOOMHIP_DECLINED, "mla_token_frame: lm_head type %d / %zu bytes not served", lm_head.type,
                    lm_head.len);
    // every layer checked (host pointers stand in for the device copies)
    // before anything is uploaded or launched
    std::vector<loomhip_moe_layer> moes(n_layers);
    for (size_t li = 0; li < n_layers; li++) {
        const loomhip_mla_layer_desc &d = descs[li];
        const int kt = d.kv_b.type;
        const loomhip_mla_attn probe{kt, d.kv_b.data, d.kv_b.data, H, nope, vd, kvr, rope, fc->scale};
        if (!d.attn_norm || !d.kv_a_norm || !d.ffn_norm || !ref_ok(d.wq, H * kd, dim) || !quant_ok(d.wq.type, dim) ||
            !ref_ok(d.kv_a, kvr + rope, dim) || !quant_ok(d.kv_a.type, dim) || !ref_ok(d.attn_out, dim, hv) ||
            !quant_ok(d.attn_out.type, hv) || !ref_ok(d.kv_b, H * (nope + vd), kvr))
            return fail(LOOMHIP_DECLINED, "mla_token_frame: layer %zu attention tensors do not match their shapes",
                        li);
        if (int rc = mla_check(&probe, pos + 1))
            return rc;
        if (d.is_moe) {
            const size_t E = fc->n_expert;
            const bool sh = d.shexp_gate.data != nullptr;
            if (d.router.type != LH_F32 || !ref_ok(d.router, E, dim) || !ref_ok(d.gate, d.ffn, dim, E) ||
                !ref_ok(d.up, d.ffn, dim, E) || !ref_ok(d.down, dim, d.ffn, E) ||
                (sh && (!ref_ok(d.shexp_gate, d.shexp_ffn, dim) || !ref_ok(d.shexp_up, d.shexp_ffn, dim) ||
                        !ref_ok(d.shexp_down, dim, d.shexp_ffn))))
                return fail(LOOMHIP_DECLINED, "mla_token_frame: layer %zu MoE tensors do not match their shapes", li);
            loomhip_moe_layer &m = moes[li];
            m.dim = dim;
            m.ffn = d.ffn;
            m.n_expert = E;
            m.n_used = fc->n_used;
            m.gating = fc->gating;
            m.weights_norm = fc->weights_norm;
            m.weights_scale = fc->weights_scale;
            m.router = (const float *)d.router.data;
            m.gate_t = d.gate.type;
            m.up_t = d.up.type;
            m.down_t = d.down.type;
            m.gate = d.gate.data;
            m.up = d.up.data;
            m.down = d.down.data;
            if (sh) {
                m.shexp_gate_t = d.shexp_gate.type;
                m.shexp_up_t = d.shexp_up.type;
                m.shexp_down_t = d.shexp_down.type;
                m.shexp_gate = d.shexp_gate.data;
                m.shexp_up = d.shexp_up.data;
                m.shexp_down = d.shexp_down.data;
                m.shexp_ffn = d.shexp_ffn;
            }
            if (int rc = moe_layer_check(&m, 1, true))
                return rc;
        } else {
            if (!ref_ok(d.dgate, d.dffn, dim) || !ref_ok(d.dup, d.dffn, dim) || !ref_ok(d.ddown, dim, d.dffn))
                return fail(LOOMHIP_DECLINED, "mla_token_frame: layer %zu FFN tensors do not match their shapes", li);
            const DenseFfn f{d.dgate.type, d.dup.type, d.ddown.type, d.dgate.data, d.dup.data, d.ddown.data, d.dffn};
            if (int rc = dense_ffn_check(f, dim))
                return rc;
        }
    }
    hipStream_t st = g_ctx.compute;
    const float *cs = yarn_table(g_mla.ctx, rope, fc->rope_base, fc->yarn_factor, fc->yarn_orig_ctx);
    if (!cs)
        return fail(LOOMHIP_ERR_HIP, "mla_token_frame: rope table");
    cs += pos * rope; // rope / 2 (cos, sin) pairs per position
    // the device copies (uploaded once per host tensor)
    struct Dev {
        const void *wq, *kv_a, *attn_out, *gate, *up, *down, *sg, *su, *sd, *dg, *du, *dd;
        const float *attn_norm, *kv_a_norm, *ffn_norm, *router;
        KvbSplit *kvb;
    };
    std::vector<Dev> dv(n_layers);
    int rc;
    auto up_ref = [&](const loomhip_weight_ref &r, size_t rows, size_t cols, size_t planes, const void **out) {
        void *p = nullptr;
        const int c = upload_weights(r.type, r.data, rows, cols, planes, &p);
        *out = p;
        return c;
    };
    auto up_f32 = [&](const float *h, size_t n, const float **out) {
        void *p = nullptr;
        const int c = upload_weights(LH_F32, h, 1, n, 1, &p);
        *out = (const float *)p;
        return c;
    };
    for (size_t li = 0; li < n_layers; li++) {
        const loomhip_mla_layer_desc &d = descs[li];
        Dev &v = dv[li];
        if ((rc = up_f32(d.attn_norm, dim, &v.attn_norm)) || (rc = up_f32(d.kv_a_norm, kvr, &v.kv_a_norm)) ||
            (rc = up_f32(d.ffn_norm, dim, &v.ffn_norm)) || (rc = up_ref(d.wq, H * kd, dim, 1, &v.wq)) ||
            (rc = up_ref(d.kv_a, kvr + rope, dim, 1, &v.kv_a)) || (rc = up_ref(d.attn_out, dim, hv, 1, &v.attn_out)) ||
            (rc = kvb_cached(d.kv_b.type, (const uint8_t *)d.kv_b.data, d.kv_b.len, H, nope, vd, kvr, st, &v.kvb)))
            return rc;
        if (d.is_moe) {
            const size_t E = fc->n_expert;
            loomhip_moe_layer &m = moes[li];
            if ((rc = up_f32(m.router, E * dim, &m.router)) || (rc = up_ref(d.gate, d.ffn, dim, E, &m.gate)) ||
                (rc = up_ref(d.up, d.ffn, dim, E, &m.up)) || (rc = up_ref(d.down, dim, d.ffn, E, &m.down)))
                return rc;
            if (m.shexp_gate &&
                ((rc = up_ref(d.shexp_gate, d.shexp_ffn, dim, 1, &m.shexp_gate)) ||
                 (rc = up_ref(d.shexp_up, d.shexp_ffn, dim, 1, &m.shexp_up)) ||
                 (rc = up_ref(d.shexp_down, dim, d.shexp_ffn, 1, &m.shexp_down))))
                return rc;
        } else if ((rc = up_ref(d.dgate, d.dffn, dim, 1, &v.dg)) || (rc = up_ref(d.dup, d.dffn, dim, 1, &v.du)) ||
                   (rc = up_ref(d.ddown, dim, d.dffn, 1, &v.dd))) {
            return rc;
        }
    }
    const float *d_out_norm;
    const void *d_lm;
    if ((rc = up_f32(out_norm, dim, &d_out_norm)) || (rc = up_ref(lm_head, vocab, dim, 1, &d_lm)))
        return rc;
    // workspace: x | normed | q | kv_a | q_nope | q_rope | heads | logits
    size_t off = 0;
    auto take = [&](size_t n) {
        const size_t o = off;
        off += align16(n * 4);
        return o;
    };
    const size_t o_x = take(dim), o_n = take(dim), o_q = take(H * kd), o_kv = take(kvr + rope), o_qn = take(H * nope),
                 o_qr = take(H * rope), o_h = take(hv), o_l = take(vocab);
    if ((rc = reserve_on(g_mla.frame, off, st)))
        return rc;
    char *base = (char *)g_mla.frame.ptr;
    float *dx = (float *)(base + o_x), *normed = (float *)(base + o_n), *q = (float *)(base + o_q);
    float *kv = (float *)(base + o_kv), *qn = (float *)(base + o_qn), *qr = (float *)(base + o_qr);
    float *heads = (float *)(base + o_h), *dlog = (float *)(base + o_l);
    hipError_t e = hipMemcpyAsync(dx, x, dim * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "mla_token_frame upload");
    for (size_t li = 0; li < n_layers; li++) {
        const loomhip_mla_layer_desc &d = descs[li];
        const Dev &v = dv[li];
        // the attention head (deepseek.zig:860-886)
        if ((rc = rmsnorm_exact_dev(dx, (int)dim, v.attn_norm, fc->eps, normed, 1, st)) ||
            (rc = matvec_dev_impl(d.wq.type, q, v.wq, normed, 1, H * kd, dim, st)) ||
            (rc = matvec_dev_impl(d.kv_a.type, kv, v.kv_a, normed, 1, kvr + rope, dim, st)) ||
            (rc = rmsnorm_exact_dev(kv, (int)kvr, v.kv_a_norm, fc->eps, cache_c(li, pos), 1, st)))
            return rc;
        hipLaunchKernelGGL(mla_rope_kernel, dim3((unsigned)(H + 1)), dim3(64), 0, st, q, (int)H, (int)nope, (int)rope,
                           kv + kvr, cs, qn, qr, cache_r(li, pos));
        note_launch();
        const loomhip_mla_attn a{d.kv_b.type, v.kvb->wk, v.kvb->wv, H, nope, vd, kvr, rope, fc->scale};
        if (d.is_moe) { // attention through the FFN residual (deepseek.zig:1044-1046, 1325-1387)
            if ((rc = mla_tail_impl(&a, cache_c(li, 0), cache_r(li, 0), pos + 1, qn, qr, d.attn_out.type, v.attn_out,
                                    v.ffn_norm, fc->eps, &moes[li], dx, st)))
                return rc;
        } else { // dense: attention, x += wo . heads, x += denseFFN(rmsnorm(x))
            const DenseFfn f{d.dgate.type, d.dup.type, d.ddown.type, v.dg, v.du, v.dd, d.dffn};
            if ((rc = mla_attn_impl(&a, cache_c(li, 0), cache_r(li, 0), pos + 1, qn, qr, heads, nullptr, st)) ||
                (rc = matvec_add(d.attn_out.type, v.attn_out, heads, (int)dim, (int)hv, dx, st)) ||
                (rc = rmsnorm_exact_dev(dx, (int)dim, v.ffn_norm, fc->eps, normed, 1, st)) ||
                (rc = dense_ffn_add(f, normed, 1, dim, dx, st, true)))
                return rc;
        }
    }
    if ((rc = rmsnorm_exact_dev(dx, (int)dim, d_out_norm, fc->eps, normed, 1, st)) ||
        (rc = matvec_dev_impl(lm_head.type, dlog, d_lm, normed, 1, vocab, dim, st)))
        return rc;
    e = hipMemcpyAsync(logits, dlog, vocab * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(x, dx, dim * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_token_frame");
}

int loomhip_mla_layer_cached_dev(const loomhip_mla_attn *a, const float *const *c_kv, const float *const *k_rope,
                                 size_t seq, size_t n, const float *q_nope, const float *q_rope, int attn_out_type,
                                 const void *attn_out, const float *ffn_norm, float eps,
                                 const loomhip_moe_layer_ec *moe, loomhip_ec *ec, float *x, uint32_t *ids_out,
                                 void *stream) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (!a || !c_kv || !k_rope || !q_nope || !q_rope || !attn_out || !ffn_norm || !moe || !ec || !x || n == 0 ||
        n > 256)
        return fail(LOOMHIP_ERR_ARG, "mla_layer_cached_dev: null pointer or %zu sequences (1..256)", n);
    for (size_t i = 0; i < n; i++)
        if (!c_kv[i] || !k_rope[i])
            return fail(LOOMHIP_ERR_ARG, "mla_layer_cached_dev: sequence %zu has no cache", i);
    if (int rc = mla_check(a, seq))
        return rc;
    const size_t hv = a->n_heads * a->vd, dim = moe->dim;
    if (attn_out_type == LH_F32 || attn_out_type == LH_F16 || !dmmv_supported(attn_out_type, (int)hv))
        return fail(LOOMHIP_DECLINED, "mla_layer_cached_dev: attn_output type %d with %zu columns not served",
                    attn_out_type, hv);
    if (dim == 0 || dim % 32 || dim > 7936)
        return fail(LOOMHIP_DECLINED, "mla_layer_cached_dev: dim %zu not served", dim);
    hipStream_t st = stream_of(stream);
    // heads [n][hv] | proj [n][dim] (then acc) | normed [n][dim]
    const size_t o_proj = align16(n * hv * 4), o_norm = o_proj + align16(n * dim * 4);
    if (int rc = reserve_on(g_mla.tail, o_norm + align16(n * dim * 4), st))
        return rc;
    float *heads = (float *)g_mla.tail.ptr;
    float *proj = (float *)((char *)g_mla.tail.ptr + o_proj);
    float *normed = (float *)((char *)g_mla.tail.ptr + o_norm);
    const size_t qn = a->n_heads * a->nope, qr = a->n_heads * a->rope;
    int rc;
    for (size_t i = 0; i < n; i++) // each sequence's attention over its own cache (deepseek.zig:977-1047)
        if ((rc = mla_attn_impl(a, c_kv[i], k_rope[i], seq, q_nope + i * qn, q_rope + i * qr, heads + i * hv,
                                nullptr, st)))
            return rc;
    const int nd = (int)(n * dim);
    // x += attn_output . heads (deepseek.zig:1044-1046): n matvecs in one
    // launch (bit-identical to one per sequence), then the residual add
    if ((rc = matvec_dev_impl(attn_out_type, proj, attn_out, heads, n, dim, hv, st)))
        return rc;
    hipLaunchKernelGGL(mla_add_kernel, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, st, x, proj, nd);
    note_launch();
    if ((rc = rmsnorm_exact_dev(x, (int)dim, ffn_norm, eps, normed, n, st)))
        return rc;
    // the routed experts through the cache plus the resident shared expert,
    // from +0 into proj's space; then x += acc (deepseek.zig:1325-1440)
    if ((rc = loomhip_moe_layer_cached(moe, ec, normed, n, proj, ids_out, nullptr, stream)))
        return rc;
    hipLaunchKernelGGL(mla_add_kernel, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, st, x, proj, nd);
    note_launch();
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_layer_cached_dev");
}

int loomhip_mla_layer_tail(size_t li, size_t pos, float *x, size_t dim, const float *q_nope, size_t qn_len,
                           const float *q_rope, size_t qr_len, int kvb_type, const uint8_t *kv_b, size_t kvb_len,
                           int attn_out_type, const uint8_t *attn_out, const float *ffn_norm, float eps,
                           int router_type, const uint8_t *router, const float *router_bias, int gate_type,
                           const uint8_t *gate, int up_type, const uint8_t *up, int down_type, const uint8_t *down,
                           int shexp_gate_type, const uint8_t *shexp_gate, int shexp_up_type,
                           const uint8_t *shexp_up, int shexp_down_type, const uint8_t *shexp_down, size_t ffn,
                           size_t shexp_ffn, size_t n_expert, size_t n_used, int gating, int weights_norm,
                           float weights_scale, size_t n_heads, size_t nope, size_t vd, float scale) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mla.mu);
    if (int rc = ensure_cache())
        return rc;
    const size_t kvr = g_mla.kvr, rope = g_mla.rope, seq = pos + 1, hv = n_heads * vd;
    if (li >= g_mla.layers || seq > g_mla.ctx)
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: layer %zu / position %zu outside the cache", li, pos);
    if (!x || !q_nope || !q_rope || !kv_b || !attn_out || !ffn_norm || !router || !gate || !up || !down ||
        qn_len != n_heads * nope || qr_len != n_heads * rope)
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: missing tensor or slice lengths that do not match");
    if (router_type != LH_F32)
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: router type %d (f32 served)", router_type);
    if (shexp_gate && (!shexp_up || !shexp_down || shexp_ffn == 0))
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: incomplete shared expert");
    if (kvb_type == LH_F32 || kvb_type == LH_F16 || !dmmv_supported(kvb_type, (int)kvr) ||
        kvb_len != n_heads * (nope + vd) * ggml_bytes(kvb_type, 1, kvr))
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: kv_b type %d / %zu bytes not served", kvb_type, kvb_len);
    // the MoE half's shapes and types, checked before anything is uploaded
    loomhip_moe_layer m{};
    m.dim = dim;
    m.ffn = ffn;
    m.n_expert = n_expert;
    m.n_used = n_used;
    m.gating = gating;
    m.weights_norm = weights_norm;
    m.weights_scale = weights_scale;
    m.gate_t = gate_type;
    m.up_t = up_type;
    m.down_t = down_type;
    m.router = (const float *)router;
    m.gate = gate;
    m.up = up;
    m.down = down;
    if (shexp_gate) {
        m.shexp_gate_t = shexp_gate_type;
        m.shexp_up_t = shexp_up_type;
        m.shexp_down_t = shexp_down_type;
        m.shexp_gate = shexp_gate;
        m.shexp_up = shexp_up;
        m.shexp_down = shexp_down;
        m.shexp_ffn = shexp_ffn;
    }
    if (int rc = moe_layer_check(&m, 1, true))
        return rc;
    if (attn_out_type == LH_F32 || attn_out_type == LH_F16 || !dmmv_supported(attn_out_type, (int)hv))
        return fail(LOOMHIP_DECLINED, "mla_layer_tail: attn_output type %d with %zu columns not served",
                    attn_out_type, hv);
    hipStream_t st = g_ctx.compute;
    KvbSplit *ks = nullptr;
    void *d_out, *d_norm, *d_router, *d_bias = nullptr, *d_gate, *d_up, *d_down;
    int rc;
    if ((rc = kvb_cached(kvb_type, kv_b, kvb_len, n_heads, nope, vd, kvr, st, &ks)) ||
        (rc = upload_weights(attn_out_type, attn_out, dim, hv, 1, &d_out)) ||
        (rc = upload_weights(LH_F32, ffn_norm, 1, dim, 1, &d_norm)) ||
        (rc = upload_weights(LH_F32, router, n_expert, dim, 1, &d_router)) ||
        (router_bias && (rc = upload_weights(LH_F32, router_bias, 1, n_expert, 1, &d_bias))) ||
        (rc = upload_weights(gate_type, gate, ffn, dim, n_expert, &d_gate)) ||
        (rc = upload_weights(up_type, up, ffn, dim, n_expert, &d_up)) ||
        (rc = upload_weights(down_type, down, dim, ffn, n_expert, &d_down)))
        return rc;
    m.router = (const float *)d_router;
    m.sel_bias = (const float *)d_bias;
    m.gate = d_gate;
    m.up = d_up;
    m.down = d_down;
    if (shexp_gate) {
        void *sg, *su, *sd;
        if ((rc = upload_weights(shexp_gate_type, shexp_gate, shexp_ffn, dim, 1, &sg)) ||
            (rc = upload_weights(shexp_up_type, shexp_up, shexp_ffn, dim, 1, &su)) ||
            (rc = upload_weights(shexp_down_type, shexp_down, dim, shexp_ffn, 1, &sd)))
            return rc;
        m.shexp_gate = sg;
        m.shexp_up = su;
        m.shexp_down = sd;
    }
    const size_t qn = n_heads * nope, qr = n_heads * rope;
    if ((rc = g_ctx.xstage.reserve((qn + qr + dim) * 4)))
        return rc;
    float *dq = (float *)g_ctx.xstage.ptr, *dx = dq + qn + qr;
    hipError_t e = hipMemcpyAsync(dq, q_nope, qn * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dq + qn, q_rope, qr * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dx, x, dim * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "mla_layer_tail upload");
    const loomhip_mla_attn a{kvb_type, ks->wk, ks->wv, n_heads, nope, vd, kvr, rope, scale};
    if ((rc = mla_tail_impl(&a, cache_c(li, 0), cache_r(li, 0), seq, dq, dq + qn, attn_out_type, d_out,
                            (const float *)d_norm, eps, &m, dx, st)))
        return rc;
    e = hipMemcpyAsync(x, dx, dim * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_layer_tail");
}

} // extern "C"
