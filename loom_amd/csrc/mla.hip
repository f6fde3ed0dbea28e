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

namespace lh {

constexpr int MLA_MAX_CTX = EXACT_MAX_CTX; // the softmax row's LDS
constexpr int MLA_MAX_KVR = 4096;
constexpr int MLA_MAX_ROPE = 512;

// ---- absorb -----------------------------------------------------------------
// qa[h][c] = chain over r of q_nope[h][r] * W_k[h][r][c] (product rounded,
// then added), from +0; W_k plane h holds nope rows of kvr values.
__global__ __launch_bounds__(64) void mla_absorb_kernel(int t, const uint8_t *__restrict__ wk, size_t plane,
                                                        const float *__restrict__ q_nope, int nope, int kvr,
                                                        int nb, int be_log2, float *__restrict__ qa) {
    const int h = blockIdx.y, c = blockIdx.x * 64 + threadIdx.x;
    if (c >= kvr)
        return;
    const uint8_t *w = wk + (size_t)h * plane;
    const float *q = q_nope + (size_t)h * nope;
    const size_t U = (size_t)nope * nb;
    const int cb = c >> be_log2, e = c & ((1 << be_log2) - 1);
    float acc = 0.0f;
    for (int r = 0; r < nope; r++) {
        const float p = q[r] * dequant_unit(t, w, U, (size_t)r * nb + cb, e);
        acc = acc + p;
    }
    qa[(size_t)h * kvr + c] = acc;
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
    softmax_row_exact<NT>(S + (size_t)blockIdx.x * s_stride, seq, e, redf, sq);
}

// ---- weighted sum of the cached rows ------------------------------------------
// o[h][c] = chain over t of p[h][t] * c_kv[t][c] (product rounded, then
// added), from +0.  Wave = head, lane = latent column; the four waves of a
// work group share the cached rows through L1.
constexpr int MW_UNROLL = 16;
__global__ __launch_bounds__(256) void mla_wsum_kernel(const float *__restrict__ S, int s_stride,
                                                       const float *__restrict__ c_kv, int seq, int H, int kvr,
                                                       float *__restrict__ o_lat) {
    const int wave = threadIdx.x >> 6, ln = threadIdx.x & 63;
    const int h = blockIdx.y * 4 + wave, c = blockIdx.x * 64 + ln;
    if (h >= H)
        return;
    const float *p = S + (size_t)h * s_stride;
    const float *col = c_kv + min(c, kvr - 1);
    float acc = 0.0f;
    int t = 0;
    for (; t + MW_UNROLL <= seq; t += MW_UNROLL) {
        float v[MW_UNROLL], w[MW_UNROLL];
#pragma unroll
        for (int u = 0; u < MW_UNROLL; u++) {
            v[u] = col[(size_t)(t + u) * kvr];
            w[u] = p[t + u];
        }
#pragma unroll
        for (int u = 0; u < MW_UNROLL; u++) {
            const float x = w[u] * v[u];
            acc = acc + x;
        }
    }
    for (; t < seq; t++) {
        const float x = p[t] * col[(size_t)t * kvr];
        acc = acc + x;
    }
    if (c < kvr)
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
    Scratch qa, S, olat, act, kvb_stage;
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
    const int be = block_elems(t);
    int be_log2 = 0;
    while ((1 << be_log2) < be)
        be_log2++;
    // 1. absorb
    int ph = prof_begin(LOOMHIP_KT_MLA_ABSORB, st);
    hipLaunchKernelGGL(mla_absorb_kernel, dim3((unsigned)((kvr + 63) / 64), (unsigned)H), dim3(64), 0, st, t,
                       (const uint8_t *)a->wk, plane_bytes(t, a->nope, kvr), q_nope, (int)a->nope, (int)kvr,
                       (int)(kvr / be), be_log2, qa);
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
    hipLaunchKernelGGL(mla_wsum_kernel, dim3((unsigned)((kvr + 63) / 64), (unsigned)((H + 3) / 4)), dim3(256), 0, st,
                       S, (int)s_stride, c_kv, (int)seq, (int)H, (int)kvr, ol);
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

static int ensure_cache() {
    if (g_mla.cache)
        return LOOMHIP_OK;
    if (!g_mla.want)
        return fail(LOOMHIP_DECLINED, "mla: no cache shape (mlaInit)");
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
    // kv_b split per head into the device layout once per host tensor
    KvbSplit &ks = g_mla.kvb[kv_b];
    if (ks.t != kvb_type || ks.len != kvb_len || ks.H != n_heads || ks.nope != nope || ks.vd != vd || ks.kvr != kvr) {
        (void)hipStreamSynchronize(st);
        if (ks.wk)
            (void)hipFree(ks.wk);
        if (ks.wv)
            (void)hipFree(ks.wv);
        ks = KvbSplit{};
        void *wk = nullptr, *wv = nullptr;
        hipError_t e = hipMalloc(&wk, plane_bytes(kvb_type, nope, kvr) * n_heads);
        if (e == hipSuccess)
            e = hipMalloc(&wv, plane_bytes(kvb_type, vd, kvr) * n_heads);
        int rc = e == hipSuccess ? reserve_on(g_mla.kvb_stage, kvb_len, st) : hip_fail(e, "hipMalloc kv_b split");
        if (rc == LOOMHIP_OK) {
            e = hipMemcpy(g_mla.kvb_stage.ptr, kv_b, kvb_len, hipMemcpyHostToDevice);
            rc = e == hipSuccess ? mla_split(kvb_type, g_mla.kvb_stage.ptr, n_heads, nope, vd, kvr, wk, wv, st)
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
        ks = KvbSplit{kvb_type, kvb_len, n_heads, nope, vd, kvr, wk, wv};
    }
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
    const loomhip_mla_attn a{kvb_type, ks.wk, ks.wv, n_heads, nope, vd, kvr, rope, scale};
    rc = mla_attn_impl(&a, cache_c(li, 0), cache_r(li, 0), seq, dq, dq + qn, (float *)g_ctx.ostage.ptr, nullptr, st);
    if (rc)
        return rc;
    e = hipMemcpyAsync(out, g_ctx.ostage.ptr, out_len * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "mla_attn_heads");
}

} // extern "C"
