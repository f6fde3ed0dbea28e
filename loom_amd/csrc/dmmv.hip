// dmmv.hip -- grouped dequant-fused matvec for Q4_0 / Q8_0 / Q4_K / Q6_K with
// int8 activations, bit-identical to the reference CPU kernels
// (src/gguf/ggml.zig:1002-1038 kBlockDot/matvecK256, 1196-1222 matvecQ40Int,
// 1277-1294 matvecQ80Int).
//
// Work map (wave64).  A block (32 or 256 weights) is served by LPB lanes:
// 8 for the K-quants (each lane owns 16 bytes of quants = 32 weights), 2 for
// Q8_0, 1 for Q4_0, so a wave covers BPI = 64/LPB blocks per step.  A wave
// walks its rows with the lane->block map fixed, so each lane's int8
// activation chunk is loaded once and reused for every row (and every token
// of its group).  Each lane computes exact integer partial dots with
// v_dot4_i32_i8, the LPB lanes of a block reduce them with DPP, and the block
// leader applies the reference's f32 tail.  Per-block results go to LDS and
// each output row is summed over its blocks sequentially in block order --
// the reference's `acc += r` -- so the result is bit-identical to the CPU.
#include "fmt.hpp"
#include "frame.hpp"

namespace lh {



// Per-block results of one row tile (TR = WAVES * rpw rows from row0) for n
// <= NT activation vectors vec[0..n) against weight plane wb (and wb2 when
// FUSED), written to lds[((m * NT + k) * TR + rl) * nb + b] for matrix m.
// The activations may live in global memory or in LDS (generic pointers).
template <int T, int NT, bool FUSED>
__device__ inline void tile_partials(const uint8_t *wb, const uint8_t *wb2, int rows, int cols,
                                     const int8_t *xq, const float *xd, const int32_t *xs,
                                     const int *vec, int n, int row0, int rpw, float *lds) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB, BPI = 64 / LPB;
    const int nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int TR = WAVES * rpw;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / LPB, j = lane % LPB;
    const bool wide = nb >= BPI;
    const int C = wide ? (nb + BPI - 1) / BPI : 1; // the last chunk may be partial
    const int RPI = wide ? 1 : BPI / nb;
    const int ro = wide ? 0 : grp / nb;
    const bool active = wide || grp < RPI * nb;
    const int nit = (rpw + RPI - 1) / RPI;
    const size_t lds_mat = (size_t)NT * TR * nb; // floats per matrix

    if constexpr (NT == 1 && !FUSED) {
        // one vector, up to 4 chunks per row: every chunk's activations, then
        // all of a row's chunks' weights, are in flight together
        if (wide && C <= 4) {
            typename F::X xc[4];
            int bcs[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int bc = c * BPI + grp;
                bcs[c] = bc;
                if (c < C)
                    xc[c] = F::load_x(xq, xd, xs, cols, vec[0], bc < nb ? bc : nb - 1, j);
            }
#pragma unroll 2
            for (int it = 0; it < rpw; it++) {
                const int rl = wave * rpw + it;
                const int row = row0 + rl;
                const bool rok = row < rows;
                typename F::W w[4];
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if (c < C) {
                        const int b = bcs[c] < nb ? bcs[c] : nb - 1;
                        w[c] = F::load_w(wb, U, (size_t)(rok ? row : 0) * nb + b, j);
                    }
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if (c < C) {
                        int is, ms;
                        F::dot(w[c], xc[c], j, is, ms);
                        is = group_sum<LPB>(is);
                        ms = group_sum<LPB>(ms);
                        if (rok && bcs[c] < nb && j == 0)
                            lds[(size_t)rl * nb + bcs[c]] = F::tail(w[c], xc[c], is, ms);
                    }
            }
            return;
        }
    }

    for (int c = 0; c < C; c++) {
        const int bc = wide ? c * BPI + grp : (grp % nb);
        const bool bok = bc < nb;
        const int b = bok ? bc : nb - 1; // lanes past the row's end read a real block, write nothing
        typename F::X xr[NT];
#pragma unroll
        for (int k = 0; k < NT; k++)
            xr[k] = F::load_x(xq, xd, xs, cols, vec[k < n ? k : 0], b, j);
#pragma unroll 2
        for (int it = 0; it < nit; it++) {
            const int rw = it * RPI + ro;    // row within this wave's span
            const int rl = wave * rpw + rw;  // row within the tile
            const int row = row0 + rl;
            const bool valid = active && bok && rw < rpw && row < rows;
            const size_t unit = (size_t)(valid ? row : 0) * nb + b;
            const typename F::W w = F::load_w(wb, U, unit, j);
            typename F::W w2;
            if constexpr (FUSED)
                w2 = F::load_w(wb2, U, unit, j);
#pragma unroll
            for (int k = 0; k < NT; k++) {
                if (k < n) {
                    int is, ms;
                    F::dot(w, xr[k], j, is, ms);
                    is = group_sum<LPB>(is);
                    ms = group_sum<LPB>(ms);
                    if (valid && j == 0)
                        lds[((size_t)k * TR + rl) * nb + b] = F::tail(w, xr[k], is, ms);
                    if constexpr (FUSED) {
                        F::dot(w2, xr[k], j, is, ms);
                        is = group_sum<LPB>(is);
                        ms = group_sum<LPB>(ms);
                        if (valid && j == 0)
                            lds[lds_mat + ((size_t)k * TR + rl) * nb + b] = F::tail(w2, xr[k], is, ms);
                    }
                }
            }
        }
    }
}

// ---- grouped matvec: one work group per (row tile, group of <= NT vectors
// sharing one weight plane) -------------------------------------------------------
template <int T, int NT, bool FUSED>
__device__ __forceinline__ void dmmv_tile(const DmmvParams &p, int tile, int group, float *lds, int *vec) {
    using F = Fmt<T>;
    const DmmvGroup g = p.groups[group];
    const int n = g.n;
    const int nb = p.cols / F::BE;
    const int TR = WAVES * p.rpw;
    const int row0 = tile * TR;
    if (threadIdx.x < NT)
        vec[threadIdx.x] = p.pair_src[g.first + ((int)threadIdx.x < n ? threadIdx.x : 0)];
    __syncthreads();
    const uint8_t *wb = p.w + (size_t)g.plane * p.plane_bytes;
    const uint8_t *wb2 = FUSED ? p.w2 + (size_t)g.plane * p.plane_bytes : nullptr;
    tile_partials<T, NT, FUSED>(wb, wb2, p.rows, p.cols, p.xq, p.xd, p.xs, vec, n, row0, p.rpw, lds);
    __syncthreads();
    const size_t lds_mat = (size_t)NT * TR * nb;
    for (int idx = threadIdx.x; idx < n * TR; idx += blockDim.x) {
        const int k = idx / TR, rl = idx % TR, row = row0 + rl;
        if (row >= p.rows)
            continue;
        float *o = p.out + (size_t)p.pair_dst[g.first + k] * p.out_stride + row;
        const float v = row_value<FUSED>(lds, lds_mat, (size_t)k * TR + rl, nb);
        *o = p.accumulate ? *o + v : v;
    }
}

template <int T, int NT, bool FUSED>
__global__ __launch_bounds__(256) void dmmv_kernel(DmmvParams p) {
    extern __shared__ float lds[];
    __shared__ int vec[NT];
    const int ng = p.n_groups_dev ? *p.n_groups_dev : p.n_groups;
    if ((int)blockIdx.y >= ng)
        return;
    dmmv_tile<T, NT, FUSED>(p, blockIdx.x, blockIdx.y, lds, vec);
}

// ---- several matrices against one activation set in one launch ------------------
// Work groups [0, tiles_0) serve segment 0, the next tiles_1 segment 1, ...;
// each segment has its own type, rows, rows per wave and output.  Same
// arithmetic per row as dmmv_kernel.
template <int NT>
__global__ __launch_bounds__(256) void dmmv_seg_kernel(DmmvSegParams sp) {
    extern __shared__ float lds[];
    __shared__ int vec[NT];
    int s = 0, bx = blockIdx.x;
    while (s + 1 < sp.n_seg && bx >= sp.seg[s].tiles) {
        bx -= sp.seg[s].tiles;
        s++;
    }
    DmmvParams p = sp.base;
    p.w = sp.seg[s].w;
    p.rows = sp.seg[s].rows;
    p.rpw = sp.seg[s].rpw;
    p.out = sp.seg[s].out;
    p.out_stride = sp.seg[s].rows;
    switch (sp.seg[s].t) {
    case LH_Q4_K:
        dmmv_tile<LH_Q4_K, NT, false>(p, bx, blockIdx.y, lds, vec);
        break;
    case LH_Q6_K:
        dmmv_tile<LH_Q6_K, NT, false>(p, bx, blockIdx.y, lds, vec);
        break;
    case LH_Q8_0:
        dmmv_tile<LH_Q8_0, NT, false>(p, bx, blockIdx.y, lds, vec);
        break;
    default:
        dmmv_tile<LH_Q4_0, NT, false>(p, bx, blockIdx.y, lds, vec);
        break;
    }
}

// ---- the attention rmsnorm fused into q, k and v (PARITY, one vector) -----------
// Every work group normalises x itself (the reference's sequential sum of the
// squares, 4 waves) and quantizes the row for the segments' activation block
// into LDS, then runs dmmv_seg_kernel's tile against that LDS copy: the norm
// launch, its HBM round trip of the int8 row and one launch gap leave the
// layer.  Same values as norm_quant_kernel<QB, true> followed by
// dmmv_seg_kernel<1>.
constexpr int NSEG_MAX_DIM = 4096;
constexpr int NSEG_XV = norm_xv(NSEG_MAX_DIM, 4);

__global__ __launch_bounds__(256) void norm_seg_kernel(DmmvSegParams sp, const float *__restrict__ x,
                                                       const float *__restrict__ nw, float eps) {
    extern __shared__ float lds[];
    __shared__ int vec[1];
    __shared__ __align__(16) float xn[NSEG_MAX_DIM];
    __shared__ SeqSumLds seq;
    __shared__ __align__(16) int8_t aq[NSEG_MAX_DIM];
    __shared__ float ad[NSEG_MAX_DIM / 32];
    __shared__ int32_t as[NSEG_MAX_DIM / 16];
    const int dim = sp.base.cols;
    float4 xv[NSEG_XV], wv[NSEG_XV];
    norm_exact_load<4, NSEG_XV>(x, nw, dim, xv, wv);
    norm_exact_block<4, NSEG_XV>(xv, wv, dim, eps, xn, seq);
    // the row for the segments' weight type (they share its activation block)
    const int qt = sp.seg[0].t;
    const int items = quant_items(qt, dim);
    for (int it = (int)threadIdx.x >> 6; it < items; it += 4)
        quant_item_wave(qt, xn, dim, 0, it, QAct{aq, ad, as});
    lds_barrier();
    int s = 0, bx = blockIdx.x;
    while (s + 1 < sp.n_seg && bx >= sp.seg[s].tiles) {
        bx -= sp.seg[s].tiles;
        s++;
    }
    DmmvParams p = sp.base;
    p.w = sp.seg[s].w;
    p.rows = sp.seg[s].rows;
    p.rpw = sp.seg[s].rpw;
    p.out = sp.seg[s].out;
    p.out_stride = sp.seg[s].rows;
    p.xq = aq;
    p.xd = ad;
    p.xs = as;
    switch (sp.seg[s].t) {
    case LH_Q4_K:
        dmmv_tile<LH_Q4_K, 1, false>(p, bx, 0, lds, vec);
        break;
    case LH_Q6_K:
        dmmv_tile<LH_Q6_K, 1, false>(p, bx, 0, lds, vec);
        break;
    case LH_Q8_0:
        dmmv_tile<LH_Q8_0, 1, false>(p, bx, 0, lds, vec);
        break;
    default:
        dmmv_tile<LH_Q4_0, 1, false>(p, bx, 0, lds, vec);
        break;
    }
}

// One vector (sp.base: n_groups 1, identity pairs): false = not served (the
// caller normalises and runs launch_dmmv_seg instead).
bool launch_norm_seg(DmmvSegParams sp, const float *x, const float *norm_w, float eps, hipStream_t st) {
    const int dim = sp.base.cols;
    if (dim > NSEG_MAX_DIM || dim % 256 || sp.base.n_groups != 1 || sp.n_seg < 1)
        return false;
    size_t lds = 0;
    int tiles = 0;
    for (int i = 0; i < sp.n_seg; i++) {
        DmmvSeg &g = sp.seg[i];
        if (act_block(g.t) != act_block(sp.seg[0].t))
            return false;
        g.rpw = dmmv_pick_rpw(g.t, dim, g.rows, 1, 1, false);
        g.tiles = (g.rows + WAVES * g.rpw - 1) / (WAVES * g.rpw);
        tiles += g.tiles;
        const size_t l = dmmv_lds_bytes(g.t, dim, 1, false, g.rpw);
        lds = l > lds ? l : lds;
    }
    if (lds > 64 * 1024)
        return false;
    hipLaunchKernelGGL(norm_seg_kernel, dim3(tiles), dim3(256), lds, st, sp, x, norm_w, eps);
    note_launch();
    return true;
}

bool launch_dmmv_seg(int nt, DmmvSegParams sp, hipStream_t st) {
    size_t lds = 0;
    int tiles = 0;
    for (int i = 0; i < sp.n_seg; i++) {
        DmmvSeg &g = sp.seg[i];
        g.rpw = dmmv_pick_rpw(g.t, sp.base.cols, g.rows, sp.base.n_groups, nt, false);
        g.tiles = (g.rows + WAVES * g.rpw - 1) / (WAVES * g.rpw);
        tiles += g.tiles;
        const size_t l = dmmv_lds_bytes(g.t, sp.base.cols, nt, false, g.rpw);
        lds = l > lds ? l : lds;
    }
    if (lds > 64 * 1024)
        return false;
    const dim3 grid(tiles, sp.base.n_groups);
    switch (nt) {
    case 1:
        hipLaunchKernelGGL(dmmv_seg_kernel<1>, grid, dim3(256), lds, st, sp);
        break;
    case 2:
        hipLaunchKernelGGL(dmmv_seg_kernel<2>, grid, dim3(256), lds, st, sp);
        break;
    case 4:
        hipLaunchKernelGGL(dmmv_seg_kernel<4>, grid, dim3(256), lds, st, sp);
        break;
    default:
        hipLaunchKernelGGL(dmmv_seg_kernel<8>, grid, dim3(256), lds, st, sp);
        break;
    }
    note_launch();
    return true;
}

bool dmmv_supported(int t, int cols) {
    if (cols <= 0)
        return false;
    switch (t) {
    case LH_Q4_K:
    case LH_Q6_K:
        return cols % 256 == 0;
    case LH_Q8_0:
    case LH_Q4_0:
        return cols % 32 == 0;
    default:
        return false;
    }
}

static int lpb_of(int t) { return (t == LH_Q4_K || t == LH_Q6_K) ? 8 : t == LH_Q8_0 ? 2 : 1; }

int dmmv_pick_rpw(int t, int cols, int rows, int groups, int nt, bool fused) {
    // Aim for >= ~2048 work groups across the chip (256 CUs x 8 waves), keep
    // at least one full wave step of rows, and stay inside the LDS budget of
    // the per-block partials ((fused ? 2 : 1) * nt * 4 * rpw * nb floats).
    const int nb = cols / block_elems(t);
    const int bpi = 64 / lpb_of(t);
    const int rpi = nb >= bpi ? 1 : bpi / nb;
    int rpw = 16;
    while (rpw > 2 && (long)((rows + WAVES * rpw - 1) / (WAVES * rpw)) * groups < 2048)
        rpw /= 2;
    if (rpw < rpi)
        rpw = rpi;
    const long per_row = (long)(fused ? 2 : 1) * nt * WAVES * nb * (long)sizeof(float);
    while (rpw > 1 && rpw > rpi && per_row * rpw > DMMV_LDS_BUDGET)
        rpw--;
    return rpw;
}

size_t dmmv_lds_bytes(int t, int cols, int nt, bool fused, int rpw) {
    return (size_t)(fused ? 2 : 1) * nt * WAVES * rpw * (cols / block_elems(t)) * sizeof(float);
}

template <int T, int NT, bool FUSED>
static void launch_t(const DmmvParams &p, hipStream_t st) {
    const int TR = WAVES * p.rpw;
    const size_t lds = dmmv_lds_bytes(T, p.cols, NT, FUSED, p.rpw);
    dim3 grid((p.rows + TR - 1) / TR, p.n_groups);
    hipLaunchKernelGGL((dmmv_kernel<T, NT, FUSED>), grid, dim3(256), lds, st, p);
}

template <int T, bool FUSED>
static void launch_nt(int nt, const DmmvParams &p, hipStream_t st) {
    switch (nt) {
    case 1:
        launch_t<T, 1, FUSED>(p, st);
        break;
    case 2:
        launch_t<T, 2, FUSED>(p, st);
        break;
    case 4:
        launch_t<T, 4, FUSED>(p, st);
        break;
    default:
        launch_t<T, 8, FUSED>(p, st);
        break;
    }
}

template <int T>
static void launch_f(int nt, bool fused, const DmmvParams &p, hipStream_t st) {
    if (fused)
        launch_nt<T, true>(nt, p, st);
    else
        launch_nt<T, false>(nt, p, st);
}

bool launch_dmmv(int t, int nt, bool fused, const DmmvParams &p, hipStream_t st) {
    if (dmmv_lds_bytes(t, p.cols, nt, fused, p.rpw) > 64 * 1024)
        return false;
    switch (t) {
    case LH_Q4_K:
        launch_f<LH_Q4_K>(nt, fused, p, st);
        break;
    case LH_Q6_K:
        launch_f<LH_Q6_K>(nt, fused, p, st);
        break;
    case LH_Q8_0:
        launch_f<LH_Q8_0>(nt, fused, p, st);
        break;
    case LH_Q4_0:
        launch_f<LH_Q4_0>(nt, fused, p, st);
        break;
    default:
        return false;
    }
    note_launch();
    return true;
}

} // namespace lh
