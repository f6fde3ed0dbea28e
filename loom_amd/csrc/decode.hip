// decode.hip -- the MoE layer's decode path (a few tokens per step): every
// (token, slot) pair runs on its own, so no bucketing is needed and no work
// group waits for another inside a launch.  Both kernels are arranged around
// memory latency: independent loads are issued together, and the weight
// loads of a work group are in flight while it routes or quantizes.
//
//   gate/up  one work group per (token, slot, row tile): the four waves rank
//            the token's experts (src/gguf/moe.zig:106-158) while every lane's
//            activation chunk is loading; then fused gate/up + SwiGLU of the
//            slot's expert (src/gguf/llama.zig denseFFN 952-958), f32 out
//   down     one work group per (token, row tile): the token's k SwiGLU vectors
//            are quantized into LDS and its gates computed while the weight
//            rows of all k slots load; then down for every slot and the gated
//            combine (llama.zig moeRun 1363-1398 / moeBatchUnion 1844-1903)
#include "fmt.hpp"

namespace lh {

// Lane map shared by the decode kernels (see fmt.hpp): a block is served by
// LPB lanes, a wave covers BPI = 64/LPB blocks per step.  Wide rows (nb >=
// BPI) take C column chunks of BPI blocks, the last one possibly partial;
// short rows put RPI rows side by side.
template <int LPB>
struct LaneMap {
    static constexpr int BPI = 64 / LPB;
    int grp, j, nb, C, RPI, ro;
    bool wide, active;
    __device__ LaneMap(int lane, int nb_) : nb(nb_) {
        grp = lane / LPB;
        j = lane % LPB;
        wide = nb >= BPI;
        C = wide ? (nb + BPI - 1) / BPI : 1;
        RPI = wide ? 1 : BPI / nb;
        ro = wide ? 0 : grp / nb;
        active = wide || grp < RPI * nb;
    }
    // block of column chunk c (clamped into range; ok = a real block)
    __device__ int block(int c, bool &ok) const {
        const int b = wide ? c * BPI + grp : grp % nb;
        ok = b < nb;
        return ok ? b : nb - 1;
    }
};

constexpr int GU_MAXIT = 2; // weight rows per lane requested at once in the gate/up kernel

// Gate/up + SwiGLU for pair (token t, slot s) = blockIdx.y, row tile
// blockIdx.x.  The four waves find slot s's expert (route_decode_slot, NI =
// ceil(E/64)) while the first column chunk's activations load; the (slot 0,
// tile 0) work group publishes the ids.  Gates are computed exactly by the
// down kernel.
template <int T, int NI>
__global__ __launch_bounds__(256) void moe_gateup_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB;
    extern __shared__ __align__(16) float lds[];
    __shared__ RouteLds<WAVES> rl;
    const int K = p.k;
    const int t = blockIdx.y / K, s = blockIdx.y % K;
    const int rows = p.ffn, cols = p.dim, nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int rpw = p.rpw_gu, TR = WAVES * rpw;
    const int row0 = blockIdx.x * TR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const LaneMap<LPB> m(lane, nb);
    const int j = m.j;
    const int nit = (rpw + m.RPI - 1) / m.RPI;
    const size_t lds_mat = (size_t)TR * nb;

    bool ok0;
    const int b0 = m.block(0, ok0);
    const typename F::X x0 = F::load_x(p.xq, p.xd, p.xs, cols, t, b0, j);
    const int e0 = route_decode_slot<NI>(p.logits + (size_t)t * p.n_expert, p.sel_bias, p.n_expert, K,
                                         p.gating, s, rl,
                                         s == 0 && blockIdx.x == 0 ? p.ids + (size_t)t * K : nullptr);
    const int e = min(max(e0, 0), p.n_expert - 1); // never address past the tensor
    const uint8_t *wb = p.gate + (size_t)e * p.gu_plane;
    const uint8_t *wb2 = p.up + (size_t)e * p.gu_plane;
    for (int c = 0; c < m.C; c++) {
        bool bok;
        const int b = m.block(c, bok);
        const typename F::X xr = c == 0 ? x0 : F::load_x(p.xq, p.xd, p.xs, cols, t, b, j);
        for (int it0 = 0; it0 < nit; it0 += GU_MAXIT) {
            typename F::W w[GU_MAXIT], w2[GU_MAXIT];
            int rlv[GU_MAXIT];
            bool valid[GU_MAXIT];
#pragma unroll
            for (int u = 0; u < GU_MAXIT; u++) {
                const int rw = (it0 + u) * m.RPI + m.ro;
                rlv[u] = wave * rpw + rw;
                const int row = row0 + rlv[u];
                valid[u] = m.active && bok && it0 + u < nit && rw < rpw && row < rows;
                const size_t unit = (size_t)(valid[u] ? row : 0) * nb + b;
                w[u] = F::load_w(wb, U, unit, j);
                w2[u] = F::load_w(wb2, U, unit, j);
            }
#pragma unroll
            for (int u = 0; u < GU_MAXIT; u++) {
                if (it0 + u < nit) {
                    int is, ms;
                    F::dot(w[u], xr, j, is, ms);
                    is = group_sum<LPB>(is);
                    ms = group_sum<LPB>(ms);
                    if (valid[u] && j == 0)
                        lds[(size_t)rlv[u] * nb + b] = F::tail(w[u], xr, is, ms);
                    F::dot(w2[u], xr, j, is, ms);
                    is = group_sum<LPB>(is);
                    ms = group_sum<LPB>(ms);
                    if (valid[u] && j == 0)
                        lds[lds_mat + (size_t)rlv[u] * nb + b] = F::tail(w2[u], xr, is, ms);
                }
            }
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < TR; r += blockDim.x) {
        const int row = row0 + r;
        if (row < rows)
            p.act[(size_t)blockIdx.y * rows + row] = row_value<true>(lds, lds_mat, r, nb);
    }
}

// Token t's exact gates by one wave (moe.zig:143-157), lane s < K returning
// slot s's: the selected experts' scores in the reference's arithmetic
// (sigmoid, raw logits for softmax_topk, or softmax's exp(l - max) times
// 1/sum with the sum sequential over experts, tensor.zig:18-36), then the
// gate post-processing.  my_id is the slot's expert (lane s < K); lv holds
// the token's logits (lane + 64i, -inf past E); sc is this wave's LDS.
__device__ __forceinline__ float decode_gates(const DecodeParams &p, int my_id,
                                              const float (&lv)[MAX_E / 64], float *sc) {
    constexpr int NI = MAX_E / 64;
    const int lane = threadIdx.x & 63, K = p.k;
    float g;
    if (p.gating == 2 || p.gating == 3) {
        // the selected logit, from the lane that holds it
        float l = 0.0f;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const float v = __int_as_float(
                __builtin_amdgcn_ds_bpermute((my_id & 63) << 2, __float_as_int(lv[i])));
            if ((my_id >> 6) == i)
                l = v;
        }
        g = p.gating == 2 ? 1.0f / (1.0f + exp_f32_poly(-l)) : l;
    } else {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NI; i++)
            mx = fmaxf(mx, lv[i]);
        mx = wave_max(mx);
#pragma unroll
        for (int i = 0; i < NI; i++)
            sc[lane + 64 * i] = exp_f32_poly(lv[i] - mx);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const float inv = 1.0f / lds_seq_sum(sc, p.n_expert);
        g = sc[my_id] * inv;
    }
    return gates_post(lane < K ? g : 0.0f, K, p.gating, p.weights_norm, p.weights_scale);
}

constexpr int DN_UB = 8; // weight rows per lane requested at once in the down kernel

// Down + gated combine for token t = blockIdx.y, row tile blockIdx.x.
//   1. every wave loads the token's expert ids (lane s: slot s), its share
//      of the token's k SwiGLU vectors (f32, as gate/up wrote them) and the
//      token's router logits (for the last wave's gates)
//   2. the weight rows of the first DN_UB iterations are requested, each
//      lane's expert taken from lane `slot` by ds_bpermute
//   3. while they load, the last wave computes the gates and the waves
//      quantize the vectors into LDS (quantizeX / quantizeX256 of the down
//      type), 32 values per lane
//   4. dots against the quantized vectors, per-block partials to LDS
//   5. every (slot, row) value summed over its blocks in block order, then
//      the combine: mode 0 (moeRun) out = ((0 + g0*y0) + g1*y1) + ... in
//      selection order; mode 1 (moeBatchUnion) out += g*y per expert in
//      ascending expert id; mode 2 out = out + (the mode-0 sum)
template <int T>
__global__ __launch_bounds__(256) void moe_down_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB;
    constexpr int QB = act_block(T);
    constexpr int NI = MAX_E / 64;
    extern __shared__ __align__(16) float lds[];
    __shared__ float s_gates[MAX_K];
    __shared__ int s_ids[MAX_K];
    __shared__ __align__(16) float s_sc[MAX_E];
    const int K = p.k, E = p.n_expert, t = blockIdx.y, cols = p.ffn, rows = p.dim;
    const int nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int rpw = p.rpw_dn, TR = WAVES * rpw; // rpw a power of two (moe_run)
    const int tr_log2 = __builtin_ctz(TR);
    const int row0 = blockIdx.x * TR;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const bool gate_wave = wave == WAVES - 1;
    const LaneMap<LPB> m(lane, nb);
    const int j = m.j;
    // virtual rows (slot, row): wave w owns [w*VPW, (w+1)*VPW)
    const int VPW = K * rpw;
    const int nit = (VPW + m.RPI - 1) / m.RPI;
    // LDS: partials [K][TR][nb] f32 | q [K][cols] i8 | d [K][cols/QB] f32 | s [K][cols/16 or /32] i32
    const int nd = cols / QB, ns = QB == 256 ? cols / 16 : cols / 32;
    float *part = lds;
    int8_t *qq = (int8_t *)(part + (size_t)K * TR * nb);
    float *qd = (float *)(qq + align16((size_t)K * cols));
    int32_t *qs = (int32_t *)(qd + align16((size_t)K * nd * 4) / 4);
    const size_t v0 = (size_t)t * K;
    const float *act = p.act + v0 * cols;

    // 1. ids, the first activation chunks, logits
    const uint32_t raw_id = p.ids[v0 + min(lane, K - 1)]; // used after the loads below are issued
    // the activations in 32-value chunks, one per lane per pass of the work
    // group: cols is a multiple of 256 (launch_moe_decode), so the k vectors
    // quantize as one buffer of k*cols values with the same LDS layout
    const int chunks = K * cols / 32;
    float4 xv[8];
    auto load_chunk = [&](int ch) {
        const float *src = act + (size_t)min(ch, chunks - 1) * 32; // clamped: unconditional loads
#pragma unroll
        for (int i = 0; i < 8; i++)
            xv[i] = *(const float4 *)(src + 4 * i);
    };
    load_chunk(threadIdx.x);
    float lv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++)
        lv[i] = p.logits[(size_t)t * E + min(lane + 64 * i, E - 1)];

    // 2. weight rows of the first iterations
    const int my_id = lane < K ? (int)min(raw_id, (uint32_t)(E - 1)) : 0;
    int c = 0, it0 = 0;
    bool bok;
    int b = m.block(0, bok);
    typename F::W w[DN_UB];
    int slot[DN_UB], rlv[DN_UB];
    bool valid[DN_UB];
    auto issue = [&]() {
        int e[DN_UB];
#pragma unroll
        for (int u = 0; u < DN_UB; u++) {
            const int vl = (it0 + u) * m.RPI + m.ro;
            const int vr = wave * VPW + vl;
            slot[u] = vr >> tr_log2; // TR is a power of two
            rlv[u] = vr & (TR - 1);
            valid[u] = m.active && bok && it0 + u < nit && vl < VPW && row0 + rlv[u] < rows;
            e[u] = __builtin_amdgcn_ds_bpermute((valid[u] ? slot[u] : 0) << 2, my_id);
        }
#pragma unroll
        for (int u = 0; u < DN_UB; u++) {
            const size_t unit = (size_t)(valid[u] ? row0 + rlv[u] : 0) * nb + b;
            w[u] = F::load_w(p.down + (size_t)e[u] * p.dn_plane, U, unit, j);
        }
    };
    issue();
    __builtin_amdgcn_sched_barrier(0); // the weight requests go out before the quantization

    // 3. the last wave computes the gates (a sequential sum over the experts
    // for softmax) while the other waves quantize: the first pass of chunks
    // covers [0, 256) and leaves the last wave idle when k*cols <= 6144
    if (gate_wave) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            lv[i] = lane + 64 * i < E ? lv[i] : -INFINITY;
        const float g = decode_gates(p, my_id, lv, s_sc);
        if (lane < K) {
            s_gates[lane] = g;
            if (blockIdx.x == 0)
                p.gates[v0 + lane] = g;
        }
    }
    // quantize into LDS; the first pass in straight-line code, so its wait
    // covers the chunk loads and not the weight loads issued after them
    // (later passes, for k*cols > 8192, wait for both)
    if (wave * 64 < chunks)
        quant_chunk32<QB>(xv, (int)threadIdx.x < chunks, threadIdx.x, qq, qd, qs);
    for (int c0 = blockDim.x; c0 < chunks; c0 += blockDim.x) {
        load_chunk(c0 + threadIdx.x);
        quant_chunk32<QB>(xv, c0 + (int)threadIdx.x < chunks, c0 + threadIdx.x, qq, qd, qs);
    }
    if (wave == 0 && lane < K)
        s_ids[lane] = my_id;
    lds_barrier();

    // 4. dots against the quantized vectors in LDS
    for (;;) {
#pragma unroll
        for (int u = 0; u < DN_UB; u++) {
            if (it0 + u < nit) {
                const typename F::X x = F::load_x(qq, qd, qs, cols, valid[u] ? slot[u] : 0, b, j);
                int is, ms;
                F::dot(w[u], x, j, is, ms);
                is = group_sum<LPB>(is);
                ms = group_sum<LPB>(ms);
                if (valid[u] && j == 0)
                    part[((size_t)slot[u] * TR + rlv[u]) * nb + b] = F::tail(w[u], x, is, ms);
            }
        }
        it0 += DN_UB;
        if (it0 >= nit) {
            it0 = 0;
            if (++c >= m.C)
                break;
            b = m.block(c, bok);
        }
        issue();
    }
    __syncthreads();
    // 5. slot values, then the combine
    float *yv = part + (size_t)K * TR * nb; // reuses the activation staging
    for (int i = threadIdx.x; i < K * TR; i += blockDim.x)
        yv[i] = row_value<false>(part, 0, i, nb); // i = slot * TR + row
    __syncthreads();
    for (int r = threadIdx.x; r < TR; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= rows)
            continue;
        float *o = p.out + (size_t)t * rows + row;
        if (p.mode != 1) {
            float acc = 0.0f;
            for (int sl = 0; sl < K; sl++) {
                const float pr = s_gates[sl] * yv[sl * TR + r];
                acc = acc + pr;
            }
            *o = p.mode == 2 ? *o + acc : acc;
        } else {
            float acc = *o;
            int prev = -1;
            for (int step = 0; step < K; step++) {
                int bs = -1, be = 0x7fffffff;
                for (int sl = 0; sl < K; sl++) {
                    const int e = s_ids[sl];
                    if (e > prev && e < be) {
                        be = e;
                        bs = sl;
                    }
                }
                if (bs < 0)
                    break;
                const float pr = s_gates[bs] * yv[bs * TR + r];
                acc = acc + pr;
                prev = be;
            }
            *o = acc;
        }
    }
}

size_t decode_down_lds(int down_t, int ffn, int k, int rpw) {
    const int nb = ffn / block_elems(down_t);
    const int QB = act_block(down_t);
    const int nd = ffn / QB, ns = QB == 256 ? ffn / 16 : ffn / 32;
    const size_t staging = align16((size_t)k * ffn) + align16((size_t)k * nd * 4) + (size_t)k * ns * 4;
    const size_t yv = (size_t)k * WAVES * rpw * 4; // the slot values reuse the staging
    return (size_t)k * WAVES * rpw * nb * 4 + (staging > yv ? staging : yv);
}

size_t decode_gateup_lds(int gate_t, int dim, int rpw) {
    return (size_t)2 * WAVES * rpw * (dim / block_elems(gate_t)) * 4;
}

template <int T>
static void launch_gateup_decode_t(const DecodeParams &p, int n, hipStream_t st) {
    const int TR = WAVES * p.rpw_gu;
    const dim3 grid((p.ffn + TR - 1) / TR, n * p.k);
    const size_t lds = decode_gateup_lds(T, p.dim, p.rpw_gu);
    if (p.n_expert <= 64)
        hipLaunchKernelGGL((moe_gateup_decode_kernel<T, 1>), grid, dim3(256), lds, st, p);
    else if (p.n_expert <= 128)
        hipLaunchKernelGGL((moe_gateup_decode_kernel<T, 2>), grid, dim3(256), lds, st, p);
    else
        hipLaunchKernelGGL((moe_gateup_decode_kernel<T, 4>), grid, dim3(256), lds, st, p);
}

template <int T>
static void launch_down_decode_t(const DecodeParams &p, int n, hipStream_t st) {
    const int TR = WAVES * p.rpw_dn;
    hipLaunchKernelGGL(moe_down_decode_kernel<T>, dim3((p.dim + TR - 1) / TR, n), dim3(256),
                       decode_down_lds(T, p.ffn, p.k, p.rpw_dn), st, p);
}

static bool decode_type(int t) { return t == LH_Q4_K || t == LH_Q6_K || t == LH_Q8_0 || t == LH_Q4_0; }

bool decode_supported(int gate_t, int down_t, int ffn) {
    return decode_type(gate_t) && decode_type(down_t) && ffn % 256 == 0;
}

bool launch_moe_decode(int gate_t, int down_t, const DecodeParams &p, int n, hipStream_t st,
                       int prof_gu, int prof_dn) {
    if (!decode_supported(gate_t, down_t, p.ffn) || p.rpw_dn <= 0 || (p.rpw_dn & (p.rpw_dn - 1)) ||
        decode_gateup_lds(gate_t, p.dim, p.rpw_gu) > 64 * 1024 ||
        decode_down_lds(down_t, p.ffn, p.k, p.rpw_dn) > 64 * 1024)
        return false;
    int ph = prof_begin(prof_gu, st);
    switch (gate_t) {
    case LH_Q4_K: launch_gateup_decode_t<LH_Q4_K>(p, n, st); break;
    case LH_Q6_K: launch_gateup_decode_t<LH_Q6_K>(p, n, st); break;
    case LH_Q8_0: launch_gateup_decode_t<LH_Q8_0>(p, n, st); break;
    default: launch_gateup_decode_t<LH_Q4_0>(p, n, st); break;
    }
    prof_end(ph, st);
    note_launch();
    ph = prof_begin(prof_dn, st);
    switch (down_t) {
    case LH_Q4_K: launch_down_decode_t<LH_Q4_K>(p, n, st); break;
    case LH_Q6_K: launch_down_decode_t<LH_Q6_K>(p, n, st); break;
    case LH_Q8_0: launch_down_decode_t<LH_Q8_0>(p, n, st); break;
    default: launch_down_decode_t<LH_Q4_0>(p, n, st); break;
    }
    prof_end(ph, st);
    note_launch();
    return true;
}

} // namespace lh
