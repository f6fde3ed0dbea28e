// decode.hip -- the MoE layer's decode path (a few tokens per step): every
// (token, slot) pair runs on its own, so no bucketing and no communication
// between work groups is needed.  Both kernels are arranged around memory
// latency: independent loads are issued together, and the weight loads of a
// work group are in flight while it routes or quantizes.
//
//   gate/up  one work group per (token, slot, row tile): wave 0 routes the
//            token (src/gguf/moe.zig:106-158) while every lane's activation
//            chunk is loading; then fused gate/up + SwiGLU of the slot's expert
//            (src/gguf/llama.zig denseFFN 952-958)
//   down     one work group per (token, row tile): the token's k SwiGLU vectors
//            are quantized into LDS while the weight rows of all k slots load;
//            then down for every slot and the gated combine in-register
//            (llama.zig moeRun 1363-1398 / moeBatchUnion 1844-1903)
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
// blockIdx.x.  The four waves rank the token's experts (route_rank) while
// the first column chunk's activations load; the (slot 0, tile 0) work group
// publishes the ids.  Ranking softmax routes on the exp values: two experts
// can only come out in the other order when their exp values round to the
// same final score (a logit gap below one ulp), the near-tie case the
// north_star allows; gates are computed exactly by moe_mid_kernel.
template <int T>
__global__ __launch_bounds__(256) void moe_gateup_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB;
    extern __shared__ float lds[];
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
    route_rank<WAVES, false>(p.logits + (size_t)t * p.n_expert, p.sel_bias, p.n_expert, K,
                             p.gating, rl);
    const int e = min(max(rl.id[s], 0), p.n_expert - 1); // never address past the tensor
    if (s == 0 && blockIdx.x == 0 && (int)threadIdx.x < K)
        p.ids[(size_t)t * K + threadIdx.x] = (uint32_t)rl.id[threadIdx.x];
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

// Between gate/up and down, one wave per work group: waves [0, items)
// quantize one item of the SwiGLU vectors for the down type each (once, for
// every down work group); the next n waves compute token t's gates exactly
// (scores of the selected experts in the reference's arithmetic, then the
// gate post-processing), off the critical path of both expert kernels.
__global__ __launch_bounds__(64) void moe_mid_kernel(DecodeParams p, int n) {
    __shared__ __align__(16) float sc[MAX_E];
    const int per = quant_items(p.down_t, p.ffn);
    const int items = n * p.k * per;
    if ((int)blockIdx.x < items) {
        const int v = blockIdx.x / per, it = blockIdx.x % per;
        quant_item_wave(p.down_t, p.act + (size_t)v * p.ffn, p.ffn, v, it, p.qa);
        return;
    }
    const int t = blockIdx.x - items;
    const int lane = threadIdx.x, E = p.n_expert, K = p.k;
    const float *lg = p.logits + (size_t)t * E;
    const int id = lane < K ? min((int)p.ids[(size_t)t * K + lane], E - 1) : 0;
    float g;
    if (p.gating == 2) { // sigmoid (tensor.zig:34-36)
        g = 1.0f / (1.0f + expf(-lg[id]));
    } else if (p.gating == 3) { // softmax_topk: raw logits
        g = lg[id];
    } else { // softmax (tensor.zig:18-28): exp(l - max), sequential sum, * (1/sum)
        constexpr int NI = MAX_E / 64;
        float lv[NI];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int e = lane + 64 * i;
            lv[i] = e < E ? lg[e] : -INFINITY;
            mx = fmaxf(mx, lv[i]);
        }
        mx = wave_max(mx);
#pragma unroll
        for (int i = 0; i < NI; i++)
            sc[lane + 64 * i] = expf(lv[i] - mx);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const float inv = 1.0f / lds_seq_sum(sc, E);
        g = sc[id] * inv;
    }
    g = gates_post(lane < K ? g : 0.0f, K, p.gating, p.weights_norm, p.weights_scale);
    if (lane < K)
        p.gates[(size_t)t * K + lane] = g;
}

constexpr int DN_UB = 8; // weight rows per lane requested at once in the down kernel

// Down + gated combine for token t = blockIdx.y, row tile blockIdx.x.  The
// token's k quantized SwiGLU vectors are staged into LDS together with its
// ids and gates; then every slot's expert runs over the tile's rows and the
// results combine in-register: mode 0 (moeRun) out = ((0 + g0*y0) + g1*y1)
// + ... in selection order; mode 1 (moeBatchUnion) out += g*y per expert in
// ascending expert id.
template <int T>
__global__ __launch_bounds__(256) void moe_down_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB;
    extern __shared__ float lds[];
    __shared__ uint32_t s_ids[MAX_K];
    __shared__ float s_gates[MAX_K];
    const int K = p.k, t = blockIdx.y, cols = p.ffn, rows = p.dim;
    const int nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int rpw = p.rpw_dn, TR = WAVES * rpw;
    const int row0 = blockIdx.x * TR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const LaneMap<LPB> m(lane, nb);
    const int j = m.j;
    // virtual rows (slot, row): wave w owns [w*VPW, (w+1)*VPW)
    const int VPW = K * rpw;
    const int nit = (VPW + m.RPI - 1) / m.RPI;
    // LDS: partials [K][TR][nb] f32 | q [K][cols] i8 | d [K][cols/32] f32 | s [K][cols/16] i32
    constexpr int QB = act_block(T);
    const int nd = cols / QB, ns = QB == 256 ? cols / 16 : cols / 32;
    float *part = lds;
    int8_t *qq = (int8_t *)(part + (size_t)K * TR * nb);
    float *qd = (float *)(qq + align16((size_t)K * cols));
    int32_t *qs = (int32_t *)(qd + align16((size_t)K * nd * 4) / 4);
    // 1. the token's ids, gates and quantized vectors (contiguous: pairs t*K..)
    const size_t v0 = (size_t)t * K;
    {
        const int4 *src = (const int4 *)(p.qa.q + v0 * cols);
        for (int i = threadIdx.x; i < K * cols / 16; i += blockDim.x)
            ((int4 *)qq)[i] = src[i];
        for (int i = threadIdx.x; i < K * nd; i += blockDim.x)
            qd[i] = p.qa.d[v0 * nd + i];
        for (int i = threadIdx.x; i < K * ns; i += blockDim.x)
            qs[i] = p.qa.s[v0 * ns + i];
        if ((int)threadIdx.x < K) {
            s_ids[threadIdx.x] = min(p.ids[v0 + threadIdx.x], (uint32_t)(p.n_expert - 1));
            s_gates[threadIdx.x] = p.gates[v0 + threadIdx.x];
        }
    }
    __syncthreads();
    for (int c = 0; c < m.C; c++) {
        bool bok;
        const int b = m.block(c, bok);
        for (int it0 = 0; it0 < nit; it0 += DN_UB) {
            // 2. the weight rows of DN_UB iterations are requested at once
            typename F::W w[DN_UB];
            int slot[DN_UB], rl_[DN_UB];
            bool valid[DN_UB];
#pragma unroll
            for (int u = 0; u < DN_UB; u++) {
                const int vl = (it0 + u) * m.RPI + m.ro;
                const int vr = wave * VPW + vl;
                slot[u] = vr / TR;
                rl_[u] = vr % TR;
                valid[u] = m.active && bok && it0 + u < nit && vl < VPW && row0 + rl_[u] < rows;
                const int sl = valid[u] ? slot[u] : 0;
                const size_t unit = (size_t)(valid[u] ? row0 + rl_[u] : 0) * nb + b;
                w[u] = F::load_w(p.down + (size_t)s_ids[sl] * p.dn_plane, U, unit, j);
            }
            // 3. dots against the slots' quantized vectors in LDS
#pragma unroll
            for (int u = 0; u < DN_UB; u++) {
                if (it0 + u < nit) {
                    const typename F::X x = F::load_x(qq, qd, qs, cols, valid[u] ? slot[u] : 0, b, j);
                    int is, ms;
                    F::dot(w[u], x, j, is, ms);
                    is = group_sum<LPB>(is);
                    ms = group_sum<LPB>(ms);
                    if (valid[u] && j == 0)
                        part[((size_t)slot[u] * TR + rl_[u]) * nb + b] = F::tail(w[u], x, is, ms);
                }
            }
        }
    }
    __syncthreads();
    // 4. every (slot, row) value in parallel (its blocks in order), then the
    // gated combine per row: mode 0 (moeRun) out = ((0 + g0*y0) + g1*y1) + ...
    // in selection order; mode 1 (moeBatchUnion) out += g*y per expert in
    // ascending expert id
    float *yv = part + (size_t)K * TR * nb; // reuses the activation staging
    for (int i = threadIdx.x; i < K * TR; i += blockDim.x)
        yv[i] = row_value<false>(part, 0, i, nb); // i = slot * TR + row
    __syncthreads();
    for (int r = threadIdx.x; r < TR; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= rows)
            continue;
        float *o = p.out + (size_t)t * rows + row;
        if (p.mode == 0) {
            float acc = 0.0f;
            for (int sl = 0; sl < K; sl++) {
                const float pr = s_gates[sl] * yv[sl * TR + r];
                acc = acc + pr;
            }
            *o = acc;
        } else {
            float acc = *o;
            int prev = -1;
            for (int step = 0; step < K; step++) {
                int bs = -1, be = 0x7fffffff;
                for (int sl = 0; sl < K; sl++) {
                    const int e = (int)s_ids[sl];
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
    hipLaunchKernelGGL(moe_gateup_decode_kernel<T>, dim3((p.ffn + TR - 1) / TR, n * p.k), dim3(256),
                       decode_gateup_lds(T, p.dim, p.rpw_gu), st, p);
}

template <int T>
static void launch_down_decode_t(const DecodeParams &p, int n, hipStream_t st) {
    const int TR = WAVES * p.rpw_dn;
    hipLaunchKernelGGL(moe_down_decode_kernel<T>, dim3((p.dim + TR - 1) / TR, n), dim3(256),
                       decode_down_lds(T, p.ffn, p.k, p.rpw_dn), st, p);
}

static bool decode_type(int t) { return t == LH_Q4_K || t == LH_Q6_K || t == LH_Q8_0 || t == LH_Q4_0; }

bool launch_moe_decode(int gate_t, int down_t, const DecodeParams &p, int n, hipStream_t st,
                       int prof_gu, int prof_dn) {
    if (!decode_type(gate_t) || !decode_type(down_t) ||
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
    const int mid = n * p.k * quant_items(down_t, p.ffn) + n;
    hipLaunchKernelGGL(moe_mid_kernel, dim3(mid), dim3(64), 0, st, p, n);
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
