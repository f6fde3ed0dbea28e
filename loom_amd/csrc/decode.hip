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

template <int T>
__global__ __launch_bounds__(256) void moe_gateup_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB, BPI = 64 / LPB;
    extern __shared__ float lds[];
    __shared__ RouteLds<WAVES> rl;
    const int K = p.k;
    const int t = blockIdx.y / K, s = blockIdx.y % K;
    const int rows = p.ffn, cols = p.dim, nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int rpw = p.rpw_gu, TR = WAVES * rpw;
    const int row0 = blockIdx.x * TR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / LPB, j = lane % LPB;
    const bool wide = nb >= BPI;
    const int C = wide ? nb / BPI : 1;
    const int RPI = wide ? 1 : BPI / nb;
    const int ro = wide ? 0 : grp / nb;
    const bool active = wide || grp < RPI * nb;
    const int nit = (rpw + RPI - 1) / RPI;
    const size_t lds_mat = (size_t)TR * nb;

    // the first column chunk's activations load while the waves route
    typename F::X xr = F::load_x(p.xq, p.xd, p.xs, cols, t, wide ? grp : grp % nb, j);
    route_select<WAVES, false>(p.logits + (size_t)t * p.n_expert, p.sel_bias, p.n_expert, K,
                               p.gating, rl);
    const int e = min(max(rl.id[s], 0), p.n_expert - 1); // never address past the tensor
    const uint8_t *wb = p.gate + (size_t)e * p.gu_plane;
    const uint8_t *wb2 = p.up + (size_t)e * p.gu_plane;
    for (int c = 0; c < C; c++) {
        const int b = wide ? c * BPI + grp : (grp % nb);
        if (c > 0)
            xr = F::load_x(p.xq, p.xd, p.xs, cols, t, b, j);
#pragma unroll 4
        for (int it = 0; it < nit; it++) {
            const int rw = it * RPI + ro;
            const int rl_ = wave * rpw + rw;
            const int row = row0 + rl_;
            const bool valid = active && rw < rpw && row < rows;
            const size_t unit = (size_t)(valid ? row : 0) * nb + b;
            const typename F::W w = F::load_w(wb, U, unit, j);
            const typename F::W w2 = F::load_w(wb2, U, unit, j);
            int is, ms;
            F::dot(w, xr, j, is, ms);
            is = group_sum<LPB>(is);
            ms = group_sum<LPB>(ms);
            if (valid && j == 0)
                lds[(size_t)rl_ * nb + b] = F::tail(w, xr, is, ms);
            F::dot(w2, xr, j, is, ms);
            is = group_sum<LPB>(is);
            ms = group_sum<LPB>(ms);
            if (valid && j == 0)
                lds[lds_mat + (size_t)rl_ * nb + b] = F::tail(w2, xr, is, ms);
        }
    }
    if (s == 0 && blockIdx.x == 0 && wave == 0) {
        // one work group per token publishes the routing for the down kernel
        const float g = route_gates<WAVES>(rl, K, p.gating, p.weights_norm, p.weights_scale);
        if (lane < K) {
            p.ids[(size_t)t * K + lane] = (uint32_t)rl.id[lane];
            p.gates[(size_t)t * K + lane] = g;
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < TR; r += blockDim.x) {
        const int row = row0 + r;
        if (row < rows)
            p.act[(size_t)blockIdx.y * rows + row] = row_value<true>(lds, lds_mat, r, nb);
    }
}

constexpr int DN_UB = 8; // weight loads in flight per lane in the down kernel
constexpr int DN_QB = 8; // activation items loaded at once per wave

template <int T>
__global__ __launch_bounds__(256) void moe_down_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB, BPI = 64 / LPB;
    extern __shared__ float lds[];
    __shared__ uint32_t s_ids[MAX_K];
    __shared__ float s_gates[MAX_K];
    const int K = p.k, t = blockIdx.y, cols = p.ffn, rows = p.dim;
    const int nb = cols / F::BE;
    const size_t U = (size_t)rows * nb;
    const int rpw = p.rpw_dn, TR = WAVES * rpw;
    const int row0 = blockIdx.x * TR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / LPB, j = lane % LPB;
    const bool wide = nb >= BPI;
    const int C = wide ? nb / BPI : 1;
    const int RPI = wide ? 1 : BPI / nb;
    const int ro = wide ? 0 : grp / nb;
    const bool active = wide || grp < RPI * nb;
    // virtual rows (slot, row): wave w owns [w*VPW, (w+1)*VPW)
    const int VPW = K * rpw;
    const int nit = (VPW + RPI - 1) / RPI;
    // LDS: partials [K][TR][nb] f32 | q [K][cols] i8 | d [K][cols/32] f32 | s [K][cols/16] i32
    float *part = lds;
    int8_t *qq = (int8_t *)(part + (size_t)K * TR * nb);
    float *qd = (float *)(qq + align16((size_t)K * cols));
    int32_t *qs = (int32_t *)(qd + (size_t)K * (cols / 32));
    const QAct qa{qq, qd, qs};

    // 1. ids/gates and the SwiGLU vectors load together
    const int per = quant_items(T, cols);
    const int items = K * per;
    constexpr bool k256 = act_block(T) == 256;
    const bool one_batch = items <= WAVES * DN_QB;
    auto act_src = [&](int it) {
        const int v_ = it / per, item = it % per;
        const float *x = p.act + ((size_t)t * K + v_) * cols;
        return k256 ? x + item * 256 + 4 * lane : blocks32_src(x, cols / 32, item * 8);
    };
    auto quantize = [&](int it, float4 v) {
        const int v_ = it / per, item = it % per;
        if (k256)
            quant256_regs(v, qq + (size_t)v_ * cols + item * 256, qd + (size_t)v_ * (cols / 256) + item,
                          qs + (size_t)v_ * (cols / 16) + item * 16);
        else
            quant32x8_regs(v, cols / 32, item * 8, qq + (size_t)v_ * cols, qd + (size_t)v_ * (cols / 32),
                           qs + (size_t)v_ * (cols / 32));
    };
    float4 av[DN_QB];
    if (one_batch) {
        // items past the end repeat the last item (identical values to the
        // same LDS locations) so the batch is straight-line code
#pragma unroll
        for (int i = 0; i < DN_QB; i++) {
            const int it = wave + WAVES * i;
            av[i] = *(const float4 *)act_src(it < items ? it : items - 1);
        }
    } else {
        // more vectors than one batch of registers: quantize them all up front
        for (int it = wave; it < items; it += WAVES)
            quantize(it, *(const float4 *)act_src(it));
    }
    if (threadIdx.x < K) {
        s_ids[threadIdx.x] = min(p.ids[(size_t)t * K + threadIdx.x], (uint32_t)(p.n_expert - 1));
        s_gates[threadIdx.x] = p.gates[(size_t)t * K + threadIdx.x];
    }
    __syncthreads();

    bool quantized = !one_batch;
    for (int c = 0; c < C; c++) {
        const int b = wide ? c * BPI + grp : (grp % nb);
        for (int it0 = 0; it0 < nit; it0 += DN_UB) {
            // 2. the weight rows of DN_UB iterations are requested at once
            typename F::W w[DN_UB];
            int slot[DN_UB], rl_[DN_UB];
            bool valid[DN_UB];
#pragma unroll
            for (int u = 0; u < DN_UB; u++) {
                const int vl = (it0 + u) * RPI + ro;
                const int vr = wave * VPW + vl;
                slot[u] = vr / TR;
                rl_[u] = vr % TR;
                valid[u] = active && it0 + u < nit && vl < VPW && row0 + rl_[u] < rows;
                const int sl = valid[u] ? slot[u] : 0;
                const size_t unit = (size_t)(valid[u] ? row0 + rl_[u] : 0) * nb + b;
                w[u] = F::load_w(p.down + (size_t)s_ids[sl] * p.dn_plane, U, unit, j);
            }
            if (!quantized) {
                // 3. quantize from registers while the weights are in flight
#pragma unroll
                for (int i = 0; i < DN_QB; i++) {
                    const int it = wave + WAVES * i;
                    quantize(it < items ? it : items - 1, av[i]);
                }
                lds_barrier();
                quantized = true;
            }
            // 4. dots against the slots' quantized vectors in LDS
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
    // 5. gated combine per row
    for (int r = threadIdx.x; r < TR; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= rows)
            continue;
        float *o = p.out + (size_t)t * rows + row;
        if (p.mode == 0) {
            float acc = 0.0f;
            for (int sl = 0; sl < K; sl++) {
                const float pr = s_gates[sl] * row_value<false>(part, 0, (size_t)sl * TR + r, nb);
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
                const float pr = s_gates[bs] * row_value<false>(part, 0, (size_t)bs * TR + r, nb);
                acc = acc + pr;
                prev = be;
            }
            *o = acc;
        }
    }
}

size_t decode_down_lds(int down_t, int ffn, int k, int rpw) {
    const int nb = ffn / block_elems(down_t);
    return (size_t)k * WAVES * rpw * nb * 4 + align16((size_t)k * ffn) + (size_t)k * (ffn / 32) * 4 +
           (size_t)k * (ffn / 16) * 4;
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
