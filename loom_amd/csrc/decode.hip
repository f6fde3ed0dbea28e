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

constexpr int GU_MAXIT = 4; // weight rows per lane requested at once in the gate/up kernel

template <int T>
__global__ __launch_bounds__(256) void moe_gateup_decode_kernel(DecodeParams p) {
    using F = Fmt<T>;
    constexpr int LPB = F::LPB, BPI = 64 / LPB;
    extern __shared__ float lds[];
    __shared__ RouteLds<WAVES> rl;
    __shared__ int s_redo;
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
    const bool exact = route_is_exact(p.gating, p.sel_bias);
    const float *lg = p.logits + (size_t)t * p.n_expert;

    // the first column chunk's activations load while the waves route
    const typename F::X x0 = F::load_x(p.xq, p.xd, p.xs, cols, t, wide ? grp : grp % nb, j);
    route_rank<WAVES, false>(lg, p.sel_bias, p.n_expert, K, p.gating, rl);
    float g = 0.0f;
    for (int pass = 0; pass < 2; pass++) {
        const int e = min(max(rl.id[s], 0), p.n_expert - 1); // never address past the tensor
        const uint8_t *wb = p.gate + (size_t)e * p.gu_plane;
        const uint8_t *wb2 = p.up + (size_t)e * p.gu_plane;
        for (int c = 0; c < C; c++) {
            const int b = wide ? c * BPI + grp : (grp % nb);
            const typename F::X xr = c == 0 ? x0 : F::load_x(p.xq, p.xd, p.xs, cols, t, b, j);
            for (int it0 = 0; it0 < nit; it0 += GU_MAXIT) {
                typename F::W w[GU_MAXIT], w2[GU_MAXIT];
                int rlv[GU_MAXIT];
                bool valid[GU_MAXIT];
#pragma unroll
                for (int u = 0; u < GU_MAXIT; u++) {
                    const int rw = (it0 + u) * RPI + ro;
                    rlv[u] = wave * rpw + rw;
                    const int row = row0 + rlv[u];
                    valid[u] = active && it0 + u < nit && rw < rpw && row < rows;
                    const size_t unit = (size_t)(valid[u] ? row : 0) * nb + b;
                    w[u] = F::load_w(wb, U, unit, j);
                    w2[u] = F::load_w(wb2, U, unit, j);
                }
                if (pass == 0 && c == 0 && it0 == 0 && wave == 0) {
                    // settle the routing (sum, tie check, gates) while the rows load
                    bool redo;
                    g = route_finish<WAVES>(rl, p.n_expert, K, p.gating, exact, p.weights_norm,
                                            p.weights_scale, redo);
                    if (lane == 0)
                        s_redo = redo;
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
        if (pass == 1 || !s_redo)
            break;
        // two experts tied on the final score: route exactly, and redo the
        // tile only if this slot's expert changed
        if (wave == 0) {
            route_exact_wave<WAVES, false>(lg, p.sel_bias, p.n_expert, K, p.gating, rl);
            bool again;
            g = route_finish<WAVES>(rl, p.n_expert, K, p.gating, true, p.weights_norm,
                                    p.weights_scale, again);
        }
        __syncthreads();
        if (min(max(rl.id[s], 0), p.n_expert - 1) == e)
            break;
    }
    if (s == 0 && blockIdx.x == 0 && wave == 0 && lane < K) {
        // one work group per token publishes the routing for the down kernel
        p.ids[(size_t)t * K + lane] = (uint32_t)rl.id[lane];
        p.gates[(size_t)t * K + lane] = g;
    }
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
                // 3. quantize from registers while the weights are in flight,
                // phase by phase over the items so their chains interleave
                float a[DN_QB], dd[DN_QB], inv[DN_QB];
                int sum[DN_QB];
                uint32_t packed[DN_QB];
#pragma unroll
                for (int i = 0; i < DN_QB; i++) {
                    float m = 0.0f;
                    if (__builtin_isfinite(av[i].x)) m = fmaxf(m, fabsf(av[i].x));
                    if (__builtin_isfinite(av[i].y)) m = fmaxf(m, fabsf(av[i].y));
                    if (__builtin_isfinite(av[i].z)) m = fmaxf(m, fabsf(av[i].z));
                    if (__builtin_isfinite(av[i].w)) m = fmaxf(m, fabsf(av[i].w));
                    a[i] = m;
                }
#pragma unroll
                for (int i = 0; i < DN_QB; i++)
                    a[i] = k256 ? wave_max(a[i]) : group8_max(a[i]);
#pragma unroll
                for (int i = 0; i < DN_QB; i++)
                    dd[i] = a[i] / 127.0f;
#pragma unroll
                for (int i = 0; i < DN_QB; i++)
                    inv[i] = (dd[i] != 0.0f && __builtin_isfinite(dd[i])) ? 1.0f / dd[i] : 0.0f;
#pragma unroll
                for (int i = 0; i < DN_QB; i++) {
                    const int q0 = to_i8_sat(av[i].x * inv[i]), q1 = to_i8_sat(av[i].y * inv[i]);
                    const int q2 = to_i8_sat(av[i].z * inv[i]), q3 = to_i8_sat(av[i].w * inv[i]);
                    packed[i] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
                    sum[i] = q0 + q1 + q2 + q3;
                }
#pragma unroll
                for (int i = 0; i < DN_QB; i++)
                    sum[i] = k256 ? group_sum<4>(sum[i]) : group_sum<8>(sum[i]);
#pragma unroll
                for (int i = 0; i < DN_QB; i++) {
                    // items past the end repeat the last one (same values, same place)
                    const int it = min(wave + WAVES * i, items - 1);
                    const int v_ = it / per, item = it % per;
                    const float dv = __builtin_isfinite(dd[i]) ? dd[i] : 0.0f;
                    if constexpr (k256) {
                        *(uint32_t *)(qq + (size_t)v_ * cols + item * 256 + 4 * lane) = packed[i];
                        if ((lane & 3) == 0)
                            qs[(size_t)v_ * (cols / 16) + item * 16 + lane / 4] = sum[i];
                        if (lane == 0)
                            qd[(size_t)v_ * (cols / 256) + item] = dv;
                    } else {
                        const int blk = item * 8 + lane / 8;
                        if (blk < cols / 32) {
                            *(uint32_t *)(qq + (size_t)v_ * cols + blk * 32 + 4 * (lane & 7)) = packed[i];
                            if ((lane & 7) == 0) {
                                qs[(size_t)v_ * (cols / 32) + blk] = sum[i];
                                qd[(size_t)v_ * (cols / 32) + blk] = dv;
                            }
                        }
                    }
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
