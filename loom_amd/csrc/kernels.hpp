// kernels.hpp -- launch interfaces shared by the kernel files and the host
// runtime of libloomhip.
#pragma once

#include "common.hpp"

namespace lh {

// Quantized activation vectors (see common.hpp for the layout).
struct QAct {
    int8_t *q;
    float *d;
    int32_t *s;
};

// One work group of the grouped matvec: `n` activation vectors (pairs
// [first, first+n) of the pair table) against weight plane `plane`.
struct DmmvGroup {
    int plane;
    int first;
    int n;
};

struct DmmvParams {
    const uint8_t *w;  // weight planes (device layout)
    const uint8_t *w2; // second matrix sharing the activations (fused up), or null
    size_t plane_bytes;
    int rows, cols;
    const int8_t *xq; // quantized activations
    const float *xd;
    const int32_t *xs;
    const int *pair_src; // activation vector index of each pair
    const int *pair_dst; // output index of each pair
    const DmmvGroup *groups;
    const int *n_groups_dev; // device-side group count, or null
    int n_groups;            // host-side group count (upper bound when n_groups_dev set)
    float *out;              // out[dst * out_stride + row]
    int out_stride;
    int rpw;        // rows per wave
    int accumulate; // 1: out = out + value (a residual add, tensor.zig:50-52)
    int ident_n;    // launch_mmq only: > 0 means ident_n vectors in groups of consecutive
                    // vectors, identity pair maps, plane 0 -- no group or pair table is read
    // the streamed gate/up of launch_mmq (mmqs_kernel) only:
    const int *group_src; // [n_groups][group_stride]: the vector of each group's t-th pair (past n: the
    int group_stride;     // last one's), read in place of pair_src at the group's index; null: pair_src
    int pos_ident;        // pair_dst (and, without group_src, pair_src) is the identity over pair positions
};

// Up to DMMV_MAX_SEG matrices of any supported types against one activation
// set (same cols, groups and pairs) in one launch.  base holds the shared
// fields; rpw and tiles are filled by launch_dmmv_seg.
constexpr int DMMV_MAX_SEG = 3;
struct DmmvSeg {
    const uint8_t *w;
    int t, rows;
    float *out; // out[dst * rows + row]
    int rpw, tiles;
};
struct DmmvSegParams {
    DmmvParams base;
    DmmvSeg seg[DMMV_MAX_SEG];
    int n_seg;
};
bool launch_dmmv_seg(int nt, DmmvSegParams sp, hipStream_t st);
// The same for one vector with the PARITY rmsnorm of x (norm weights norm_w)
// computed by the launch itself; false = not served.
bool launch_norm_seg(DmmvSegParams sp, const float *x, const float *norm_w, float eps, hipStream_t st);

void note_launch();
// Event timing around tagged launches (LOOMHIP_KT_*); -1 when disabled.
int prof_begin(int tag, hipStream_t st);
void prof_end(int handle, hipStream_t st);

void launch_quant_act(int wtype, const float *x, int cols, int x_stride, int nvec, QAct qa,
                      hipStream_t st);
void launch_dequant(int t, const void *w, size_t rows, size_t cols, float *out, hipStream_t st);
void launch_repack(int t, const void *src, void *dst, size_t rows, size_t cols, size_t planes,
                   hipStream_t st);
void launch_repack_strided(int t, const void *src, size_t src_plane, void *dst, size_t rows, size_t cols,
                           size_t planes, hipStream_t st);
void launch_synth(int t, void *dst, size_t rows, size_t cols, size_t planes, uint64_t seed,
                  float stddev, hipStream_t st);

// Grouped int8-activation matvec (bit-identical to the reference CPU kernels).
// nt = max pairs per group (1, 2, 4 or 8); fused = SwiGLU(gate, up) epilogue.
bool dmmv_supported(int t, int cols);
// Returns false (launching nothing) when the partials would not fit in LDS.
bool launch_dmmv(int t, int nt, bool fused, const DmmvParams &p, hipStream_t st);
// Matrix-core variant for Q4_K / Q6_K with groups of up to max_tok (<= 32)
// tokens: the same results bit for bit.  False (nothing launched) when the
// type or the LDS need is not served.
bool mmq_supported(int t, int cols, int max_tok, bool fused);
bool launch_mmq(int t, int max_tok, bool fused, const DmmvParams &p, hipStream_t st);
bool launch_mmq_seg(DmmvSegParams sp, hipStream_t st);
// Rows per wave chosen for a launch of `rows` rows x `groups` groups.
int dmmv_pick_rpw(int t, int cols, int rows, int groups, int nt, bool fused);
size_t dmmv_lds_bytes(int t, int cols, int nt, bool fused, int rpw);
constexpr size_t DMMV_LDS_BUDGET = 48 * 1024;

// f32 GEMV in dotF32 order (src/gguf/ggml.zig:198-217), plus optional bias:
// out[v][r] for n vectors.
void launch_router_gemv(const float *w, const float *bias, const float *x, int n_expert, int dim,
                        int n, float *logits, hipStream_t st);

// Token -> expert bucketing: pairs sorted by (expert, token), groups of at
// most `nt` pairs per expert, pair_of[t][s] = pair index of token t slot s.
struct MoeBuckets {
    int *pair_tok;    // [n*k]
    int *pair_of;     // [n*k]
    int *iota;        // [n*k] identity
    DmmvGroup *groups; // [max_groups]
    int *n_groups;    // [1]; null = route only, no bucketing
    int *group_src;   // [groups made][nt]: each group's pairs' tokens (the last repeated to nt), or null
};
int moe_max_groups(int n, int k, int n_expert, int nt);

// The gate kernel: router GEMV (router != null) or given logits, routing
// (src/gguf/moe.zig:106-158), bucketing, and quantization of x for weight
// type qt (0 = none), in one launch.
struct GateParams {
    const float *router, *router_bias, *sel_bias, *x, *logits_in;
    int n, dim, n_expert, k, gating, weights_norm;
    float weights_scale;
    float *logits;
    uint32_t *ids;
    float *gates;
    int qt;
    QAct qx;
    MoeBuckets b;
    int nt;
    int *sync;
    int chain; // 1: route + bucket after the GEMV (last-arrival chain); 0: GEMV + quantize only
    // decode router only: x is the residual stream and the kernel applies
    // rmsnorm (weights norm_w, tree-summed squares) itself; null: x is normed
    const float *norm_w;
    float norm_eps;
    int norm_exact; // with norm_w, one token: the squares summed in the reference's order
    // set by launch_gate
    int n_chunks, wgs_per_chunk, gemv_wgs, quant_wgs;
};
bool gate_supported(int n, int n_expert, int k);
void launch_gate(GateParams p, hipStream_t st);
// Decode path: router GEMV (router != null) + quantization of x, no routing.
void launch_router_small(GateParams p, hipStream_t st);
// the exact-norm form of the fused-norm router (norm_exact): one token, dim a
// multiple of 32 that fits its LDS row
bool router_exact_supported(int n, int dim);

// Decode path (few tokens): gate/up with an in-kernel routing prologue per
// (token, slot) pair, then down + gated combine per token.  No bucketing and
// no communication between work groups.
struct DecodeParams {
    const float *logits, *sel_bias; // router logits [n][n_expert] (bias included)
    int n_expert, k, gating, weights_norm;
    float weights_scale;
    uint32_t *ids; // [n][k] written by the gate/up kernel
    float *gates;
    const uint8_t *gate, *up, *down; // device-layout planes, one per expert
    size_t gu_plane, dn_plane;
    int dim, ffn, down_t;
    const int8_t *xq; // quantized x [n][dim]
    const float *xd;
    const int32_t *xs;
    float *act; // [n*k][ffn]
    float *out; // [n][dim]
    int mode;   // LOOMHIP_COMBINE_*: 0 selection order, 1 ascending expert (accumulate),
                // 2 selection order added to out
    int rpw_gu, rpw_dn;
};
bool decode_supported(int gate_t, int down_t, int ffn); // ffn a multiple of 256
size_t decode_down_lds(int down_t, int ffn, int k, int rpw);
size_t decode_gateup_lds(int gate_t, int dim, int rpw);
bool launch_moe_decode(int gate_t, int down_t, const DecodeParams &p, int n, hipStream_t st,
                       int prof_gu, int prof_dn);
void launch_combine(const float *y, const float *gates, const uint32_t *ids, const int *pair_of,
                    int n, int k, int dim, int mode, float *out, hipStream_t st);
// The rmsnorm the next consumer of the residual row applies (the next
// layer's attention, or the output head): weights, eps, the activation
// block of the weight it feeds (32 or 256), the int8 target, exact sum.
struct NextNorm {
    const float *w;
    float eps;
    int qb;
    QAct qa;
    bool exact;
};
// The batched combine (ascending expert, mode 1) with the next rmsnorm in the
// same launch; false: not served (a tree-summed norm, dim), the caller
// launches them apart.
bool launch_combine_norm(const float *y, const float *gates, const uint32_t *ids, const int *pair_of, int n,
                         int k, int dim, float *out, const NextNorm &nx, hipStream_t st);

// Sync-buffer size (ints): the gate kernel's completion counters.
constexpr int SYNC_INTS = 1024;

} // namespace lh
