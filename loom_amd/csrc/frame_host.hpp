// frame_host.hpp -- the decode frame's host-side pieces (frame.hip), shared
// by the device entry point (loomhip_token_frame_dev) and the seam's frame
// calls over host buffers (seam_frame.hip): the checks made before anything
// launches, the per-call set-up, one layer, and the output head.
#pragma once

#include "frame.hpp"
#include "runtime.hpp"

namespace lh {

// A call's device workspace (one per call, laid out in g_frame's scratch).
struct FrameWs {
    float *x, *normed, *q, *k, *v, *qrot, *part, *act, *amax_v;
    float *S, *att; // PARITY attention: scores / p [n][n_heads][s_stride], output [n][qd]
    int s_stride;
    uint16_t *qsplit; // the rotated queries as (f16 hi, f16 lo) planes, [2][n][qd]
    int *amax_i;
    QAct qa_dim, qa_att, qa_ffn;
    const DmmvGroup *groups; // lanes in groups of nt against plane 0
    int n_groups, nt;
    size_t bytes;
};

// What one call's layers share.
struct FrameCall {
    FrameDims D;
    FrameWs w;
    size_t n;
    bool parity;
    const float *rope_cs;
    int32_t *pos;     // [n] device
    uint16_t *kc, *vc; // fp16 K/V caches [n][n_layers][ctx][kvd]
    int n_chunks;
    size_t att_lds, att_lds_direct, cmb_lds;
    hipStream_t st;
};

// The model-wide dims and numerics the frame serves (no layer, no head).
int frame_dims_check(const loomhip_model *m, size_t n);
// One layer's types and shapes; ffn_max grows to a dense FFN's width.
int frame_layer_check(const loomhip_model *m, const loomhip_layer &l, size_t li, size_t n, size_t *ffn_max);
// Everything loomhip_token_frame_dev checks: dims, the output head, every layer.
int frame_check(const loomhip_model *m, size_t n, size_t *ffn_max);
// Workspace, dims, LDS limits and the RoPE table for n lanes of model m
// (layers and head already checked); scale is the attention's logit scale.
int frame_setup(const loomhip_model *m, size_t n, size_t ffn_max, float scale, int32_t *pos, uint16_t *kc,
                uint16_t *vc, hipStream_t st, FrameCall &c);
// One layer (llama.zig:1127-1224): attention with the K/V append at pos,
// x += wo . attn, then the FFN and its residual add, on c.w.x.  ids (device,
// [n][n_used]) receives a MoE layer's routed ids, or is NULL.
// next (optional): the rmsnorm the residual row meets after this layer; on
// the batched MoE path the combine forms it and sets *next_done.
// prenormed: the previous layer's combine formed this layer's attention norm.
int frame_layer(const FrameCall &c, const loomhip_layer &l, size_t li, uint32_t *ids, const NextNorm *next = nullptr,
                bool *next_done = nullptr, bool prenormed = false);
// The output norm and head (llama.zig:1225-1227) into logits [n][vocab].
int frame_head(const FrameCall &c, const loomhip_model *m, float *logits, bool prenormed = false);

} // namespace lh
