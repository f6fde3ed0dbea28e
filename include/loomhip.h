/*
 * loomhip.h -- C ABI of libloomhip, the MI355X (gfx950) backend for Loom's
 * quantized MoE forward.
 *
 * Every entry point is plain C: pointers, sizes and ints, no HIP or torch
 * types.  It is what a `-Dgpu=hip` arm of src/compute/backend.zig binds
 * through @cImport (the shim is shown in INTEGRATION.md), and what the Python
 * harness binds through ctypes.
 *
 * Two families:
 *   - seam calls (host slices in, host slices out, synchronous), one per
 *     backend.zig name they replace; they return LOOMHIP_OK when the device
 *     did the work and LOOMHIP_DECLINED / an error otherwise, in which case
 *     the caller runs its own CPU path, exactly as the reference's GPU
 *     backends fall back (src/vulkan/backend.zig:365-378) or decline
 *     (src/compute/backend.zig:75-96);
 *   - device-resident calls (suffix _dev): every tensor pointer is a device
 *     pointer in the device weight layout, work is stream-ordered on the
 *     given stream (NULL = the library's compute stream) and nothing is
 *     copied to or from the host.  These are the hot path.
 *
 * Numerics: LOOMHIP_NUM_CPU_PARITY (default) quantizes activations to int8
 * exactly as the reference CPU path does (src/gguf/ggml.zig:776-800,
 * 1077-1098), runs exact integer block dots and reproduces the f32 tail and
 * the block summation order, so matvec/matmul are bit-identical to the
 * reference's CPU kernels.
 */
#ifndef LOOMHIP_H
#define LOOMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define LOOMHIP_OK 0
#define LOOMHIP_DECLINED 1  /* shape/type not served: caller runs its own path */
#define LOOMHIP_ERR_ARG -1  /* invalid argument (message in loomhip_last_error) */
#define LOOMHIP_ERR_HIP -2  /* HIP runtime error */
#define LOOMHIP_ERR_INIT -3 /* no device / not initialised */

/* GGML type tags (src/gguf/ggml.zig:23-47) */
#define LOOMHIP_F32 0
#define LOOMHIP_F16 1
#define LOOMHIP_Q4_0 2
#define LOOMHIP_Q8_0 8
#define LOOMHIP_Q4_K 12
#define LOOMHIP_Q6_K 14

/* gating (src/gguf/moe.zig:36-44) */
#define LOOMHIP_GATING_SOFTMAX 1
#define LOOMHIP_GATING_SIGMOID 2
#define LOOMHIP_GATING_SOFTMAX_TOPK 3

/* MoE combine order */
#define LOOMHIP_COMBINE_SELECTION 0 /* out = sum over slots in selection order
                                       (llama.zig moeRun 1363-1398) */
#define LOOMHIP_COMBINE_EXPERT_ASC 1 /* out += per expert in ascending id order
                                        (llama.zig moeBatchUnion 1844-1903) */
#define LOOMHIP_COMBINE_SELECTION_ADD 2 /* out = out + (the selection-order sum):
                                           moeLayer then the residual add
                                           (llama.zig:1222) */

/* ---- lifecycle ------------------------------------------------------------ */

/* Replaces backend.parallelBegin's device bring-up (src/vulkan/backend.zig:
 * 185-229): selects the device, creates the compute and expert-copy streams. */
int loomhip_init(int device);
void loomhip_shutdown(void);
/* Diagnostic for the last failed call (backend.arenaError, backend.zig:118). */
const char *loomhip_last_error(void);
/* Launches submitted since the last call, then reset (backend.takeCmdBufCount,
 * src/compute/backend.zig:112-116).  Tests assert it moved to prove the
 * device path ran. */
uint64_t loomhip_take_launch_count(void);
/* Kernel timing with HIP events recorded on the launching stream around
 * every launch of the tagged kernels (the reference's LOOM_VK_KERNEL_PROF
 * timestamps, src/vulkan/device.zig:158-167,245-252).  Enabling resets the
 * totals; launches inside a stream capture are not timed. */
#define LOOMHIP_KT_GATE_UP 0 /* grouped gate/up + SwiGLU expert kernel */
#define LOOMHIP_KT_DOWN 1    /* grouped down expert kernel */
#define LOOMHIP_KT_DENSE 2   /* dense dequant-fused matvec */
#define LOOMHIP_KT_ATTN 3    /* token frame: attention over the K/V cache (partials) */
#define LOOMHIP_KT_HEAD 4    /* token frame: output head matvec */
#define LOOMHIP_KT_QKV 5     /* token frame: q, k, v and wo matvecs */
#define LOOMHIP_KT_COUNT 6
void loomhip_profile_kernels(int enable);
/* Waits for the recorded events; total milliseconds and launch count of tag. */
int loomhip_kernel_time(int tag, double *total_ms, uint64_t *launches);
/* Library version string. */
const char *loomhip_version(void);

/* ---- weight residency ---------------------------------------------------- */

/* Bytes of one [rows][cols] plane of type t in the device layout: Q4_K keeps
 * GGML's 144-byte blocks; Q6_K, Q8_0 and Q4_0 are split per plane into
 * structure-of-arrays (quants, then high bits / scales, then f16 d) so every
 * load is 16-byte aligned.  Same byte count as GGML's, no padding inside a
 * plane. */
size_t loomhip_plane_bytes(int t, size_t rows, size_t cols);
/* GGML bytes of the same plane (src/gguf/ggml.zig:103 rowBytes * rows). */
size_t loomhip_ggml_bytes(int t, size_t rows, size_t cols);

/* Pointer-keyed upload of an immutable host tensor of `planes` stacked
 * [rows][cols] planes (replaces the Vulkan weightBuffer cache,
 * src/vulkan/backend.zig:244-261; a length mismatch on a known pointer
 * re-uploads).  Returns LOOMHIP_OK and the device pointer in *dev_out. */
int loomhip_register_weights(int t, const void *host, size_t rows, size_t cols, size_t planes,
                             void **dev_out);
/* Drop every cached upload (tests recycle host addresses,
 * src/vulkan/backend.zig:159-172). */
void loomhip_clear_weight_cache(void);
/* Bytes currently resident through the cache (backend.materializeArenas). */
size_t loomhip_resident_bytes(void);

/* Convert `planes` GGML planes at src (device memory) into the device layout
 * at dst (device memory, loomhip_plane_bytes * planes). */
int loomhip_repack_dev(int t, void *dst, const void *src, size_t rows, size_t cols, size_t planes,
                       void *stream);
/* Fill `planes` planes in GGML layout (loomhip_ggml_bytes each) with seeded
 * synthetic blocks whose dequantized values have roughly the given standard
 * deviation: the bench's input generator, deterministic in seed.  Feed the
 * bytes to loomhip_repack_dev for the device layout. */
int loomhip_synth_weights_dev(int t, void *dst, size_t rows, size_t cols, size_t planes,
                              uint64_t seed, float stddev, void *stream);

/* ---- seam calls: host in, host out (src/compute/backend.zig:56-63) ------- */

/* backend.matvec (src/gguf/ggml.zig:602): out[rows] = W[rows][cols] . x */
int loomhip_matvec(int t, float *out, const uint8_t *w, const float *x, size_t rows, size_t cols);
/* backend.matmul (src/gguf/ggml.zig:504): out[n][rows], bit-identical to n
 * matvecs. */
int loomhip_matmul(int t, float *out, const uint8_t *w, const float *xs, size_t n, size_t rows,
                   size_t cols);
/* backend.dequantRow (src/gguf/ggml.zig:1739): bit-exact f32 row r. */
int loomhip_dequant_row(int t, float *out, const uint8_t *w, size_t r, size_t cols);
/* backend.moeRoute (src/compute/cpu.zig:86; src/vulkan/backend.zig:437):
 * scores, top-k with lowest-index ties, gates from unbiased scores, renorm
 * with the f16-min clamp, scale. */
int loomhip_moe_route(const float *logits, const float *bias, size_t n_expert, size_t n_used,
                      int gating, int weights_norm, float weights_scale, uint32_t *ids_out,
                      float *gates_out);
/* backend.moeFfnBlockRouted (src/compute/cpu.zig:68; metal 1505; vulkan
 * 455-551) generalised to n_tok tokens: router logits in, the routed experts'
 * gate/up/SwiGLU/down and gated combine out.  gate/up/down are whole 3D
 * tensors in GGML layout ([n_expert][ffn][dim] and [n_expert][dim][ffn]).
 * combine = LOOMHIP_COMBINE_*.  out is [n_tok][dim] (overwritten for
 * SELECTION, accumulated into for EXPERT_ASC). */
int loomhip_moe_ffn_routed(const float *normed, size_t n_tok, size_t dim, const float *logits,
                           const float *sel_bias, size_t n_expert, size_t n_used, int gating,
                           int weights_norm, float weights_scale, int gate_t, const void *gate_w,
                           int up_t, const void *up_w, int down_t, const void *down_w, size_t ffn,
                           int combine, float *out);

/* ---- device-resident hot path ------------------------------------------- */

/* out[n][rows] = W . x_k for n activation vectors x[n][cols] (device f32). */
int loomhip_matvec_dev(int t, float *out, const void *w, const float *x, size_t n, size_t rows,
                       size_t cols, void *stream);
int loomhip_dequant_dev(int t, float *out, const void *w, size_t rows, size_t cols, void *stream);

/* One MoE layer on device for n_tok tokens: router GEMV (f32 [n_expert][dim],
 * plus optional logit bias), route, bucketing, grouped gate/up+SwiGLU, down,
 * combine.  ids_out/gates_out ([n_tok][n_used]) are optional device outputs.
 * Weights are device-layout planes, one per expert, contiguous per tensor. */
typedef struct {
    size_t dim, ffn, n_expert, n_used;
    int gating, weights_norm;
    float weights_scale;
    const float *router;      /* [n_expert][dim] f32 */
    const float *router_bias; /* [n_expert] logit bias or NULL */
    const float *sel_bias;    /* [n_expert] selection-only bias or NULL */
    int gate_t, up_t, down_t;
    const void *gate, *up, *down; /* device-layout, plane per expert */
} loomhip_moe_layer;

int loomhip_moe_layer_dev(const loomhip_moe_layer *L, const float *normed, size_t n_tok,
                          int combine, float *out, uint32_t *ids_out, float *gates_out,
                          void *stream);

/* ---- whole-token decode frame --------------------------------------------- */

/* Numerics of the frame's f32 reductions.  PARITY: every rmsnorm sums its
 * squares in the reference's sequential order (tensor.zig:9-15), so with
 * the matvecs, the attention within 64 positions and the per-head norms
 * already in the reference's order the step is bit-identical to the CPU
 * path wherever exp agrees (a sliver of inputs) -- at ~dim dependent adds per
 * norm.  FAST: rmsnorm sums as a fixed tree (the embedding row's excepted);
 * last-bit differences may then move one int8 step of a quantized matvec
 * input (the 2e-3 logit tolerance). */
#define LOOMHIP_NUMERICS_PARITY 0
#define LOOMHIP_NUMERICS_FAST 1

/* One GQA layer, the LayerSpec of src/compute/cpu.zig:116-138 with device
 * pointers: norms f32, weights in the device layout ([out][in] rows), and
 * either the routed MoE layer (is_moe) or a dense SwiGLU FFN. */
typedef struct {
    const float *attn_norm, *ffn_norm; /* [dim] */
    const float *q_norm, *k_norm;      /* [head_dim] per-head RMSNorm weights, NULL when absent */
    int wq_t, wk_t, wv_t, wo_t;
    const void *wq, *wk, *wv, *wo; /* [n_heads*hd][dim], [kvd][dim] x2, [dim][n_heads*hd] */
    int is_moe;
    loomhip_moe_layer moe;
    int ffn_gate_t, ffn_up_t, ffn_down_t; /* dense FFN (is_moe == 0) */
    const void *ffn_gate, *ffn_up, *ffn_down;
    size_t ffn;
} loomhip_layer;

typedef struct {
    size_t dim, head_dim, n_layers, n_heads, n_kv_heads, vocab, ctx_len, rope_dim;
    float rope_base, eps;
    int rope_neox; /* 1: NEOX (split-half) pairs, 0: NORM (adjacent) pairs */
    int embed_t;
    const void *embed; /* [vocab][dim] device layout */
    const float *out_norm;
    int output_t;
    const void *output;           /* [vocab][dim] device layout */
    const loomhip_layer *layers;  /* host array of n_layers */
    /* RoPE (cos, sin) per (position, pair) [ctx_len][rope_dim/2][2] on the
     * device, as the caller's ropeTheta computes them (llama.zig:821-826), or
     * NULL: the library computes them once on the host with the C library's
     * powf/cosf/sinf in ropeTheta's expressions and keeps them. */
    const float *rope_cs;
    int numerics; /* LOOMHIP_NUMERICS_* */
    /* Optional telemetry: each MoE layer li writes its routed expert ids to
     * ids_out[li][n][n_used] (device), the per-expert access counts of
     * Stats/hottestWithinBudget (src/core/stats.zig:135-160). */
    uint32_t *ids_out;
} loomhip_model;

/* One decode step of n lanes on the device, the whole token as one
 * stream-ordered submission: embedding of tokens[n] (device), every layer
 * (attention against the fp16 K/V caches [n][n_layers][ctx_len][kvd], the
 * new row appended at pos[n] (device)), the output head into logits
 * [n][vocab] (device), then the greedy token into next[n] (device, may be
 * NULL or alias tokens) and pos += 1.  n == 1 follows llama.step (MoE in
 * selection order, then the residual add); n > 1 decodeBatch
 * (moeBatchUnion).  Replaces the frame calls of src/compute/backend.zig:
 * 141-191 (beginFrame, layerBlock x n_layers, endFrame; attnInit/kvAppend/
 * attnHeads for the cache) for a model held on the device.  Capturable in a
 * HIP graph once one eager call has sized the workspace for this n. */
int loomhip_token_frame_dev(const loomhip_model *m, const uint32_t *tokens, int32_t *pos, size_t n,
                            uint16_t *k_cache, uint16_t *v_cache, float *logits, uint32_t *next,
                            void *stream);

#ifdef __cplusplus
}
#endif
#endif
