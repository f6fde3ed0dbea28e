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
 *     given stream (NULL = the null stream, as in HIP) and nothing is
 *     copied to or from the host.  These are the hot path.
 *
 * Numerics: every matvec/matmul quantizes activations to int8
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
#define LOOMHIP_KT_GATE_UP 0      /* grouped gate/up + SwiGLU expert kernel */
#define LOOMHIP_KT_DOWN 1         /* grouped down expert kernel */
#define LOOMHIP_KT_DENSE 2        /* dense dequant-fused matvec */
#define LOOMHIP_KT_ATTN 3         /* token frame, FAST: split-context attention partials */
#define LOOMHIP_KT_HEAD 4         /* token frame: output head matvec */
#define LOOMHIP_KT_QKV 5          /* token frame: the q/k/v matvec launch */
#define LOOMHIP_KT_WO 6           /* token frame: the wo matvec (+ residual) */
#define LOOMHIP_KT_ATTN_SCORES 7  /* token frame, PARITY: attention scores */
#define LOOMHIP_KT_ATTN_SOFTMAX 8 /* token frame, PARITY: softmax (max, exp, ordered sum, p) */
#define LOOMHIP_KT_ATTN_PV 9      /* token frame, PARITY: position-ordered P.V */
#define LOOMHIP_KT_MLA_ABSORB 10  /* MLA: qa = W_k^T q_nope */
#define LOOMHIP_KT_MLA_SCORES 11  /* MLA: scores over the compressed cache */
#define LOOMHIP_KT_MLA_SOFTMAX 12 /* MLA: softmax (ordered sum) */
#define LOOMHIP_KT_MLA_WSUM 13    /* MLA: o = sum_t p_t c_t in position order */
#define LOOMHIP_KT_MLA_WV 14      /* MLA: W_v (quantize + grouped matvec) */
#define LOOMHIP_KT_COUNT 15
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
/* Drop every cached upload, moe_ffn_block's HBM tier and the registered
 * arenas (tests recycle host addresses, src/vulkan/backend.zig:159-172). */
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
 * shexp (the seam's `shexp: ?[3]WeightRef` and `shexp_ffn`): the shared
 * expert's three GGML tensors ([shexp_ffn][dim] x2, [dim][shexp_ffn]), or
 * shexp_gate_w NULL; its FFN is added after the routed sum, in the same
 * submission (src/vulkan/backend.zig:527-548).
 * combine = LOOMHIP_COMBINE_*.  out is [n_tok][dim] (overwritten for
 * SELECTION, accumulated into for EXPERT_ASC). */
int loomhip_moe_ffn_routed(const float *normed, size_t n_tok, size_t dim, const float *logits,
                           const float *sel_bias, size_t n_expert, size_t n_used, int gating,
                           int weights_norm, float weights_scale, int gate_t, const void *gate_w,
                           int up_t, const void *up_w, int down_t, const void *down_w,
                           int shexp_gate_t, const void *shexp_gate_w, int shexp_up_t,
                           const void *shexp_up_w, int shexp_down_t, const void *shexp_down_w,
                           size_t ffn, size_t shexp_ffn, int combine, float *out);

/* backend.moeFfnBlock (src/compute/cpu.zig:23-30 ExpertRef / moeFfnBlock;
 * the Metal form src/metal/backend.zig:2322-2410): one MoE layer's selected
 * experts -- the shared one joining as one more ref of weight 1 and its own
 * width (src/gguf/deepseek.zig:1405-1440) -- as host GGML slices of one plane
 * each ([ffn][dim] gate and up, [dim][ffn] down), with their router weights.
 * out[dim] = sum over the refs, in order, of weight * FFN(normed).  Each
 * slice is copied into a slot of a library-held HBM LRU (repacked where the
 * device layout differs): a slice inside a registered arena stays there
 * across calls (keyed by pointer, length, type and shape), any other slice --
 * a Source RAM-cache slot whose bytes change on refill -- is copied on every
 * call.  Slices need only stay valid during the call (the Source's
 * stablePointers).  1..16 refs; DECLINED otherwise or on an unserved type or
 * shape, before anything is recorded. */
typedef struct {
    int gate_t, up_t, down_t;
    const void *gate, *up, *down; /* host GGML bytes */
    float weight;
    size_t ffn;
} loomhip_expert_ref;
int loomhip_moe_ffn_block(const float *normed, size_t dim, const loomhip_expert_ref *experts, size_t n_experts,
                          float *out);
/* Source.prefetchAsync for the HBM tier (src/p2p/expert_fetch.zig:385-400):
 * the refs' arena slices not resident start their copies on the library's
 * copy stream and return at once; the moe_ffn_block call that uses them waits
 * for each fill on the device.  Slices outside the arenas are skipped (their
 * bytes may change before use), as are refs wider than the cache's slots. */
int loomhip_moe_ffn_block_prefetch(size_t dim, const loomhip_expert_ref *experts, size_t n_experts);
/* Hit / miss counters of moe_ffn_block's HBM LRU (tensor slices) and the
 * bytes its misses and prefetches copied in. */
int loomhip_moe_ffn_block_stats(uint64_t *hits, uint64_t *misses, uint64_t *bytes_read);
/* backend.registerArena (src/compute/cpu.zig:33-36; src/metal/backend.zig:
 * 744-760): a read-only host region (the model's mapping) whose bytes stay
 * fixed while registered; moe_ffn_block keeps its slices in HBM across calls.
 * Registering a covered region again is OK; DECLINED past 16 regions. */
int loomhip_register_arena(const void *mem, size_t len);
/* backend.materializeArenas (src/compute/cpu.zig:38-45): the registered
 * arena bytes (page-rounded). */
size_t loomhip_materialize_arenas(void);

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
    /* The shared expert (ffn_{gate,up,down}_shexp, src/gguf/deepseek.zig:
     * 1354-1358): one device-layout plane each, [shexp_ffn][dim] x2 and
     * [dim][shexp_ffn]; always on and unweighted, its FFN added after the
     * routed sum (deepseek.zig:1497-1502).  shexp_gate NULL: none.  Served
     * with the SELECTION and EXPERT_ASC combines. */
    int shexp_gate_t, shexp_up_t, shexp_down_t;
    const void *shexp_gate, *shexp_up, *shexp_down;
    size_t shexp_ffn;
} loomhip_moe_layer;

int loomhip_moe_layer_dev(const loomhip_moe_layer *L, const float *normed, size_t n_tok,
                          int combine, float *out, uint32_t *ids_out, float *gates_out,
                          void *stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  loomhip_moe_layer_dev with its workspace (the quantized
 * activations, routing tables, expert groups and partial outputs) in a fixed
 * per-GPU device array of LOOMHIP_MOE_NOALLOC_BYTES, resolved once per device
 * by loomhip_init; the call itself allocates nothing.  A call whose workspace
 * would exceed the array returns LOOMHIP_ERR_ARG before launching anything
 * (config-3 shapes: up to 128 tokens).  Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (other streams, other host
 * threads) race; nothing in it needs to start at zero.  Same kernels and
 * results as loomhip_moe_layer_dev. */
#define LOOMHIP_MOE_NOALLOC_BYTES ((size_t)16 << 20)
int loomhip_moe_layer_dev_noalloc(const loomhip_moe_layer *L, const float *normed, size_t n_tok,
                                  int combine, float *out, uint32_t *ids_out, float *gates_out,
                                  void *stream);

/* ---- whole-token decode frame --------------------------------------------- */

/* Numerics of the frame's f32 reductions.  PARITY: every reduction in the
 * reference's own order -- rmsnorm's squares and softmax's exponentials
 * summed sequentially (tensor.zig:9-28, evaluated by speculative
 * composition), the scores in dotF32's order, P.V position by position
 * (ggml.zig:221-230) -- so, with the matvecs already exact, the step is
 * bit-identical to the CPU path at any context up to 7936 positions wherever
 * exp agrees (a sliver of inputs).  FAST: rmsnorm sums as a fixed tree (the
 * embedding row's excepted) and split-context attention on the matrix cores;
 * last-bit differences then move int8 steps of quantized matvec inputs, and
 * logits by up to ~2e-2 relative at a 4096-token context. */
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
/* The checks loomhip_token_frame_dev makes before it launches anything, for
 * n lanes: OK when the frame serves the model, DECLINED (or ERR_ARG) with the
 * reason in loomhip_last_error otherwise.  What the HIP arm's
 * gpuLayersSupported (src/gguf/llama.zig:985-1009) asks once at load, since
 * a frame must never decline halfway through a token. */
int loomhip_frame_check(const loomhip_model *m, size_t n);

/* ---- the seam's frame calls over host buffers ------------------------------
 * A model held by the engine (host GGML bytes, mapped from the GGUF file),
 * one sequence.  Weights are uploaded and repacked on first use, keyed by
 * host pointer like every seam call.  The device K/V cache is fp16
 * [n_layers][ctx_len][kvd] (config 4's fp16 cache; the engine's own cache is
 * f32): attention over it is the PARITY frame's, in the reference's order.
 * The engine's host cache stays authoritative -- kvAppend mirrors the rows
 * the host path writes (rounded to fp16, as the frame's own append rounds),
 * and after a frame the rows it wrote are read back with loomhip_read_kv (the
 * fp16 values widened), so a later decline falls back to a cache holding
 * exactly what the device attended over.  Calls are synchronous except
 * inside a begin_frame / end_frame bracket. */

/* A tensor as the engine hands it over (cpu.zig WeightRef: type and the
 * GGML bytes as a slice); a call declines when len is not the size its shape
 * implies. */
typedef struct {
    int type;
    const void *data;
    size_t len;
} loomhip_weight_ref;

/* attnInit (src/compute/backend.zig:121-123; cpu.zig:104-107): allocate the
 * device cache (zeroed).  DECLINED past 7,936 positions (the PARITY
 * attention's limit) or for kvd 0. */
int loomhip_attn_init(size_t layers, size_t ctx_len, size_t kvd);
/* hasKvCache / releaseKvCache (backend.zig:130-133): 1 when a cache exists;
 * free it. */
int loomhip_has_kv_cache(void);
void loomhip_release_kv_cache(void);
/* kvAppend (backend.zig:125-127; cpu.zig:153-156): mirror one host row of
 * layer li at pos (kvd f32 each) into the device cache. */
int loomhip_kv_append(size_t li, size_t pos, const float *k_new, const float *v_new, size_t kvd);
/* The read-back that keeps the host cache authoritative (the GQA form of
 * mlaReadCache, backend.zig:191): the device rows of layer li at pos as f32.
 * After a frame, the rows of its position come from a host mirror copied
 * with the frame's results. */
int loomhip_read_kv(size_t li, size_t pos, float *k_out, float *v_out, size_t kvd);
/* attnHeads (backend.zig:151-160; cpu.zig:157-170): every query head of
 * layer li over cache rows [0, pos] (row pos already appended), q
 * [n_heads*hd] normalised and rotated, out [n_heads*hd]: dotF32 scores
 * times scale, the sequential softmax, P.V in position order
 * (llama.zig:1162-1192), bit-identical to the host loop over the same
 * cache. */
int loomhip_attn_heads(size_t li, size_t pos, const float *q, float *out, size_t n_heads, size_t n_kv_heads,
                       size_t hd, float scale);

/* beginFrame / frameOpen / frameLoadX / layerBlock / endFrame / frameStoreX
 * (backend.zig:141-149; llama.zig:1067-1108 stepRecorded): layers of one
 * token recorded on the library's stream with the residual in device memory,
 * submitted and waited for by end_frame.  LayerSpec is cpu.zig:116-138 (a
 * dense SwiGLU layer, as gpuLayersSupported admits).  layer_block checks
 * and uploads everything before it records anything, and DECLINES (nothing
 * recorded for that layer) for an unserved shape or type, a missing device
 * cache or a position other than the frame's.  Every layer appends its K/V
 * row at pos on the device; loomhip_read_kv returns them. */
typedef struct {
    size_t li, pos;
    const float *attn_norm, *ffn_norm; /* [dim] */
    float eps;
    loomhip_weight_ref wq, wk, wv, wo, gate, up, down;
    size_t dim, ffn, n_heads, n_kv_heads, hd, rope_dim;
    float rope_base;
    int rope_neox;
    float attn_scale;
} loomhip_layer_spec;
int loomhip_begin_frame(void);
int loomhip_frame_open(void); /* 1 while a frame is open */
int loomhip_frame_load_x(const float *x, size_t dim);
int loomhip_layer_block(const loomhip_layer_spec *s);
int loomhip_end_frame(void);
int loomhip_frame_store_x(float *x, size_t dim);

/* The GQA+MoE whole token as one submission, the qwen3moe form of
 * mlaTokenFrame (backend.zig:186-191; cpu.zig:73-79; the Vulkan arm
 * src/vulkan/backend.zig:905-916), one descriptor per layer as MlaLayerDesc:
 * in, the residual stream after embedding (x [dim], host); every layer --
 * attention norm, q/k/v, per-head Q/K norm (q_norm NULL: none), RoPE, the
 * K/V append at pos, attention, wo and residual, then the routed MoE layer
 * (router f32 [n_expert][dim] with an optional logit bias and selection-
 * only bias, gate/up/down stacked [n_expert] planes; a layer with a shared
 * expert, shexp_gate.data set, is DECLINED: the frame adds the routed output
 * to the residual directly) or the dense FFN -- then the output norm and head.
 * Out: x after the last layer and logits [vocab].  PARITY numerics: the
 * engine's own llama.step arithmetic, bit for bit (moeRun's selection
 * order).  DECLINED, with nothing launched, for anything the frame does not
 * serve (loomhip_frame_check's rules), a weight whose length does not match
 * its shape, or a device cache of other dims. */
typedef struct {
    const float *attn_norm, *ffn_norm; /* [dim] */
    const float *q_norm, *k_norm;      /* [head_dim] or NULL */
    loomhip_weight_ref wq, wk, wv, wo;
    int is_moe;
    loomhip_weight_ref router;                     /* f32 [n_expert][dim] */
    const float *router_bias;                      /* [n_expert] logit bias (ffn_gate_inp.bias) or NULL */
    const float *sel_bias;                         /* [n_expert] selection-only bias (exp_probs_b) or NULL */
    loomhip_weight_ref gate, up, down;             /* [n_expert][ffn][dim] x2, [n_expert][dim][ffn] */
    loomhip_weight_ref shexp_gate, shexp_up, shexp_down; /* [shexp_ffn][dim] x2, [dim][shexp_ffn] */
    size_t ffn, shexp_ffn;
    loomhip_weight_ref dgate, dup, ddown; /* dense FFN (is_moe == 0): [dffn][dim] x2, [dim][dffn] */
    size_t dffn;
} loomhip_gqa_layer_desc;
typedef struct {
    size_t dim, n_heads, n_kv_heads, head_dim, rope_dim;
    float eps, scale, rope_base;
    int rope_neox;
    /* RoutedCfg (cpu.zig) */
    size_t n_expert, n_used;
    int gating, weights_norm; /* LOOMHIP_GATING_* */
    float weights_scale;
} loomhip_gqa_frame_cfg;
int loomhip_gqa_token_frame(const loomhip_gqa_layer_desc *descs, size_t n_layers, const loomhip_gqa_frame_cfg *fc,
                            float *x, size_t pos, const float *out_norm, loomhip_weight_ref lm_head, float *logits,
                            size_t vocab);

/* ---- MLA attention over the compressed cache (src/gguf/deepseek.zig) ------
 * The seam's mlaInit / mlaAppend / hasMlaCache / mlaReadCache / mlaSetWk /
 * mlaAttnHeads (src/compute/backend.zig:162-169,193-197; the CPU arm
 * declines, src/compute/cpu.zig:47-96; the Vulkan arm
 * src/vulkan/backend.zig:589-771).  The cache holds, per layer and
 * position, the normalised latent c_kv (kvr floats) and the rotated shared
 * rope key (rope floats), f32 as the engine's own cache
 * (deepseek.zig:523-524).  Attention follows the host head loop
 * (deepseek.zig:988-1047) in its own order: absorb qa = sum_r q_nope[r] W_k[r]
 * (axpy order), s_t = (dotF32(qa, c_t) + dotF32(q_rope, kr_t)) * scale, the
 * exact softmax, o = sum_t p_t c_t (axpy order), out = matvec(W_v, o) -- so
 * o and out are bit-identical to the CPU path.  Slices are (pointer, length)
 * pairs; a length that does not match the cache declines, as the Vulkan arm. */

/* mlaInit: records the cache shape (allocated on first use); DECLINED for a
 * context over 7,936 positions, kvr over 4096 or rope over 512. */
int loomhip_mla_init(size_t layers, size_t ctx_len, size_t kvr, size_t rope);
/* hasMlaCache: 1 when the device cache exists (allocating it), else 0. */
int loomhip_has_mla_cache(void);
/* mlaAppend: one position's rows into layer li of the device cache. */
int loomhip_mla_append(size_t li, size_t pos, const float *c_kv, size_t c_len, const float *k_rope,
                       size_t r_len);
/* mlaReadCache: one position's rows back (after the compute stream drains). */
int loomhip_mla_read_cache(size_t li, size_t pos, float *c_kv, size_t c_len, float *k_rope, size_t r_len);
/* mlaSetWk: layers in order, as the reference requires.  The device keeps no
 * f32 copy: the absorb dequantizes kv_b's W_k rows in the kernel (the same
 * values at 1/7 of the bytes), so this only validates the order. */
int loomhip_mla_set_wk(size_t li, const float *wk_f32, size_t n);
/* mlaAttnHeads: every head's attention at position pos of layer li, W_v
 * applied: out [n_heads][vd].  kv_b is the fused GGML tensor (rows h*(nope+vd)
 * .. +nope: head h's W_k, the next vd rows its W_v; Q4_0/Q8_0/Q4_K/Q6_K),
 * split per head into the device layout on first use and kept, keyed by its
 * host pointer. */
int loomhip_mla_attn_heads(size_t li, size_t pos, const float *q_nope, size_t qn_len, const float *q_rope,
                           size_t qr_len, int kvb_type, const uint8_t *kv_b, size_t kvb_len, float *out,
                           size_t out_len, size_t n_heads, size_t nope, size_t vd, float scale);

/* Device-resident form (no seam counterpart): the same attention over a
 * caller-held cache, stream-ordered.  wk / wv: kv_b split per head into
 * W_k planes [n_heads][nope][kvr] and W_v planes [n_heads][vd][kvr] of the
 * device layout (loomhip_mla_split_kvb_dev). */
typedef struct {
    int kvb_type;
    const void *wk, *wv;
    size_t n_heads, nope, vd, kvr, rope;
    float scale;
} loomhip_mla_attn;
/* kv_b (GGML bytes on the device) into wk (plane_bytes(t, nope, kvr) *
 * n_heads) and wv (plane_bytes(t, vd, kvr) * n_heads). */
int loomhip_mla_split_kvb_dev(int t, const void *kv_b, size_t n_heads, size_t nope, size_t vd, size_t kvr,
                              void *wk, void *wv, void *stream);
/* c_kv [>= seq][kvr], k_rope [>= seq][rope]: one layer's rows; q_nope
 * [n_heads][nope], q_rope [n_heads][rope] (rope applied); out [n_heads][vd];
 * o_lat (nullable) receives o [n_heads][kvr].  Capturable once an eager call
 * has sized the workspace for this seq. */
int loomhip_mla_attn_dev(const loomhip_mla_attn *a, const float *c_kv, const float *k_rope, size_t seq,
                         const float *q_nope, const float *q_rope, float *out, float *o_lat, void *stream);

/* mlaLayerTail (src/compute/cpu.zig:63; Vulkan src/vulkan/backend.zig:773):
 * the rest of an MLA layer after its attention head, one submission: the
 * attention above (cache layer li, position pos), x = x + attn_output . heads,
 * normed = rmsnorm(x) * ffn_norm (the squares summed in order), the routed
 * MoE from router logits router . normed (f32 router; router_bias is the
 * selection-only bias, exp_probs_b) in selection order plus the shared
 * expert (shexp_gate NULL: none), x = x + that sum -- the engine's own
 * sequence (deepseek.zig:1044-1046, 1325-1387), bit-identical to it.  x [dim]
 * is read and written.  gating/weights_norm/weights_scale: RoutedCfg. */
int loomhip_mla_layer_tail(size_t li, size_t pos, float *x, size_t dim, const float *q_nope, size_t qn_len,
                           const float *q_rope, size_t qr_len, int kvb_type, const uint8_t *kv_b, size_t kvb_len,
                           int attn_out_type, const uint8_t *attn_out, const float *ffn_norm, float eps,
                           int router_type, const uint8_t *router, const float *router_bias, int gate_type,
                           const uint8_t *gate, int up_type, const uint8_t *up, int down_type, const uint8_t *down,
                           int shexp_gate_type, const uint8_t *shexp_gate, int shexp_up_type,
                           const uint8_t *shexp_up, int shexp_down_type, const uint8_t *shexp_down, size_t ffn,
                           size_t shexp_ffn, size_t n_expert, size_t n_used, int gating, int weights_norm,
                           float weights_scale, size_t n_heads, size_t nope, size_t vd, float scale);
/* Device-resident form (no seam counterpart): the same tail over a
 * caller-held cache and device weights (attn_out [dim][n_heads * vd] device
 * layout, ffn_norm [dim] f32, moe the layer's device MoE -- for a DeepSeek
 * layer its sel_bias is exp_probs_b), x [dim] in place, stream-ordered. */
int loomhip_mla_layer_tail_dev(const loomhip_mla_attn *a, const float *c_kv, const float *k_rope, size_t seq,
                               const float *q_nope, const float *q_rope, int attn_out_type, const void *attn_out,
                               const float *ffn_norm, float eps, const loomhip_moe_layer *moe, float *x,
                               void *stream);

/* mlaTokenFrame (src/compute/backend.zig:186-191; cpu.zig:73-79; the Vulkan
 * arm src/vulkan/backend.zig:905-1000): the whole MLA token as one
 * submission over the device cache of mlaInit, one MlaLayerDesc per layer.
 * In: the residual stream after embedding (x [dim], host).  Per layer, the
 * engine's own sequence (deepseek.zig:851-1048 attnLayer, 1275-1440 step):
 * normed = rmsnorm(x) * attn_norm; q = wq . normed (the direct-q path);
 * kv_a = kv_a_mqa . normed; the cache row c_kv = rmsnorm(kv_a[0, kvr)) *
 * kv_a_norm and k_rope = rope(kv_a[kvr, kvr + rope), pos); q's rope slice of
 * every head rotated; the attention (loomhip_mla_attn_dev's order);
 * x += attn_output . heads; normed = rmsnorm(x) * ffn_norm; then the routed
 * MoE (f32 router, RoutedCfg; moeRun's selection order; the shared expert
 * when shexp_gate.data is set) or the dense SwiGLU FFN, and x += that.  Then
 * logits = lm_head . (rmsnorm(x) * out_norm).  Out: x after the last layer
 * and logits [vocab]; the cache holds this position's rows (mlaReadCache).
 * rope is deepseek.zig:581-629's ropeApply: NORM pairs, with YaRN when
 * yarn_factor > 1, its cos/sin computed on the host with the C library's
 * logf/powf/cosf/sinf in ropeApply's expressions.  Bit-identical to the
 * engine's host path on the oracle.  DECLINED, with nothing launched, for a
 * shape or type the kernels do not serve, a weight whose length does not
 * match its shape, or more layers / another position than the cache has. */
typedef struct {
    const float *attn_norm;                 /* [dim] */
    loomhip_weight_ref wq;                  /* [n_heads * (nope + rope)][dim] */
    loomhip_weight_ref kv_a;                /* [kvr + rope][dim] */
    const float *kv_a_norm;                 /* [kvr] */
    loomhip_weight_ref kv_b;                /* [n_heads * (nope + v_head_dim)][kvr] */
    loomhip_weight_ref attn_out;            /* [dim][n_heads * v_head_dim] */
    const float *ffn_norm;                  /* [dim] */
    int is_moe;
    loomhip_weight_ref router, gate, up, down; /* f32 [n_expert][dim]; [n_expert] planes */
    loomhip_weight_ref shexp_gate, shexp_up, shexp_down;
    size_t ffn, shexp_ffn;
    loomhip_weight_ref dgate, dup, ddown; /* dense FFN (is_moe == 0) */
    size_t dffn;
} loomhip_mla_layer_desc;
typedef struct {
    size_t dim, n_heads, nope, rope, kvr, v_head_dim;
    float eps, scale, rope_base, yarn_factor, yarn_orig_ctx;
    /* RoutedCfg (cpu.zig) */
    size_t n_expert, n_used;
    int gating, weights_norm; /* LOOMHIP_GATING_* */
    float weights_scale;
} loomhip_mla_frame_cfg;
int loomhip_mla_token_frame(const loomhip_mla_layer_desc *descs, size_t n_layers, const loomhip_mla_frame_cfg *fc,
                            float *x, size_t pos, const float *out_norm, loomhip_weight_ref lm_head, float *logits,
                            size_t vocab);

/* ---- GGUF v3 files (src/gguf/gguf.zig) ------------------------------------
 * gguf.zig:251-332 parse: the header, the metadata key/values and the tensor
 * table, with the whole file mapped read-only so a tensor's bytes are a
 * pointer into it (the data section starts at the first general.alignment
 * boundary after the table; tensor offsets are relative to it).  Malformed
 * files return LOOMHIP_ERR_ARG with the reference's error name first in
 * loomhip_last_error (NotGguf, UnsupportedGgufVersion, TruncatedGguf,
 * UnknownValueType, ArrayNestingTooDeep, BadTensorDims, BadAlignment). */
typedef struct loomhip_gguf loomhip_gguf;
int loomhip_gguf_open(const char *path, loomhip_gguf **out);
void loomhip_gguf_close(loomhip_gguf *g);
typedef struct {
    uint32_t version;
    uint64_t alignment, n_tensors, n_kv, data_offset, file_size;
    const uint8_t *base; /* the mapped file */
} loomhip_gguf_info;
int loomhip_gguf_get_info(const loomhip_gguf *g, loomhip_gguf_info *info);
/* Tensor i (gguf.zig:36-47 TensorInfo): dims[0] is the row length (unused
 * dims read 1); nbytes is its GGML size for F32/F16/Q4_0/Q8_0/Q4_K/Q6_K (0
 * for other types and for a size that overflows 64 bits, every product
 * checked as ggml.zig:143-153 tensorBytesChecked does), data its bytes in
 * the mapping (NULL when unknown or outside the file, the offset sum
 * checked too). */
typedef struct {
    const char *name;
    uint32_t n_dims;
    uint64_t dims[8];
    uint32_t ggml_type;
    uint64_t offset, nbytes;
    const void *data;
} loomhip_gguf_tensor;
int loomhip_gguf_get_tensor(const loomhip_gguf *g, size_t i, loomhip_gguf_tensor *t);
/* Parsed.findTensor (gguf.zig:139-144); DECLINED when absent. */
int loomhip_gguf_find_tensor(const loomhip_gguf *g, const char *name, size_t *index);
/* Key/value i (gguf.zig:49-71 MetaValue / MetaKV): kind 0 int (i), 1 uint
 * (u), 2 float (f), 3 bool (u), 4 string (s, s_len), 5 string array (strs,
 * count), 6 f32 array (f32s), 7 i32 array (i32s), 8 array of another element
 * type (elem_type, count; contents skipped); type is the file's value type;
 * [span_start, span_end) the pair's bytes in the file. */
typedef struct {
    const char *key;
    uint32_t type;
    int kind;
    int64_t i;
    uint64_t u;
    double f;
    const char *s;
    size_t s_len;
    uint32_t elem_type;
    uint64_t count;
    const char *const *strs;
    const float *f32s;
    const int32_t *i32s;
    uint64_t span_start, span_end;
} loomhip_gguf_kv;
int loomhip_gguf_get_kv(const loomhip_gguf *g, size_t i, loomhip_gguf_kv *kv);
/* Parsed.getUint / getFloat / getString / getBool (gguf.zig:97-137), with
 * the same coercions; DECLINED when the key is absent or of another kind. */
int loomhip_gguf_get_uint(const loomhip_gguf *g, const char *key, uint64_t *v);
int loomhip_gguf_get_float(const loomhip_gguf *g, const char *key, double *v);
int loomhip_gguf_get_string(const loomhip_gguf *g, const char *key, const char **s, size_t *len);
int loomhip_gguf_get_bool(const loomhip_gguf *g, const char *key, int *v);

/* A GGUF v3 writer laid out as the reference's fixture writers lay theirs
 * out (gguf.zig:643-912): key/values in call order, then tensor infos in call
 * order with offsets aligned to `alignment`, zero padding to the data
 * section and between tensors.  writer_kv: a GGUF value type (0-12) with
 * its scalar bytes at value, a string value[0..len), or an array of
 * elem_type with len elements at value (strings: len NUL-terminated const
 * char * pointers).  writer_tensor copies the bytes (checked against the
 * shape for known types).  finish writes the file and frees the writer;
 * abort only frees it. */
typedef struct loomhip_gguf_writer loomhip_gguf_writer;
int loomhip_gguf_writer_begin(uint64_t alignment, loomhip_gguf_writer **out);
int loomhip_gguf_writer_kv(loomhip_gguf_writer *w, const char *key, uint32_t type, const void *value,
                           uint64_t len, uint32_t elem_type);
int loomhip_gguf_writer_tensor(loomhip_gguf_writer *w, const char *name, uint32_t n_dims, const uint64_t *dims,
                               uint32_t ggml_type, const void *data, uint64_t nbytes);
int loomhip_gguf_writer_finish(loomhip_gguf_writer *w, const char *path);
void loomhip_gguf_writer_abort(loomhip_gguf_writer *w);

/* ---- expert cache: pinned host memory -> HBM LRU ----------------------------
 * The tiers of ExpertCache (src/engine/expert_cache.zig:150-249) with HBM as
 * the cache and pinned host memory as the backing store that readBlock
 * (197-215) reads: a pinned hot set held in HBM for good (pin, 217-227), an
 * LRU of `capacity` HBM slots (Lru, 39-148: touch-to-front on a hit, fill
 * never-used slots before evicting the tail, abort on a failed fill), and
 * the host copy.  A miss copies the block host -> HBM on the library's copy
 * stream; the caller's stream waits for that copy and nothing else, and a
 * refill of an evicted slot waits for the work that last used the slot.
 * Single-threaded, like the reference's generation thread. */
typedef struct loomhip_ec loomhip_ec;

/* Stats (expert_cache.zig:18-36): misses = disk_misses, bytes_read their
 * bytes; warm-up reads (pin, prefetch) are counted apart. */
typedef struct {
    uint64_t pin_hits, lru_hits, misses, bytes_read, warmup_reads, warmup_bytes;
} loomhip_ec_stats;

/* Pinned (page-locked) host memory for the backing store: the copy source
 * must be pinned for the copies to run asynchronously. */
void *loomhip_host_alloc(size_t bytes);
void loomhip_host_free(void *p);

/* ExpertCache.init (expert_cache.zig:160-185): `capacity` LRU slots and
 * `pin_slots` pinned ones of `slot_bytes` each in HBM, expert ids
 * [0, n_ids). */
int loomhip_ec_create(size_t capacity, size_t pin_slots, size_t slot_bytes, size_t n_ids,
                      loomhip_ec **out);
void loomhip_ec_destroy(loomhip_ec *ec);
/* The backing block of expert `id` (the manifest entry readBlock reads,
 * expert_cache.zig:197-200): len <= slot_bytes bytes of host memory, which
 * the caller keeps alive and unchanged while the cache exists. */
int loomhip_ec_set_source(loomhip_ec *ec, size_t id, const void *host, size_t len);
/* ExpertCache.pin (217-227): load `ids` into the pinned HBM set; idempotent
 * per id; warm-up reads.  Returns when the copies are done. */
int loomhip_ec_pin(loomhip_ec *ec, const uint32_t *ids, size_t n);
/* ExpertCache.get (230-249): the HBM address of expert `id`'s block, valid
 * for work enqueued on `stream` until a later get or prefetch evicts it.
 * access_count[id] += 1; pinned hit, LRU hit, or miss (reserve a slot,
 * async copy, `stream` waits for it).  A missing source aborts the reserve
 * (Lru.abort, 138-147) and fails. */
int loomhip_ec_get(loomhip_ec *ec, size_t id, void *stream, void **dev_out);
/* Record that the blocks handed out since the last release are used by work
 * already enqueued on `stream`: a later refill of their slots waits for that
 * work only (without it, a refill waits for all work enqueued on the stream
 * by the time of the eviction). */
int loomhip_ec_release(loomhip_ec *ec, void *stream);
/* Warm the LRU with `ids` ahead of their gets: absent ids are reserved (MRU)
 * and copied asynchronously (warm-up reads); present ones are left as they
 * are.  Not in the reference's cache: the GPU tier's copy/compute overlap. */
int loomhip_ec_prefetch(loomhip_ec *ec, const uint32_t *ids, size_t n);
int loomhip_ec_get_stats(const loomhip_ec *ec, loomhip_ec_stats *out);
/* access_count[0..n) (the STATS input of hottestWithinBudget, stats.zig:
 * 135-160). */
int loomhip_ec_access_counts(const loomhip_ec *ec, uint64_t *out, size_t n);
/* Lru.clear (128-133): drop every LRU entry (pinned set and stats kept). */
int loomhip_ec_clear(loomhip_ec *ec);

/* A routed MoE layer whose experts live in the cache: expert e's block is
 * cache id id_base + e (checkpoint.expertId, src/engine/checkpoint.zig:
 * 162-164) holding gate [ffn][dim] and up [ffn][dim] of type gate_t and down
 * [dim][ffn] of type down_t (device layout) at the given byte offsets. */
typedef struct {
    size_t dim, ffn, n_expert, n_used;
    int gating, weights_norm;
    float weights_scale;
    const float *router;      /* [n_expert][dim] f32, device */
    const float *router_bias; /* [n_expert] logit bias or NULL */
    const float *sel_bias;    /* [n_expert] selection-only bias or NULL */
    int gate_t, down_t;
    size_t id_base;
    size_t gate_off, up_off, down_off;
    /* the shared expert, resident in HBM (device layout), as in
     * loomhip_moe_layer; shexp_gate NULL: none */
    int shexp_gate_t, shexp_up_t, shexp_down_t;
    const void *shexp_gate, *shexp_up, *shexp_down;
    size_t shexp_ffn;
} loomhip_moe_layer_ec;

/* moe.moeFFN's routed part (src/engine/moe.zig:97-124) on the device with
 * the cache: router, route (device), the ids to the host, then one get per
 * routed expert and the experts' SwiGLU FFNs, out[t] = sum g * FFN_e(x_t)
 * from +0.  n_tok == 1: the selection order of moeFFN (one get per slot);
 * n_tok > 1: each distinct expert once per call in ascending order, its
 * tokens batched (moeBatchUnion, llama.zig:1828-1924).  More distinct
 * experts than capacity run in rounds of at most `capacity` gets.  out is
 * [n_tok][dim] (device, overwritten; undefined after a failed call);
 * ids_out/gates_out ([n_tok][n_used], host) are optional.  Synchronises
 * `stream` once per call (the ids). */
int loomhip_moe_layer_cached(const loomhip_moe_layer_ec *L, loomhip_ec *ec, const float *normed,
                             size_t n_tok, float *out, uint32_t *ids_out, float *gates_out,
                             void *stream);

/* Config 5's block with its routed experts streamed: deepseek.step's MLA
 * layer with an expert Source behind it (src/gguf/deepseek.zig:1275-1440;
 * the experts' bytes through the HBM LRU of src/engine/expert_cache.zig).
 * For n sequences at one position each: the MLA attention of sequence i over
 * its own cache rows (c_kv[i], k_rope[i]: host arrays of n device pointers,
 * seq positions each), x_i += attn_output . heads_i, normed_i = rmsnorm(x_i)
 * * ffn_norm (the squares summed in order), acc = the routed experts read
 * through the cache plus the resident shared expert (loomhip_moe_layer_
 * cached: moeRun's selection order at one sequence, moeBatchUnion's
 * ascending order for more), x_i += acc_i.  x [n][dim], q_nope [n][n_heads *
 * nope], q_rope [n][n_heads * rope] (device); ids_out (host, [n][n_used],
 * optional) receives the routed ids.  Synchronises the stream once per call
 * (the routed ids, as the cached layer does). */
int loomhip_mla_layer_cached_dev(const loomhip_mla_attn *a, const float *const *c_kv, const float *const *k_rope,
                                 size_t seq, size_t n, const float *q_nope, const float *q_rope, int attn_out_type,
                                 const void *attn_out, const float *ffn_norm, float eps,
                                 const loomhip_moe_layer_ec *moe, loomhip_ec *ec, float *x, uint32_t *ids_out,
                                 void *stream);

#ifdef __cplusplus
}
#endif
#endif
