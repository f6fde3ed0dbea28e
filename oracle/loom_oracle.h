/*
 * loom_oracle.h -- CPU restatement of Loom's CPU SIMD path for the quantized
 * MoE forward (the correctness oracle and the timed CPU baseline).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library (loom_amd/) links,
 * loads or calls this code.  It is used by tests/ (as the checker),
 * __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg
 * (as the thing timed for the CPU column).  The reference is Zig 0.16, which
 * cannot be built in this environment, so every function below restates the
 * reference's algorithm and f32 evaluation order in C; each definition cites
 * the reference file:line it follows.  Build with -ffp-contract=off and no
 * fast-math so no multiply-add is contracted and no float sum is reordered.
 */
#ifndef LOOM_ORACLE_H
#define LOOM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml.zig:23-47 -- GGML type tags (the subset this path covers). */
enum {
    LO_F32 = 0,
    LO_F16 = 1,
    LO_Q4_0 = 2,
    LO_Q8_0 = 8,
    LO_Q4_K = 12,
    LO_Q6_K = 14,
};

#define LO_QK_0 32
#define LO_QK_K 256
#define LO_MAX_BATCH 8 /* ggml.zig:417 */

/* ---- formats (ggml.zig:86-153) ------------------------------------------ */
size_t lo_block_elems(int t);
size_t lo_block_bytes(int t);
size_t lo_row_bytes(int t, size_t n);
float lo_f16_to_f32(uint16_t h);
uint16_t lo_f32_to_f16(float f);

/* ---- exact dequant (ggml.zig:1739-1857) --------------------------------- */
void lo_dequant_row(int t, float *out, const uint8_t *data, size_t r, size_t cols);

/* ---- int8 activation quantizers (ggml.zig:738-800, 1067-1098) ----------- */
typedef struct {
    float d;
    int32_t sum;
    int8_t q[LO_QK_0];
} lo_xblock; /* ggml.zig:738 XBlock */

typedef struct {
    float d;
    int8_t q[LO_QK_K];
    int32_t bsum[LO_QK_K / 16];
} lo_xblockk; /* ggml.zig:762 XBlockK */

int8_t lo_to_i8_saturating(float v);
void lo_quantize_x(const float *x, size_t n, lo_xblock *out);
void lo_quantize_x256(const float *x, size_t n, lo_xblockk *out);

/* ---- matrix ops (ggml.zig:198-217, 504-639, 1024-1059, 1196-1294) -------- */
float lo_dot_f32(const float *a, const float *b, size_t n);
void lo_axpy(float *out, const float *v, float w, size_t n);
void lo_matvec(int t, float *out, const uint8_t *w, const float *x, size_t rows, size_t cols);
void lo_matmul(int t, float *out, const uint8_t *w, const float *xs, size_t n, size_t rows,
               size_t cols);
/* Worker pool (ggml.zig:279-399): n = total threads including the caller. */
void lo_parallel_begin(int n);
void lo_parallel_end(void);
int lo_parallel_threads(void);

/* ---- input generators ---------------------------------------------------- */
/* ggml.zig:1861-1904 test quantizers, restated. */
void lo_quantize_q4_0(uint8_t *dst, const float *src, size_t n);
void lo_quantize_q8_0(uint8_t *dst, const float *src, size_t n);
/* GGML's published reference quantizers (quantize_row_q4_K_ref /
 * quantize_row_q6_K_ref); the reference has no Q4_K/Q6_K quantizer. */
void lo_quantize_q4_k(uint8_t *dst, const float *src, size_t n);
void lo_quantize_q6_k(uint8_t *dst, const float *src, size_t n);
/* Row-wise quantize of a [rows][cols] f32 matrix into format t. */
void lo_quantize_rows(int t, uint8_t *dst, const float *src, size_t rows, size_t cols);
/* Seeded generators: splitmix64 stream, Box-Muller normals. */
void lo_fill_normal(float *dst, size_t n, uint64_t seed, float mean, float stddev);
void lo_fill_uniform(float *dst, size_t n, uint64_t seed, float lo, float hi);

/* ---- elementwise (core/tensor.zig:9-57, llama.zig:821-949) -------------- */
void lo_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
void lo_softmax(float *x, size_t n);
float lo_silu(float x);
float lo_sigmoid(float x);
void lo_swiglu(float *out, const float *g, const float *u, size_t n);
void lo_add(float *dst, const float *src, size_t n);
void lo_rope_norm(float *vec, size_t rope_dim, size_t pos, float base);
void lo_rope_neox(float *vec, size_t rope_dim, size_t pos, float base);
void lo_head_norm(float *vec, const float *w, size_t n_heads, size_t hd, float eps);
size_t lo_argmax(const float *logits, size_t n);

/* ---- routing (gguf/moe.zig:53-158) --------------------------------------- */
enum { LO_GATING_SOFTMAX = 1, LO_GATING_SIGMOID = 2, LO_GATING_SOFTMAX_TOPK = 3 };
typedef struct {
    size_t n_expert;
    size_t n_used;
    int gating;
    int weights_norm;
    float weights_scale;
} lo_route_cfg;

void lo_route(const lo_route_cfg *cfg, const float *logits, const float *bias, uint32_t *ids,
              float *gates);

/* ---- tensors and the MoE layer (llama.zig:127-142, 952-958, 1262-1419,
 *      1828-1924) -------------------------------------------------------- */
typedef struct {
    int ty;
    const uint8_t *data;
    size_t ne0; /* row length (input dim) */
    size_t ne1; /* rows (output dim) */
    size_t ne2; /* experts for the stacked 3D tensors, else 1 */
} lo_tensor;

typedef struct {
    size_t dim;
    size_t ffn; /* per-expert intermediate */
    lo_route_cfg route;
    lo_tensor router;         /* f32 [n_expert][dim] (ffn_gate_inp) */
    const float *router_bias; /* ffn_gate_inp.bias (logit bias), nullable */
    const float *sel_bias;    /* exp_probs_b (selection-only), nullable */
    lo_tensor gate_exps, up_exps, down_exps;
    /* the shared expert (ffn_{gate,up,down}_shexp), data NULL when absent:
     * always on, unweighted, added after the routed sum (deepseek.zig:
     * 1497-1502) */
    lo_tensor shexp_gate, shexp_up, shexp_down;
} lo_moe_layer;

/* llama.moeLayer + moeRun at one token: acc = sum_sel gate * ffn(x), in
 * selection order.  ids/gates (n_used) receive the routing when non-null. */
void lo_moe_layer_token(const lo_moe_layer *L, const float *normed, float *acc, uint32_t *ids,
                        float *gates);
/* llama.moeBatchUnion: bx[k] += sum_e gate * ffn_e(bnormed[k]) with experts
 * visited in ascending id order; ids/gates are [n][n_used] when non-null. */
void lo_moe_batch_union(const lo_moe_layer *L, const float *bnormed, float *bx, size_t n,
                        uint32_t *ids, float *gates);

/* backend.moeFfnBlock (compute/cpu.zig:23-30, metal/backend.zig:2322-2410):
 * out = sum over the refs, in order, of weight * denseFFN_ref(normed) (the
 * reference's host loop acc += gate * ffn_out, deepseek.zig:1485-1487; the
 * shared expert joins as one more ref of weight 1). */
typedef struct {
    lo_tensor gate, up, down; /* one plane each: [ffn][dim], [ffn][dim], [dim][ffn] */
    float weight;
} lo_expert_ref;
void lo_moe_ffn_block(const float *normed, size_t dim, const lo_expert_ref *refs, size_t n, float *out);

/* ---- whole-model decode (llama.zig:1111-1227, 1939-2043) ----------------- */
typedef struct {
    const float *attn_norm;
    lo_tensor wq, wk, wv, wo;
    const float *q_norm; /* nullable (qwen3moe per-head norm) */
    const float *k_norm;
    const float *ffn_norm;
    int is_moe;
    lo_tensor ffn_gate, ffn_up, ffn_down; /* dense FFN */
    lo_moe_layer moe;
} lo_layer;

typedef struct {
    size_t dim, head_dim, n_layers, n_heads, n_kv_heads, vocab, ctx_len, rope_dim;
    float rope_base, eps;
    int rope_neox;
    int kv_f16; /* store K/V as fp16 and widen for the dot (config-4 deviation) */
    lo_tensor embed;
    const float *out_norm;
    lo_tensor output;
    const lo_layer *layers;
} lo_model;

typedef struct {
    void *k_cache; /* [n_layers][ctx][kv_dim] f32 or f16 */
    void *v_cache;
    size_t pos;
} lo_seq;

size_t lo_seq_cache_bytes(const lo_model *m);
/* One token at batch 1 (llama.step): logits[vocab]. Advances seq->pos. */
int lo_step(const lo_model *m, lo_seq *seq, uint32_t token, float *logits);
/* Continuous batching (llama.decodeBatch): n lanes, out [n][vocab]. */
int lo_decode_batch(const lo_model *m, lo_seq *seqs, const uint32_t *tokens, size_t n, float *out);
/* backend.attnHeads (llama.zig:1162-1192): every query head over cache rows
 * [0, pos] of layer li (a lo_seq cache layout), into attn_out [n_heads][hd]. */
void lo_attn_heads(const lo_model *m, const void *k_cache, const void *v_cache, size_t li, size_t pos,
                   const float *q, float *attn_out, float scale);
/* Test-only planted mistakes in lo_decode_batch (0 = none): 1 cross-lane cache
 * read, 2 K/V row written at the batch index, 3 rope at lane 0's position. */
void lo_set_batch_slip(int slip);

/* ---- expert cache bookkeeping (engine/expert_cache.zig:18-148,
 *      core/stats.zig:135-160) ------------------------------------------- */
typedef struct lo_lru lo_lru;
lo_lru *lo_lru_create(size_t capacity);
void lo_lru_destroy(lo_lru *l);
/* Returns the slot holding id and marks it MRU, or -1. */
long lo_lru_find(lo_lru *l, size_t id);
/* Reserve a slot for id (fill free slots first, else evict the tail).
 * *evicted receives the evicted id or SIZE_MAX.  Returns the slot. */
long lo_lru_reserve(lo_lru *l, size_t id, size_t *evicted);
void lo_lru_abort(lo_lru *l, size_t id);
void lo_lru_clear(lo_lru *l);
/* Replay an access trace through pinned set + LRU (ExpertCache.get order):
 * counts[0]=pin_hits, [1]=lru_hits, [2]=misses.  hit_mask[i] = 0 miss,
 * 1 pinned hit, 2 lru hit. */
void lo_cache_replay(size_t capacity, const uint8_t *pinned, size_t n_ids, const uint32_t *trace,
                     size_t n_trace, uint64_t *counts, uint8_t *hit_mask);
size_t lo_hottest_within_budget(const uint64_t *access_count, size_t n, size_t expert_bytes,
                                uint64_t budget, size_t *out_ids);

/* ---- MLA attention over the compressed cache (gguf/deepseek.zig) ------- */
/* deepseek.zig:581-629 ropeApply: NORM pairs, YaRN when factor > 1. */
void lo_rope_yarn(float *vec, size_t n, size_t pos, float base, float factor, float orig_ctx);
/* deepseek.zig:988-1047 host head loop (fused kv_b): absorb, scores,
 * softmax, weighted sum of c_t, W_v.  out [n_heads][vd]; o_lat (nullable)
 * [n_heads][kvr]. */
void lo_mla_attn_heads(const float *c_kv, const float *k_rope, size_t seq, size_t kvr, size_t rope,
                       const float *q_nope, const float *q_rope, int kvb_type, const uint8_t *kv_b,
                       size_t n_heads, size_t nope, size_t vd, float scale, float *out, float *o_lat);

/* The MLA token (deepseek.zig:851-1048 attnLayer, 1275-1440 step) in the
 * shape mlaTokenFrame records: direct q, fused kv_b, MoE layers as
 * moeRun + shared expert, or dense SwiGLU layers. */
typedef struct {
    const float *attn_norm; /* [dim] */
    lo_tensor wq;           /* [n_heads * (nope + rope)][dim] */
    lo_tensor kv_a;         /* [kvr + rope][dim] */
    const float *kv_a_norm; /* [kvr] */
    lo_tensor kv_b;         /* [n_heads * (nope + vd)][kvr] */
    lo_tensor attn_out;     /* [dim][n_heads * vd] */
    const float *ffn_norm;  /* [dim] */
    int is_moe;
    lo_moe_layer moe;
    lo_tensor dgate, dup, ddown; /* dense FFN */
} lo_mla_layer;
typedef struct {
    size_t dim, n_heads, nope, rope, kvr, vd, n_layers, ctx_len, vocab;
    float eps, scale, rope_base, yarn_factor, yarn_orig_ctx;
    const lo_mla_layer *layers;
    const float *out_norm;
    lo_tensor output;
} lo_mla_model;
/* One token at pos: x [dim] is the embedding row in and the residual stream
 * after the last layer out; the caches ([n_layers][ctx_len][kvr] and
 * [n_layers][ctx_len][rope]) receive this position's rows; logits [vocab]. */
int lo_mla_step(const lo_mla_model *m, float *c_kv_cache, float *k_rope_cache, size_t pos, float *x, float *logits);
/* Test-only planted mistakes in lo_mla_step (0 = none): 1 k_rope cached
 * unrotated, 2 q's rope on the nope slice, 3 kv_a's norm skipped. */
void lo_set_mla_slip(int slip);

#ifdef __cplusplus
}
#endif
#endif
