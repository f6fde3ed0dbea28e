/*
 * model_ref.c -- TEST INFRASTRUCTURE: restatement of the elementwise ops
 * (src/core/tensor.zig), the router (src/gguf/moe.zig:106-158), the MoE layer
 * (src/gguf/llama.zig moeLayer/moeRun/moeBatchUnion) and the GQA decode step
 * (llama.zig step/decodeBatch) for the architectures on this path: llama
 * (NORM rope, dense SwiGLU FFN) and qwen3moe (NEOX rope, per-head Q/K RMSNorm,
 * routed MoE).  QKV biases, sliding windows, attention sinks, YaRN, MTP and
 * shared experts are absent from every config here and are not restated.
 *
 * Unpinned without running Zig: @exp, @sqrt, std.math.pow, @cos, @sin map to
 * C libm sqrtf, powf, cosf, sinf and, for @exp, the once-rounded double
 * exponential (float)exp((double)x) -- the f32 exponential rounded once from
 * a double result, which is the correctly rounded value except where the
 * double lands within an ulp of a float midpoint (about 2^-29 of inputs).
 * Any libm expf agrees with it to within an ulp; the GPU computes the same
 * expression, so softmax, SiLU and sigmoid agree bit for bit.
 */
#include "loom_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- core/tensor.zig ------------------------------------------------------ */

/* @exp on f32 (tensor.zig:24,31,35): the once-rounded double exponential. */
static inline float exp_f32(float x) { return (float)exp((double)x); }

/* tensor.zig:9-15 */
void lo_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float p = x[i] * x[i];
        ss = ss + p;
    }
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) {
        float a = x[i] * scale;
        out[i] = a * w[i];
    }
}

/* tensor.zig:18-28 */
void lo_softmax(float *x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++)
        m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = exp_f32(x[i] - m);
        sum = sum + x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++)
        x[i] = x[i] * inv;
}

/* tensor.zig:30-36 */
float lo_silu(float x) { return x / (1.0f + exp_f32(-x)); }
float lo_sigmoid(float x) { return 1.0f / (1.0f + exp_f32(-x)); }

/* tensor.zig:55-57 */
void lo_swiglu(float *out, const float *g, const float *u, size_t n) {
    for (size_t i = 0; i < n; i++)
        out[i] = lo_silu(g[i]) * u[i];
}

/* tensor.zig:50-52 */
void lo_add(float *dst, const float *src, size_t n) {
    for (size_t i = 0; i < n; i++)
        dst[i] = dst[i] + src[i];
}

/* llama.zig:821-826 ropeTheta */
static inline void rope_theta(size_t i, size_t rope_dim, size_t pos, float base, float *c,
                              float *s) {
    float exponent = (float)i / (float)rope_dim;
    float freq = powf(base, -exponent);
    float angle = (float)pos * freq;
    *c = cosf(angle);
    *s = sinf(angle);
}

/* llama.zig:830-839 ropeNorm: adjacent pairs */
void lo_rope_norm(float *vec, size_t rope_dim, size_t pos, float base) {
    for (size_t i = 0; i + 1 < rope_dim; i += 2) {
        float c, s;
        rope_theta(i, rope_dim, pos, base, &c, &s);
        float a = vec[i], b = vec[i + 1];
        vec[i] = a * c - b * s;
        vec[i + 1] = a * s + b * c;
    }
}

/* llama.zig:845-855 ropeNeox: split-half pairs */
void lo_rope_neox(float *vec, size_t rope_dim, size_t pos, float base) {
    size_t half = rope_dim / 2;
    for (size_t i = 0; i < half; i++) {
        float c, s;
        rope_theta(2 * i, rope_dim, pos, base, &c, &s);
        float a = vec[i], b = vec[i + half];
        vec[i] = a * c - b * s;
        vec[i + half] = a * s + b * c;
    }
}

/* llama.zig:938-949 headNorm */
void lo_head_norm(float *vec, const float *w, size_t n_heads, size_t hd, float eps) {
    if (!w)
        return;
    for (size_t h = 0; h < n_heads; h++) {
        float *head = vec + h * hd;
        float ss = 0.0f;
        for (size_t i = 0; i < hd; i++) {
            float p = head[i] * head[i];
            ss = ss + p;
        }
        float inv = 1.0f / sqrtf(ss / (float)hd + eps);
        for (size_t i = 0; i < hd; i++) {
            float a = head[i] * inv;
            head[i] = a * w[i];
        }
    }
}

/* engine/sampler.zig:7-15: first maximum wins. */
size_t lo_argmax(const float *logits, size_t n) {
    size_t best = 0;
    float best_v = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    return best;
}

/* ---- gguf/moe.zig:106-158 route ------------------------------------------ */

void lo_route(const lo_route_cfg *cfg, const float *logits, const float *bias, uint32_t *ids,
              float *gates) {
    size_t ne = cfg->n_expert, k = cfg->n_used;
    float *scores = (float *)malloc(ne * sizeof(float));
    float *choice = (float *)malloc(ne * sizeof(float));
    unsigned char *used = (unsigned char *)calloc(ne, 1);
    if (cfg->gating == LO_GATING_SIGMOID) {
        for (size_t i = 0; i < ne; i++)
            scores[i] = lo_sigmoid(logits[i]);
    } else {
        memcpy(scores, logits, ne * sizeof(float));
        if (cfg->gating == LO_GATING_SOFTMAX)
            lo_softmax(scores, ne);
    }
    for (size_t i = 0; i < ne; i++)
        choice[i] = bias ? scores[i] + bias[i] : scores[i];
    /* k rounds of argmax over the unused experts; strict '>' keeps the
     * lowest index on ties; gates come from the unbiased scores. */
    for (size_t s = 0; s < k; s++) {
        size_t best = 0;
        float best_v = -INFINITY;
        for (size_t e = 0; e < ne; e++)
            if (!used[e] && choice[e] > best_v) {
                best_v = choice[e];
                best = e;
            }
        used[best] = 1;
        ids[s] = (uint32_t)best;
        gates[s] = scores[best];
    }
    if (cfg->gating == LO_GATING_SOFTMAX_TOPK)
        lo_softmax(gates, k);
    if (cfg->weights_norm) {
        float sum = 0.0f;
        for (size_t s = 0; s < k; s++)
            sum = sum + gates[s];
        float denom = fmaxf(sum, 6.103515625e-5f);
        for (size_t s = 0; s < k; s++)
            gates[s] = gates[s] / denom;
    }
    if (cfg->weights_scale != 1.0f)
        for (size_t s = 0; s < k; s++)
            gates[s] = gates[s] * cfg->weights_scale;
    free(scores);
    free(choice);
    free(used);
}

/* ---- MoE layer ----------------------------------------------------------- */

/* llama.zig:136-142 Tensor.expert: byte plane of expert e. */
static const uint8_t *expert_plane(const lo_tensor *t, size_t e) {
    return t->data + e * t->ne1 * lo_row_bytes(t->ty, t->ne0);
}

/* llama.zig:1262-1272 moeLayer (router mv + logit bias + route) */
static void route_token(const lo_moe_layer *L, const float *normed, uint32_t *ids, float *gates) {
    size_t ne = L->route.n_expert;
    float *logits = (float *)malloc(ne * sizeof(float));
    lo_matvec(L->router.ty, logits, L->router.data, normed, ne, L->dim);
    if (L->router_bias)
        for (size_t i = 0; i < ne; i++)
            logits[i] = logits[i] + L->router_bias[i];
    lo_route(&L->route, logits, L->sel_bias, ids, gates);
    free(logits);
}

/* llama.zig:1307-1419 moeRun (local path) + denseFFN 952-958 */
/* llama.zig:952-958 denseFFN of one plane each: gate and up matvecs, SwiGLU,
 * down; out[dim]. */
static void dense_ffn(const lo_tensor *gt, const lo_tensor *ut, const lo_tensor *dt, const float *x, size_t dim,
                      float *out) {
    size_t f = gt->ne1;
    float *g = (float *)malloc(f * sizeof(float)), *u = (float *)malloc(f * sizeof(float));
    float *a = (float *)malloc(f * sizeof(float));
    lo_matvec(gt->ty, g, gt->data, x, f, dim);
    lo_matvec(ut->ty, u, ut->data, x, f, dim);
    lo_swiglu(a, g, u, f);
    lo_matvec(dt->ty, out, dt->data, a, dim, f);
    free(g);
    free(u);
    free(a);
}

/* acc += the shared expert's FFN of x (tensor.zig add: acc[i] + v[i]). */
static void shared_ffn_add(const lo_moe_layer *L, const float *x, float *acc) {
    float *o = (float *)malloc(L->dim * sizeof(float));
    dense_ffn(&L->shexp_gate, &L->shexp_up, &L->shexp_down, x, L->dim, o);
    lo_add(acc, o, L->dim);
    free(o);
}

void lo_moe_ffn_block(const float *normed, size_t dim, const lo_expert_ref *refs, size_t n, float *out) {
    float *o = (float *)malloc(dim * sizeof(float));
    memset(out, 0, dim * sizeof(float));
    for (size_t r = 0; r < n; r++) {
        dense_ffn(&refs[r].gate, &refs[r].up, &refs[r].down, normed, dim, o);
        for (size_t i = 0; i < dim; i++) {
            float p = refs[r].weight * o[i];
            out[i] = out[i] + p;
        }
    }
    free(o);
}

void lo_moe_layer_token(const lo_moe_layer *L, const float *normed, float *acc, uint32_t *ids_out,
                        float *gates_out) {
    size_t k = L->route.n_used, dim = L->dim, f = L->ffn;
    uint32_t *ids = (uint32_t *)malloc(k * sizeof(uint32_t));
    float *gates = (float *)malloc(k * sizeof(float));
    route_token(L, normed, ids, gates);
    float *g = (float *)malloc(f * sizeof(float)), *u = (float *)malloc(f * sizeof(float));
    float *a = (float *)malloc(f * sizeof(float)), *o = (float *)malloc(dim * sizeof(float));
    memset(acc, 0, dim * sizeof(float));
    for (size_t s = 0; s < k; s++) {
        size_t e = ids[s];
        lo_matvec(L->gate_exps.ty, g, expert_plane(&L->gate_exps, e), normed, f, dim);
        lo_matvec(L->up_exps.ty, u, expert_plane(&L->up_exps, e), normed, f, dim);
        lo_swiglu(a, g, u, f);
        lo_matvec(L->down_exps.ty, o, expert_plane(&L->down_exps, e), a, dim, f);
        for (size_t i = 0; i < dim; i++) {
            float p = gates[s] * o[i];
            acc[i] = acc[i] + p;
        }
    }
    if (L->shexp_gate.data) /* deepseek.zig:1497-1502: denseFFN(shexp), add(acc, ffn_out) */
        shared_ffn_add(L, normed, acc);
    if (ids_out)
        memcpy(ids_out, ids, k * sizeof(uint32_t));
    if (gates_out)
        memcpy(gates_out, gates, k * sizeof(float));
    free(ids);
    free(gates);
    free(g);
    free(u);
    free(a);
    free(o);
}

/* llama.zig:1828-1903 moeBatchUnion: route every lane, then visit experts in
 * ascending id order, run each expert once over the lanes that chose it, and
 * add gate * out straight into that lane's residual. */
void lo_moe_batch_union(const lo_moe_layer *L, const float *bnormed, float *bx, size_t n,
                        uint32_t *ids_out, float *gates_out) {
    size_t k = L->route.n_used, dim = L->dim, f = L->ffn, ne = L->route.n_expert;
    uint32_t *ids = (uint32_t *)malloc(n * k * sizeof(uint32_t));
    float *gates = (float *)malloc(n * k * sizeof(float));
    for (size_t t = 0; t < n; t++)
        route_token(L, bnormed + t * dim, ids + t * k, gates + t * k);
    size_t *lanes = (size_t *)malloc(n * sizeof(size_t));
    float *lg = (float *)malloc(n * sizeof(float));
    float *gather = (float *)malloc(n * dim * sizeof(float));
    float *bg = (float *)malloc(n * f * sizeof(float)), *bu = (float *)malloc(n * f * sizeof(float));
    float *ba = (float *)malloc(n * f * sizeof(float)), *bo = (float *)malloc(n * dim * sizeof(float));
    for (size_t e = 0; e < ne; e++) {
        size_t m = 0;
        for (size_t t = 0; t < n; t++)
            for (size_t s = 0; s < k; s++)
                if (ids[t * k + s] == e) {
                    lanes[m] = t;
                    lg[m] = gates[t * k + s];
                    m++;
                    break;
                }
        if (m == 0)
            continue;
        for (size_t j = 0; j < m; j++)
            memcpy(gather + j * dim, bnormed + lanes[j] * dim, dim * sizeof(float));
        lo_matmul(L->gate_exps.ty, bg, expert_plane(&L->gate_exps, e), gather, m, f, dim);
        lo_matmul(L->up_exps.ty, bu, expert_plane(&L->up_exps, e), gather, m, f, dim);
        for (size_t j = 0; j < m; j++)
            lo_swiglu(ba + j * f, bg + j * f, bu + j * f, f);
        lo_matmul(L->down_exps.ty, bo, expert_plane(&L->down_exps, e), ba, m, dim, f);
        for (size_t j = 0; j < m; j++) {
            float *dst = bx + lanes[j] * dim;
            for (size_t i = 0; i < dim; i++) {
                float p = lg[j] * bo[j * dim + i];
                dst[i] = dst[i] + p;
            }
        }
    }
    if (L->shexp_gate.data) /* the shared expert of every lane, after its routed experts */
        for (size_t t = 0; t < n; t++)
            shared_ffn_add(L, bnormed + t * dim, bx + t * dim);
    if (ids_out)
        memcpy(ids_out, ids, n * k * sizeof(uint32_t));
    if (gates_out)
        memcpy(gates_out, gates, n * k * sizeof(float));
    free(ids);
    free(gates);
    free(lanes);
    free(lg);
    free(gather);
    free(bg);
    free(bu);
    free(ba);
    free(bo);
}

/* ---- GQA decode ------------------------------------------------------------ */

static size_t kv_dim(const lo_model *m) { return m->n_kv_heads * m->head_dim; }

size_t lo_seq_cache_bytes(const lo_model *m) {
    return m->n_layers * m->ctx_len * kv_dim(m) * (m->kv_f16 ? 2 : 4);
}

static void kv_store(const lo_model *m, void *cache, size_t idx, const float *src, size_t n) {
    if (m->kv_f16) {
        uint16_t *c = (uint16_t *)cache + idx;
        for (size_t i = 0; i < n; i++)
            c[i] = lo_f32_to_f16(src[i]);
    } else {
        memcpy((float *)cache + idx, src, n * sizeof(float));
    }
}

/* Widening of fp16 cache values (exact), through a table of all 65536. */
static float f16_table[65536];
static int f16_table_ready;

static void f16_table_init(void) {
    if (f16_table_ready)
        return;
    for (uint32_t h = 0; h < 65536; h++)
        f16_table[h] = lo_f16_to_f32((uint16_t)h);
    f16_table_ready = 1;
}

/* n consecutive cache rows of one KV head (hd values at stride kvd) as f32. */
static void kv_rows(const lo_model *m, const void *cache, size_t idx, size_t rows, size_t kvd, float *dst) {
    size_t hd = m->head_dim;
    for (size_t r = 0; r < rows; r++) {
        if (m->kv_f16) {
            const uint16_t *c = (const uint16_t *)cache + idx + r * kvd;
            for (size_t i = 0; i < hd; i++)
                dst[r * hd + i] = f16_table[c[i]];
        } else {
            memcpy(dst + r * hd, (const float *)cache + idx + r * kvd, hd * sizeof(float));
        }
    }
}

static void rope_vec(const lo_model *m, float *v, size_t pos) {
    if (m->rope_neox)
        lo_rope_neox(v, m->rope_dim, pos, m->rope_base);
    else
        lo_rope_norm(v, m->rope_dim, pos, m->rope_base);
}

/* Planted-mistake switch for the batch-invariant test (test infrastructure
 * only; 0 in every other use): 1 = each lane attends over the next lane's
 * cache, 2 = each lane writes its K/V row at its batch index instead of its
 * position, 3 = every lane rotates q and k at lane 0's position. */
static int batch_slip;
void lo_set_batch_slip(int slip) { batch_slip = slip; }

/* llama.zig:1162-1192, the per-head attention loop (backend.attnHeads'
 * contract, src/compute/cpu.zig:163-176): for each query head h of KV head
 * kvh, s_t = dotF32(q_h, k_t) * scale over cache rows [0, pos] of layer li,
 * softmax, then o_h = sum_t p_t v_t by axpy in position order from +0.
 * kf/vf hold one KV head's rows widened to f32 (pos + 1 rows of head_dim),
 * scores pos + 1 floats. */
static void attn_heads_impl(const lo_model *m, const void *k_cache, const void *v_cache, size_t li, size_t pos,
                            const float *q, float *attn_out, float scale, float *scores, float *kf, float *vf) {
    size_t hd = m->head_dim, kvd = kv_dim(m);
    size_t q_per_kv = m->n_heads / m->n_kv_heads;
    for (size_t kvh = 0; kvh < m->n_kv_heads; kvh++) {
        size_t row0 = (li * m->ctx_len) * kvd + kvh * hd;
        kv_rows(m, k_cache, row0, pos + 1, kvd, kf);
        kv_rows(m, v_cache, row0, pos + 1, kvd, vf);
        for (size_t h = kvh * q_per_kv; h < (kvh + 1) * q_per_kv; h++) {
            const float *qh = q + h * hd;
            for (size_t t = 0; t <= pos; t++)
                scores[t] = lo_dot_f32(qh, kf + t * hd, hd) * scale;
            lo_softmax(scores, pos + 1);
            float *oh = attn_out + h * hd;
            memset(oh, 0, hd * sizeof(float));
            for (size_t t = 0; t <= pos; t++)
                lo_axpy(oh, vf + t * hd, scores[t], hd);
        }
    }
}

/* llama.zig:1127-1192: q/k/v for one lane, Q/K norm, rope, KV append and the
 * per-head attention loop, into attn_out.  The lane writes its own cache at
 * write_pos and reads rows [0, pos] of read_seq's cache (both its own outside
 * the planted mistakes).  kf/vf hold one KV head's rows widened to f32 (ctx x
 * head_dim each): every query head of the group reads the same exact values
 * the reference's f32 cache would hold. */
static void attention_lane(const lo_model *m, const lo_layer *l, size_t li, lo_seq *seq,
                           const lo_seq *read_seq, size_t write_pos, size_t rope_pos, float *q, float *k,
                           const float *v, float *attn_out, float *scores, float *kf, float *vf) {
    size_t hd = m->head_dim, kvd = kv_dim(m), pos = seq->pos;
    f16_table_init();
    lo_head_norm(q, l->q_norm, m->n_heads, hd, m->eps);
    lo_head_norm(k, l->k_norm, m->n_kv_heads, hd, m->eps);
    for (size_t h = 0; h < m->n_heads; h++)
        rope_vec(m, q + h * hd, rope_pos);
    for (size_t h = 0; h < m->n_kv_heads; h++)
        rope_vec(m, k + h * hd, rope_pos);
    size_t base = (li * m->ctx_len + write_pos) * kvd;
    kv_store(m, seq->k_cache, base, k, kvd);
    kv_store(m, seq->v_cache, base, v, kvd);
    attn_heads_impl(m, read_seq->k_cache, read_seq->v_cache, li, pos, q, attn_out, 1.0f / sqrtf((float)hd),
                    scores, kf, vf);
}

void lo_attn_heads(const lo_model *m, const void *k_cache, const void *v_cache, size_t li, size_t pos,
                   const float *q, float *attn_out, float scale) {
    float *scores = (float *)malloc((pos + 1) * 4);
    float *kf = (float *)malloc((pos + 1) * m->head_dim * 4), *vf = (float *)malloc((pos + 1) * m->head_dim * 4);
    f16_table_init();
    attn_heads_impl(m, k_cache, v_cache, li, pos, q, attn_out, scale, scores, kf, vf);
    free(scores);
    free(kf);
    free(vf);
}

static void mv(const lo_tensor *t, float *out, const float *x) {
    lo_matvec(t->ty, out, t->data, x, t->ne1, t->ne0);
}

/* llama.zig:1111-1227 step */
int lo_step(const lo_model *m, lo_seq *seq, uint32_t token, float *logits) {
    if (token >= m->vocab || seq->pos >= m->ctx_len)
        return -1;
    size_t dim = m->dim, hd = m->head_dim, qd = m->n_heads * hd, kvd = kv_dim(m);
    size_t fmax = 0;
    for (size_t li = 0; li < m->n_layers; li++) {
        size_t f = m->layers[li].is_moe ? m->layers[li].moe.ffn : m->layers[li].ffn_gate.ne1;
        if (f > fmax)
            fmax = f;
    }
    float *x = (float *)malloc(dim * 4), *normed = (float *)malloc(dim * 4);
    float *q = (float *)malloc(qd * 4), *k = (float *)malloc(kvd * 4), *v = (float *)malloc(kvd * 4);
    float *att = (float *)malloc(qd * 4), *proj = (float *)malloc(dim * 4);
    float *scores = (float *)malloc(m->ctx_len * 4);
    float *kf = (float *)malloc(m->ctx_len * hd * 4), *vf = (float *)malloc(m->ctx_len * hd * 4);
    float *g = (float *)malloc(fmax * 4), *u = (float *)malloc(fmax * 4), *a = (float *)malloc(fmax * 4);
    float *acc = (float *)malloc(dim * 4);
    lo_dequant_row(m->embed.ty, x, m->embed.data, token, dim);
    for (size_t li = 0; li < m->n_layers; li++) {
        const lo_layer *l = &m->layers[li];
        lo_rmsnorm(normed, x, l->attn_norm, dim, m->eps);
        mv(&l->wq, q, normed);
        mv(&l->wk, k, normed);
        mv(&l->wv, v, normed);
        attention_lane(m, l, li, seq, seq, seq->pos, seq->pos, q, k, v, att, scores, kf, vf);
        mv(&l->wo, proj, att);
        lo_add(x, proj, dim);
        lo_rmsnorm(normed, x, l->ffn_norm, dim, m->eps);
        if (l->is_moe) {
            lo_moe_layer_token(&l->moe, normed, acc, NULL, NULL);
            lo_add(x, acc, dim);
        } else {
            size_t f = l->ffn_gate.ne1;
            mv(&l->ffn_gate, g, normed);
            mv(&l->ffn_up, u, normed);
            lo_swiglu(a, g, u, f);
            mv(&l->ffn_down, proj, a);
            lo_add(x, proj, dim);
        }
    }
    lo_rmsnorm(normed, x, m->out_norm, dim, m->eps);
    mv(&m->output, logits, normed);
    seq->pos++;
    free(x);
    free(normed);
    free(q);
    free(k);
    free(v);
    free(att);
    free(proj);
    free(scores);
    free(kf);
    free(vf);
    free(g);
    free(u);
    free(a);
    free(acc);
    return 0;
}

/* llama.zig:1939-2043 decodeBatch (any n: matmul is bit-identical to n
 * matvecs, so lanes beyond MAX_BATCH run the same arithmetic). */
int lo_decode_batch(const lo_model *m, lo_seq *seqs, const uint32_t *tokens, size_t n, float *out) {
    size_t dim = m->dim, hd = m->head_dim, qd = m->n_heads * hd, kvd = kv_dim(m);
    for (size_t t = 0; t < n; t++)
        if (tokens[t] >= m->vocab || seqs[t].pos >= m->ctx_len)
            return -1;
    size_t fmax = 0;
    for (size_t li = 0; li < m->n_layers; li++) {
        size_t f = m->layers[li].is_moe ? m->layers[li].moe.ffn : m->layers[li].ffn_gate.ne1;
        if (f > fmax)
            fmax = f;
    }
    float *bx = (float *)malloc(n * dim * 4), *bn = (float *)malloc(n * dim * 4);
    float *bq = (float *)malloc(n * qd * 4), *bk = (float *)malloc(n * kvd * 4);
    float *bv = (float *)malloc(n * kvd * 4), *ba = (float *)malloc(n * qd * 4);
    float *bp = (float *)malloc(n * dim * 4), *scores = (float *)malloc(m->ctx_len * 4);
    float *kf = (float *)malloc(m->ctx_len * hd * 4), *vf = (float *)malloc(m->ctx_len * hd * 4);
    float *bg = (float *)malloc(n * fmax * 4), *bu = (float *)malloc(n * fmax * 4);
    float *bact = (float *)malloc(n * fmax * 4), *normed = (float *)malloc(dim * 4);
    for (size_t t = 0; t < n; t++)
        lo_dequant_row(m->embed.ty, bx + t * dim, m->embed.data, tokens[t], dim);
    for (size_t li = 0; li < m->n_layers; li++) {
        const lo_layer *l = &m->layers[li];
        for (size_t t = 0; t < n; t++)
            lo_rmsnorm(bn + t * dim, bx + t * dim, l->attn_norm, dim, m->eps);
        lo_matmul(l->wq.ty, bq, l->wq.data, bn, n, l->wq.ne1, l->wq.ne0);
        lo_matmul(l->wk.ty, bk, l->wk.data, bn, n, l->wk.ne1, l->wk.ne0);
        lo_matmul(l->wv.ty, bv, l->wv.data, bn, n, l->wv.ne1, l->wv.ne0);
        for (size_t t = 0; t < n; t++) {
            const lo_seq *rs = batch_slip == 1 ? &seqs[(t + 1) % n] : &seqs[t];
            size_t wp = batch_slip == 2 ? t : seqs[t].pos;
            size_t rp = batch_slip == 3 ? seqs[0].pos : seqs[t].pos;
            attention_lane(m, l, li, &seqs[t], rs, wp, rp, bq + t * qd, bk + t * kvd, bv + t * kvd,
                           ba + t * qd, scores, kf, vf);
        }
        lo_matmul(l->wo.ty, bp, l->wo.data, ba, n, l->wo.ne1, l->wo.ne0);
        for (size_t t = 0; t < n; t++)
            lo_add(bx + t * dim, bp + t * dim, dim);
        for (size_t t = 0; t < n; t++)
            lo_rmsnorm(bn + t * dim, bx + t * dim, l->ffn_norm, dim, m->eps);
        if (l->is_moe) {
            lo_moe_batch_union(&l->moe, bn, bx, n, NULL, NULL);
        } else {
            size_t f = l->ffn_gate.ne1;
            lo_matmul(l->ffn_gate.ty, bg, l->ffn_gate.data, bn, n, f, dim);
            lo_matmul(l->ffn_up.ty, bu, l->ffn_up.data, bn, n, f, dim);
            for (size_t t = 0; t < n; t++)
                lo_swiglu(bact + t * f, bg + t * f, bu + t * f, f);
            lo_matmul(l->ffn_down.ty, bp, l->ffn_down.data, bact, n, dim, f);
            for (size_t t = 0; t < n; t++)
                lo_add(bx + t * dim, bp + t * dim, dim);
        }
    }
    for (size_t t = 0; t < n; t++) {
        lo_rmsnorm(normed, bx + t * dim, m->out_norm, dim, m->eps);
        mv(&m->output, out + t * m->vocab, normed);
        seqs[t].pos++;
    }
    free(bx);
    free(bn);
    free(bq);
    free(bk);
    free(bv);
    free(ba);
    free(bp);
    free(scores);
    free(kf);
    free(vf);
    free(bg);
    free(bu);
    free(bact);
    free(normed);
    return 0;
}
