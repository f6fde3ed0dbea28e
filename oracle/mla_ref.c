/*
 * mla_ref.c -- CPU restatement of Loom's MLA attention over the compressed
 * cache (src/gguf/deepseek.zig), the checker of libloomhip's MLA kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see loom_oracle.h).  Built with
 * -ffp-contract=off: every product is rounded before its add, as the
 * reference's Zig vector code evaluates it.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "loom_oracle.h"

/* deepseek.zig:581-613 ropeApply with YaRN (yarn_factor > 1): each adjacent
 * pair's angle blends the interpolated (theta / factor) and extrapolated
 * angle by a ramp over the corrected dimension range (beta_fast 32,
 * beta_slow 1); factor <= 1 is the plain NORM rope (deepseek.zig:615-629,
 * the same expressions as llama.zig's ropeNorm). */
static float yarn_corr_dim(float nd, float orig, float beta, float base) {
    const float two_pi = (float)(2.0 * 3.14159265358979323846); /* comptime 2*pi as f32 */
    return nd * logf(orig / (beta * two_pi)) / (2.0f * logf(base));
}

void lo_rope_yarn(float *vec, size_t n, size_t pos, float base, float factor, float orig_ctx) {
    if (!(factor > 1.0f)) {
        lo_rope_norm(vec, n, pos, base);
        return;
    }
    const float d = (float)n;
    const float low = fmaxf(0.0f, floorf(yarn_corr_dim(d, orig_ctx, 32.0f, base)));
    const float high = fminf(d - 1.0f, ceilf(yarn_corr_dim(d, orig_ctx, 1.0f, base)));
    for (size_t i = 0; 2 * i + 1 < n; i++) {
        const float exponent = (float)(2 * i) / d;
        const float freq = powf(base, -exponent);
        const float theta_extrap = (float)pos * freq;
        const float theta_interp = theta_extrap / factor;
        const float y = ((float)i - low) / fmaxf(0.001f, high - low);
        const float ramp_mix = 1.0f - fminf(fmaxf(y, 0.0f), 1.0f);
        const float theta = theta_interp * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
        const float c = cosf(theta), sn = sinf(theta);
        const float a = vec[2 * i], b = vec[2 * i + 1];
        vec[2 * i] = a * c - b * sn;
        vec[2 * i + 1] = a * sn + b * c;
    }
}

/* deepseek.zig:988-1047, the host loop over heads with the fused kv_b
 * (rows h*(nope+vd) .. +nope are head h's W_k, the next vd rows its W_v;
 * each row kvr long):
 *
 *   qa   = 0;  qa += q_nope[r] * W_k row r, r = 0 .. nope-1   (axpy, ggml.zig:222-231)
 *   s_t  = (dotF32(qa, c_t) + dotF32(q_rope, kr_t)) * scale    (ggml.zig:198-217)
 *   softmax(s)                                                  (tensor.zig:18-28)
 *   c_acc = 0;  c_acc += s_t * c_t, t = 0 .. seq-1              (axpy)
 *   out  = matvec(W_v, c_acc)                                   (ggml.zig:602)
 *
 * c_kv / k_rope are this layer's cache rows ([seq][kvr], [seq][rope]).
 * o_lat, when non-null, receives every head's c_acc ([n_heads][kvr]). */
void lo_mla_attn_heads(const float *c_kv, const float *k_rope, size_t seq, size_t kvr, size_t rope,
                       const float *q_nope, const float *q_rope, int kvb_type, const uint8_t *kv_b,
                       size_t n_heads, size_t nope, size_t vd, float scale, float *out, float *o_lat) {
    const size_t rb = lo_row_bytes(kvb_type, kvr);
    float *qa = (float *)malloc(kvr * sizeof(float));
    float *row = (float *)malloc(kvr * sizeof(float));
    float *sc = (float *)malloc((seq ? seq : 1) * sizeof(float));
    float *acc = (float *)malloc(kvr * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) {
        const size_t kb = h * (nope + vd);
        memset(qa, 0, kvr * sizeof(float));
        for (size_t r = 0; r < nope; r++) {
            lo_dequant_row(kvb_type, row, kv_b, kb + r, kvr);
            lo_axpy(qa, row, q_nope[h * nope + r], kvr);
        }
        for (size_t t = 0; t < seq; t++) {
            const float a = lo_dot_f32(qa, c_kv + t * kvr, kvr);
            const float b = lo_dot_f32(q_rope + h * rope, k_rope + t * rope, rope);
            sc[t] = (a + b) * scale;
        }
        lo_softmax(sc, seq);
        memset(acc, 0, kvr * sizeof(float));
        for (size_t t = 0; t < seq; t++)
            lo_axpy(acc, c_kv + t * kvr, sc[t], kvr);
        if (o_lat)
            memcpy(o_lat + h * kvr, acc, kvr * sizeof(float));
        lo_matvec(kvb_type, out + h * vd, kv_b + (kb + nope) * rb, acc, vd, kvr);
    }
    free(qa);
    free(row);
    free(sc);
    free(acc);
}

/* Planted-mistake switch for the step's pin test (test infrastructure only;
 * 0 in every other use): 1 = k_rope cached before its rope, 2 = q's rope
 * applied to the nope slice, 3 = kv_a's norm skipped. */
static int mla_slip;
void lo_set_mla_slip(int slip) { mla_slip = slip; }

/* deepseek.zig:851-1048 attnLayer and 1275-1440 step, in the shape
 * mlaTokenFrame records (compute/cpu.zig:73-79): per layer
 *   normed = rmsnorm(x) * attn_norm;  q = wq . normed;  kv_a = kv_a_mqa . normed
 *   c_kv row = rmsnorm(kv_a[0, kvr)) * kv_a_norm;  k_rope row = rope(kv_a[kvr, kvr + rope), pos)
 *   q's rope slice of every head = rope(., pos);  heads = the host head loop
 *   x += attn_output . heads;  normed = rmsnorm(x) * ffn_norm
 *   MoE: acc = moeRun + shared expert (moeFfnBlockRouted's sum), x += acc
 *   dense: x += down . swiglu(gate . normed, up . normed)
 * then logits = output . (rmsnorm(x) * out_norm). */
int lo_mla_step(const lo_mla_model *m, float *c_kv_cache, float *k_rope_cache, size_t pos, float *x, float *logits) {
    if (pos >= m->ctx_len)
        return -1;
    const size_t dim = m->dim, H = m->n_heads, nope = m->nope, rope = m->rope, kvr = m->kvr, vd = m->vd;
    const size_t kd = nope + rope;
    size_t fmax = 1;
    for (size_t li = 0; li < m->n_layers; li++) {
        const lo_mla_layer *L = &m->layers[li];
        const size_t f = L->is_moe ? 0 : L->dgate.ne1;
        fmax = f > fmax ? f : fmax;
    }
    float *normed = (float *)malloc(dim * 4), *q = (float *)malloc(H * kd * 4);
    float *kv_a = (float *)malloc((kvr + rope) * 4), *qn = (float *)malloc(H * nope * 4);
    float *qr = (float *)malloc(H * rope * 4), *heads = (float *)malloc(H * vd * 4), *tmp = (float *)malloc(dim * 4);
    float *g = (float *)malloc(fmax * 4), *u = (float *)malloc(fmax * 4), *act = (float *)malloc(fmax * 4);
    for (size_t li = 0; li < m->n_layers; li++) {
        const lo_mla_layer *L = &m->layers[li];
        lo_rmsnorm(normed, x, L->attn_norm, dim, m->eps);
        lo_matvec(L->wq.ty, q, L->wq.data, normed, L->wq.ne1, L->wq.ne0);
        lo_matvec(L->kv_a.ty, kv_a, L->kv_a.data, normed, L->kv_a.ne1, L->kv_a.ne0);
        float *c_row = c_kv_cache + (li * m->ctx_len + pos) * kvr;
        float *r_row = k_rope_cache + (li * m->ctx_len + pos) * rope;
        if (mla_slip == 3)
            memcpy(c_row, kv_a, kvr * 4);
        else
            lo_rmsnorm(c_row, kv_a, L->kv_a_norm, kvr, m->eps);
        memcpy(r_row, kv_a + kvr, rope * 4);
        if (mla_slip != 1)
            lo_rope_yarn(r_row, rope, pos, m->rope_base, m->yarn_factor, m->yarn_orig_ctx);
        for (size_t h = 0; h < H; h++)
            lo_rope_yarn(q + h * kd + (mla_slip == 2 ? 0 : nope), rope, pos, m->rope_base, m->yarn_factor,
                         m->yarn_orig_ctx);
        for (size_t h = 0; h < H; h++) {
            memcpy(qn + h * nope, q + h * kd, nope * 4);
            memcpy(qr + h * rope, q + h * kd + nope, rope * 4);
        }
        lo_mla_attn_heads(c_kv_cache + li * m->ctx_len * kvr, k_rope_cache + li * m->ctx_len * rope, pos + 1, kvr,
                          rope, qn, qr, L->kv_b.ty, L->kv_b.data, H, nope, vd, m->scale, heads, NULL);
        lo_matvec(L->attn_out.ty, tmp, L->attn_out.data, heads, dim, H * vd);
        lo_add(x, tmp, dim);
        lo_rmsnorm(normed, x, L->ffn_norm, dim, m->eps);
        if (L->is_moe) {
            lo_moe_layer_token(&L->moe, normed, tmp, NULL, NULL);
        } else {
            const size_t f = L->dgate.ne1;
            lo_matvec(L->dgate.ty, g, L->dgate.data, normed, f, dim);
            lo_matvec(L->dup.ty, u, L->dup.data, normed, f, dim);
            lo_swiglu(act, g, u, f);
            lo_matvec(L->ddown.ty, tmp, L->ddown.data, act, dim, f);
        }
        lo_add(x, tmp, dim);
    }
    lo_rmsnorm(normed, x, m->out_norm, dim, m->eps);
    lo_matvec(m->output.ty, logits, m->output.data, normed, m->vocab, dim);
    free(normed);
    free(q);
    free(kv_a);
    free(qn);
    free(qr);
    free(heads);
    free(tmp);
    free(g);
    free(u);
    free(act);
    return 0;
}
