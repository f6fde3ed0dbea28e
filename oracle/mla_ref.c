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
