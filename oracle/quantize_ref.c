/*
 * quantize_ref.c -- TEST INFRASTRUCTURE: input generators.
 *
 *  - lo_quantize_q4_0 / lo_quantize_q8_0 restate the reference's test-only
 *    quantizers (src/gguf/ggml.zig:1861-1904).
 *  - lo_quantize_q4_k / lo_quantize_q6_k implement GGML's published reference
 *    quantizers (quantize_row_q4_K_ref with make_qkx2_quants, and
 *    quantize_row_q6_K_ref with make_qx_quants, llama.cpp ggml-quants.c, MIT).
 *    The reference repository contains no Q4_K/Q6_K quantizer and no golden
 *    vectors for one, so these are pinned only by their own round-trip error
 *    bounds (tests/test_oracle_ggml.py); every dequant/matvec parity claim is
 *    defined on whatever bytes they emit.
 *  - splitmix64-based seeded normals/uniforms for synthetic inputs.
 */
#include "loom_oracle.h"

#include <math.h>
#include <string.h>

/* ggml.zig:1861-1884 quantizeQ40: scale = vmax / -8 (signed value of largest
 * magnitude), stored as f16; q = clamp(trunc(x/scale + 8.5), 0, 15) with the
 * f32 scale's reciprocal. Lane j low nibble, lane j+16 high nibble. */
void lo_quantize_q4_0(uint8_t *dst, const float *src, size_t n) {
    for (size_t b = 0; b * LO_QK_0 < n; b++) {
        const float *in = src + b * LO_QK_0;
        uint8_t *blk = dst + b * 18;
        float amax = 0.0f, vmax = 0.0f;
        for (int i = 0; i < LO_QK_0; i++)
            if (fabsf(in[i]) > amax) {
                amax = fabsf(in[i]);
                vmax = in[i];
            }
        float scale = vmax / -8.0f;
        uint16_t h = lo_f32_to_f16(scale);
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        for (int j = 0; j < 16; j++) {
            float a = in[j] * inv, c = in[j + 16] * inv;
            int lo = (int)(a + 8.5f), hi = (int)(c + 8.5f);
            lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
            hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
            blk[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* ggml.zig:1886-1904 quantizeQ80: scale = amax/127 (f16), q = round(x*inv). */
void lo_quantize_q8_0(uint8_t *dst, const float *src, size_t n) {
    for (size_t b = 0; b * LO_QK_0 < n; b++) {
        const float *in = src + b * LO_QK_0;
        uint8_t *blk = dst + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < LO_QK_0; i++)
            amax = fmaxf(amax, fabsf(in[i]));
        float scale = amax / 127.0f;
        uint16_t h = lo_f32_to_f16(scale);
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        for (int j = 0; j < LO_QK_0; j++) {
            int q = (int)roundf(in[j] * inv);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            blk[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}

/* GGML's round-to-nearest-even via the 1.5*2^23 bias. */
static inline int nearest_int(float f) {
    float v = f + 12582912.0f;
    int32_t i;
    memcpy(&i, &v, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* make_qkx2_quants: asymmetric (scale, min) fit of n values to 0..nmax,
 * weighted least squares over a small grid of candidate scales. */
static float fit_scale_min(int n, int nmax, const float *x, const float *w, uint8_t *L,
                           float *the_min, uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float mn = x[0], mx = x[0];
    float sum_w = w[0], sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < mn)
            mn = x[i];
        if (x[i] > mx)
            mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0)
        mn = 0;
    if (mx == mn) {
        for (int i = 0; i < n; i++)
            L[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1.0f / iscale;
    float best_err = 0.0f;
    for (int i = 0; i < n; i++) {
        int l = nearest_int(iscale * (x[i] - mn));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * L[i] + mn - x[i];
        best_err += w[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * (x[i] - mn));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float err = 0;
            for (int i = 0; i < n; i++) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                err += w[i] * (diff * diff);
            }
            if (err < best_err) {
                memcpy(L, Laux, (size_t)n);
                best_err = err;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

/* quantize_row_q4_K_ref: eight 32-value groups, each fitted with
 * fit_scale_min; group scales/mins quantized to 6 bits against the block
 * maxima; f16 d = max_scale/63, dmin = max_min/63; values re-quantized
 * against the stored scales. */
void lo_quantize_q4_k(uint8_t *dst, const float *src, size_t n) {
    for (size_t b = 0; b * LO_QK_K < n; b++) {
        const float *x = src + b * LO_QK_K;
        uint8_t *blk = dst + b * 144;
        uint8_t L[LO_QK_K], Laux[32];
        float weights[32], mins[8], scales[8];
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; j++) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; l++)
                sum_x2 += x[32 * j + l] * x[32 * j + l];
            float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; l++)
                weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = fit_scale_min(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.0f,
                                      0.1f, 20);
            if (scales[j] > max_scale)
                max_scale = scales[j];
            if (mins[j] > max_min)
                max_min = mins[j];
        }
        float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
        uint8_t *sc = blk + 4;
        memset(sc, 0, 12);
        for (int j = 0; j < 8; j++) {
            int ls = nearest_int(inv_scale * scales[j]);
            int lm = nearest_int(inv_min * mins[j]);
            ls = ls > 63 ? 63 : ls;
            lm = lm > 63 ? 63 : lm;
            if (j < 4) {
                sc[j] = (uint8_t)ls;
                sc[j + 4] = (uint8_t)lm;
            } else {
                sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        uint16_t hd = lo_f32_to_f16(max_scale / 63.0f), hm = lo_f32_to_f16(max_min / 63.0f);
        blk[0] = (uint8_t)(hd & 0xff);
        blk[1] = (uint8_t)(hd >> 8);
        blk[2] = (uint8_t)(hm & 0xff);
        blk[3] = (uint8_t)(hm >> 8);
        float d_all = lo_f16_to_f32(hd), dmin_all = lo_f16_to_f32(hm);
        for (int j = 0; j < 8; j++) {
            uint8_t s, m;
            if (j < 4) {
                s = sc[j] & 63;
                m = sc[j + 4] & 63;
            } else {
                s = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
                m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
            }
            float d = d_all * s;
            if (d == 0.0f)
                continue;
            float dm = dmin_all * m;
            for (int i = 0; i < 32; i++) {
                int l = nearest_int((x[32 * j + i] + dm) / d);
                L[32 * j + i] = (uint8_t)(l < 0 ? 0 : (l > 15 ? 15 : l));
            }
        }
        uint8_t *q = blk + 16;
        for (int j = 0; j < LO_QK_K; j += 64) {
            for (int l = 0; l < 32; l++)
                q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
    }
}

/* make_qx_quants with rmse_type 1 (weights x^2): symmetric fit of n values
 * to -nmax..nmax-1, trying 18 perturbed scales around nmax/max. */
static float fit_symmetric(int n, int nmax, const float *x, int8_t *L) {
    float mx = 0, amax = 0;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            mx = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; i++)
            L[i] = 0;
        return 0.0f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; i++) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; is++) {
        if (is == 0)
            continue;
        iscale = -(nmax + 0.1f * is) / mx;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; i++) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + (l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* quantize_row_q6_K_ref: sixteen 16-value groups fitted symmetrically; the
 * group scales quantized to i8 against the largest-magnitude one (d = that
 * scale / -128); values re-quantized to 6 bits against the stored scales. */
void lo_quantize_q6_k(uint8_t *dst, const float *src, size_t n) {
    for (size_t b = 0; b * LO_QK_K < n; b++) {
        const float *x = src + b * LO_QK_K;
        uint8_t *blk = dst + b * 210;
        int8_t L[LO_QK_K];
        float scales[16];
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < 16; ib++) {
            float s = fit_symmetric(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = s;
            if (fabsf(s) > max_abs_scale) {
                max_abs_scale = fabsf(s);
                max_scale = s;
            }
        }
        memset(blk, 0, 210);
        if (max_abs_scale < 1e-15f)
            continue; /* all-zero block, d = +0 */
        float iscale = -128.0f / max_scale;
        uint16_t hd = lo_f32_to_f16(1.0f / iscale);
        blk[208] = (uint8_t)(hd & 0xff);
        blk[209] = (uint8_t)(hd >> 8);
        int8_t *sc = (int8_t *)(blk + 192);
        for (int ib = 0; ib < 16; ib++) {
            int v = nearest_int(iscale * scales[ib]);
            sc[ib] = (int8_t)(v > 127 ? 127 : v);
        }
        float d_all = lo_f16_to_f32(hd);
        for (int j = 0; j < 16; j++) {
            float d = d_all * sc[j];
            if (d == 0.0f)
                continue;
            for (int i = 0; i < 16; i++) {
                int l = nearest_int(x[16 * j + i] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + i] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = blk, *qh = blk + 128;
        for (int j = 0; j < LO_QK_K; j += 128) {
            for (int l = 0; l < 32; l++) {
                uint8_t q1 = (uint8_t)L[j + l] & 0xF, q2 = (uint8_t)L[j + l + 32] & 0xF;
                uint8_t q3 = (uint8_t)L[j + l + 64] & 0xF, q4 = (uint8_t)L[j + l + 96] & 0xF;
                ql[l] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)(((uint8_t)L[j + l] >> 4) | (((uint8_t)L[j + l + 32] >> 4) << 2) |
                                  (((uint8_t)L[j + l + 64] >> 4) << 4) |
                                  (((uint8_t)L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}

void lo_quantize_rows(int t, uint8_t *dst, const float *src, size_t rows, size_t cols) {
    size_t rb = lo_row_bytes(t, cols);
    for (size_t r = 0; r < rows; r++) {
        const float *s = src + r * cols;
        uint8_t *d = dst + r * rb;
        switch (t) {
        case LO_Q4_0:
            lo_quantize_q4_0(d, s, cols);
            break;
        case LO_Q8_0:
            lo_quantize_q8_0(d, s, cols);
            break;
        case LO_Q4_K:
            lo_quantize_q4_k(d, s, cols);
            break;
        case LO_Q6_K:
            lo_quantize_q6_k(d, s, cols);
            break;
        case LO_F32:
            memcpy(d, s, cols * 4);
            break;
        case LO_F16:
            for (size_t i = 0; i < cols; i++) {
                uint16_t h = lo_f32_to_f16(s[i]);
                d[2 * i] = (uint8_t)(h & 0xff);
                d[2 * i + 1] = (uint8_t)(h >> 8);
            }
            break;
        default:
            break;
        }
    }
}

/* ---- seeded generators --------------------------------------------------- */

static inline uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline double unit_open(uint64_t *s) { /* (0, 1) */
    return ((double)(splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

void lo_fill_normal(float *dst, size_t n, uint64_t seed, float mean, float stddev) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = unit_open(&s), u2 = unit_open(&s);
        double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
        dst[i] = (float)(mean + stddev * r * cos(th));
        if (i + 1 < n)
            dst[i + 1] = (float)(mean + stddev * r * sin(th));
    }
}

void lo_fill_uniform(float *dst, size_t n, uint64_t seed, float lo, float hi) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++)
        dst[i] = (float)(lo + (hi - lo) * unit_open(&s));
}
