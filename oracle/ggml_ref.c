/*
 * ggml_ref.c -- TEST INFRASTRUCTURE: restatement of src/gguf/ggml.zig for the
 * formats on this path (Q4_0, Q8_0, Q4_K, Q6_K, F32, F16).
 *
 * Evaluation order of every f32 expression follows the Zig source exactly
 * (left-associative products, no contraction, sequential block sums), so the
 * int8 kernels here are bit-identical to the reference wherever the reference
 * is deterministic.  The one unpinned detail is the lane order of
 * `@reduce(.Add)` over f32 vectors in dotF32 (ggml.zig:214): it is taken as
 * sequential lane order, which is what LLVM's ordered `vector.reduce.fadd`
 * (Zig's strict float mode) produces.
 */
#include "loom_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdbool.h>
#include <stdlib.h>
#include <string.h>

/* ---- formats: ggml.zig:86-153 ------------------------------------------- */

size_t lo_block_elems(int t) {
    switch (t) {
    case LO_Q4_0:
    case LO_Q8_0:
        return LO_QK_0;
    case LO_Q4_K:
    case LO_Q6_K:
        return LO_QK_K;
    default:
        return 1;
    }
}

size_t lo_block_bytes(int t) {
    switch (t) {
    case LO_F32:
        return 4;
    case LO_F16:
        return 2;
    case LO_Q4_0:
        return 18; /* f16 d + 16 nibble bytes */
    case LO_Q8_0:
        return 34; /* f16 d + 32 x i8 */
    case LO_Q4_K:
        return 144; /* d, dmin, 12 B scales, 128 B nibbles */
    case LO_Q6_K:
        return 210; /* ql 128, qh 64, 16 x i8 scales, f16 d */
    default:
        return 0;
    }
}

size_t lo_row_bytes(int t, size_t n) { return (n / lo_block_elems(t)) * lo_block_bytes(t); }

/* ggml.zig:260-263: exact f16 -> f32 widening. */
float lo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                mant <<= 1;
                e++;
            } while ((mant & 0x400u) == 0);
            mant &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> f16 with round-to-nearest-even (Zig @floatCast to f16). */
uint16_t lo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31)
        return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) { /* subnormal or zero in f16 */
        if (e < -10)
            return (uint16_t)sign;
        mant |= 0x800000u;
        int shift = 14 - e;
        uint32_t half = 1u << (shift - 1);
        uint32_t rest = mant & ((1u << shift) - 1);
        uint32_t q = mant >> shift;
        if (rest > half || (rest == half && (q & 1)))
            q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fff;
    if (rest > 0x1000 || (rest == 0x1000 && (q & 1)))
        q++; /* may carry into the exponent, which is the correct result */
    return (uint16_t)(sign | q);
}

static inline float f16_at(const uint8_t *p) { return lo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---- exact dequant: ggml.zig:1332-1471, 1739-1857 ------------------------ */

/* ggml.zig:1332-1340 scaleMinK4 */
static inline void scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ggml.zig:1342-1374: value = (d*sc)*q - (dmin*m), two roundings, no FMA. */
static void dequant_block_q4k(const uint8_t *blk, float *vals) {
    float d = f16_at(blk), dmin = f16_at(blk + 2);
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    for (int p = 0; p < 4; p++) {
        uint8_t sc, mn;
        scale_min_k4(2 * p, scales, &sc, &mn);
        float d1 = d * (float)sc, m1 = dmin * (float)mn;
        scale_min_k4(2 * p + 1, scales, &sc, &mn);
        float d2 = d * (float)sc, m2 = dmin * (float)mn;
        for (int l = 0; l < 32; l++) {
            uint8_t b = qs[32 * p + l];
            vals[64 * p + l] = d1 * (float)(b & 0xF) - m1;
            vals[64 * p + 32 + l] = d2 * (float)(b >> 4) - m2;
        }
    }
}

/* ggml.zig:1420-1471: value = (d*sc)*(q-32), sc signed i8. */
static void dequant_block_q6k(const uint8_t *blk, float *vals) {
    const uint8_t *ql_all = blk, *qh_all = blk + 128;
    const int8_t *sc_all = (const int8_t *)(blk + 192);
    float d = f16_at(blk + 208);
    for (int h = 0; h < 2; h++) {
        const uint8_t *ql = ql_all + 64 * h, *qh = qh_all + 32 * h;
        const int8_t *sc = sc_all + 8 * h;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            float s1 = d * (float)sc[is], s2 = d * (float)sc[is + 2];
            float s3 = d * (float)sc[is + 4], s4 = d * (float)sc[is + 6];
            int q1 = (ql[l] & 0xF) | ((qh[l] & 3) << 4);
            int q2 = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
            int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
            int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
            vals[128 * h + l] = s1 * ((float)q1 - 32.0f);
            vals[128 * h + l + 32] = s2 * ((float)q2 - 32.0f);
            vals[128 * h + l + 64] = s3 * ((float)q3 - 32.0f);
            vals[128 * h + l + 96] = s4 * ((float)q4 - 32.0f);
        }
    }
}

void lo_dequant_row(int t, float *out, const uint8_t *data, size_t r, size_t cols) {
    size_t rb = lo_row_bytes(t, cols);
    const uint8_t *row = data + r * rb;
    switch (t) {
    case LO_F32:
        memcpy(out, row, cols * 4);
        break;
    case LO_F16:
        for (size_t i = 0; i < cols; i++)
            out[i] = f16_at(row + 2 * i);
        break;
    case LO_Q4_K:
        for (size_t b = 0; b * LO_QK_K < cols; b++)
            dequant_block_q4k(row + b * 144, out + b * LO_QK_K);
        break;
    case LO_Q6_K:
        for (size_t b = 0; b * LO_QK_K < cols; b++)
            dequant_block_q6k(row + b * 210, out + b * LO_QK_K);
        break;
    case LO_Q4_0: /* ggml.zig:1834-1843: f32(q - 8) * d */
        for (size_t b = 0; b * LO_QK_0 < cols; b++) {
            const uint8_t *blk = row + b * 18;
            float s = f16_at(blk);
            for (int j = 0; j < 16; j++) {
                out[b * 32 + j] = (float)((int)(blk[2 + j] & 0xF) - 8) * s;
                out[b * 32 + j + 16] = (float)((int)(blk[2 + j] >> 4) - 8) * s;
            }
        }
        break;
    case LO_Q8_0: /* ggml.zig:1845-1849: f32(q) * d */
        for (size_t b = 0; b * LO_QK_0 < cols; b++) {
            const uint8_t *blk = row + b * 34;
            float s = f16_at(blk);
            for (int j = 0; j < 32; j++)
                out[b * 32 + j] = (float)(int8_t)blk[2 + j] * s;
        }
        break;
    default:
        break;
    }
}

/* ---- activation quantizers: ggml.zig:1067-1098, 776-800 ----------------- */

/* ggml.zig:1067-1073: round half away from zero, saturate at +-127, non-finite -> 0. */
int8_t lo_to_i8_saturating(float v) {
    if (!isfinite(v))
        return 0;
    float r = roundf(v);
    if (r >= 127.0f)
        return 127;
    if (r <= -127.0f)
        return -127;
    return (int8_t)(int)r;
}

/* ggml.zig:1077-1098 quantizeX: per 32 values, d = amax/127, q = rnd(x*(1/d)). */
void lo_quantize_x(const float *x, size_t n, lo_xblock *out) {
    size_t nb = n / LO_QK_0;
    for (size_t b = 0; b < nb; b++) {
        const float *src = x + b * LO_QK_0;
        float amax = 0.0f;
        for (int i = 0; i < LO_QK_0; i++)
            if (isfinite(src[i]))
                amax = fmaxf(amax, fabsf(src[i]));
        float d = amax / 127.0f;
        float inv = (d != 0.0f && isfinite(d)) ? 1.0f / d : 0.0f;
        int32_t sum = 0;
        for (int i = 0; i < LO_QK_0; i++) {
            int8_t q = lo_to_i8_saturating(src[i] * inv);
            out[b].q[i] = q;
            sum += q;
        }
        out[b].d = isfinite(d) ? d : 0.0f;
        out[b].sum = sum;
    }
}

/* ggml.zig:776-800 quantizeX256: one scale per 256 values, per-16 sums. */
void lo_quantize_x256(const float *x, size_t n, lo_xblockk *out) {
    size_t nb = n / LO_QK_K;
    for (size_t b = 0; b < nb; b++) {
        const float *src = x + b * LO_QK_K;
        float amax = 0.0f;
        for (int i = 0; i < LO_QK_K; i++)
            if (isfinite(src[i]))
                amax = fmaxf(amax, fabsf(src[i]));
        float d = amax / 127.0f;
        float inv = (d != 0.0f && isfinite(d)) ? 1.0f / d : 0.0f;
        for (int s = 0; s < 16; s++) {
            int32_t sum = 0;
            for (int i = 0; i < 16; i++) {
                int8_t q = lo_to_i8_saturating(src[s * 16 + i] * inv);
                out[b].q[s * 16 + i] = q;
                sum += q;
            }
            out[b].bsum[s] = sum;
        }
        out[b].d = isfinite(d) ? d : 0.0f;
    }
}

/* ---- f32 dot: ggml.zig:198-217 ------------------------------------------ */

/* Four accumulators of eight lanes; per lane ((a0+a1)+a2)+a3, then the eight
 * lanes summed in order, then the scalar tail. */
float lo_dot_f32(const float *a, const float *b, size_t n) {
    float acc[4][8] = {{0}};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int v = 0; v < 4; v++)
            for (int l = 0; l < 8; l++) {
                float p = a[i + 8 * v + l] * b[i + 8 * v + l];
                acc[v][l] = acc[v][l] + p;
            }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            float p = a[i + l] * b[i + l];
            acc[0][l] = acc[0][l] + p;
        }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) {
        float lane = ((acc[0][l] + acc[1][l]) + acc[2][l]) + acc[3][l];
        s = s + lane;
    }
    for (; i < n; i++) {
        float p = a[i] * b[i];
        s = s + p;
    }
    return s;
}

/* ggml.zig:221-230: out += w * v, per element o + w*v. */
void lo_axpy(float *out, const float *v, float w, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float p = w * v[i];
        out[i] = out[i] + p;
    }
}

/* ---- K-quant decode + block dot: ggml.zig:882-1020 ----------------------- */

typedef struct {
    int8_t ws[256];
    int32_t scs[16];
    int32_t mns[16];
    float d, dmin;
} kdec;

static void kdecode(int t, const uint8_t *blk, kdec *dec) {
    if (t == LO_Q4_K) { /* ggml.zig:886-916 */
        dec->d = f16_at(blk);
        dec->dmin = f16_at(blk + 2);
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        for (int j = 0; j < 8; j++) {
            uint8_t sc, mn;
            scale_min_k4(j, scales, &sc, &mn);
            dec->scs[2 * j] = dec->scs[2 * j + 1] = sc;
            dec->mns[2 * j] = dec->mns[2 * j + 1] = mn;
            const uint8_t *src = qs + (j / 2) * 32;
            for (int i = 0; i < 32; i++)
                dec->ws[32 * j + i] = (int8_t)((j & 1) ? (src[i] >> 4) : (src[i] & 0xF));
        }
    } else { /* Q6_K: ggml.zig:919-948 */
        const uint8_t *ql_all = blk, *qh_all = blk + 128;
        dec->d = f16_at(blk + 208);
        dec->dmin = 0.0f;
        for (int j = 0; j < 16; j++) {
            dec->scs[j] = (int8_t)blk[192 + j];
            dec->mns[j] = 0;
        }
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = ql_all + 64 * h, *qh = qh_all + 32 * h;
            for (int l = 0; l < 32; l++) {
                int g0 = (ql[l] & 0xF) | ((qh[l] & 3) << 4);
                int g1 = (ql[32 + l] & 0xF) | (((qh[l] >> 2) & 3) << 4);
                int g2 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
                int g3 = (ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4);
                dec->ws[128 * h + l] = (int8_t)(g0 - 32);
                dec->ws[128 * h + 32 + l] = (int8_t)(g1 - 32);
                dec->ws[128 * h + 64 + l] = (int8_t)(g2 - 32);
                dec->ws[128 * h + 96 + l] = (int8_t)(g3 - 32);
            }
        }
    }
}

/* ggml.zig:1002-1020 kBlockDot: integer until one f32 tail. */
static inline float kblock_dot(int t, const kdec *dec, const lo_xblockk *xb) {
    int32_t isum = 0;
    for (int s = 0; s < 16; s++) {
        int32_t dot = 0;
        for (int i = 0; i < 16; i++)
            dot += (int32_t)dec->ws[16 * s + i] * (int32_t)xb->q[16 * s + i];
        isum += dot * dec->scs[s];
    }
    if (t == LO_Q4_K) {
        int32_t min_isum = 0;
        for (int j = 0; j < 16; j++)
            min_isum += dec->mns[j] * xb->bsum[j];
        float a = dec->d * (float)isum;
        float b = dec->dmin * (float)min_isum;
        return xb->d * (a - b);
    }
    float s = xb->d * dec->d;
    return s * (float)isum;
}

/* ggml.zig:1024-1038 matvecK256 */
static void matvec_k256(int t, float *out, const uint8_t *data, const lo_xblockk *qx, size_t rows,
                        size_t cols) {
    size_t bs = lo_block_bytes(t), nb = cols / LO_QK_K, rb = nb * bs;
    kdec dec;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = data + r * rb;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            kdecode(t, row + b * bs, &dec);
            acc = acc + kblock_dot(t, &dec, &qx[b]);
        }
        out[r] = acc;
    }
}

/* ggml.zig:1196-1222 matvecQ40Int */
static void matvec_q40(float *out, const uint8_t *data, const lo_xblock *qx, size_t rows,
                       size_t cols) {
    size_t nb = cols / LO_QK_0, rb = nb * 18;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = data + r * rb;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * 18;
            float d = f16_at(blk);
            const uint8_t *qs = blk + 2;
            int32_t dot = 0, sum = 0;
            for (int i = 0; i < 16; i++) {
                int32_t lo = qs[i] & 0xF, hi = qs[i] >> 4;
                dot += lo * qx[b].q[i] + hi * qx[b].q[i + 16];
                sum += qx[b].q[i] + qx[b].q[i + 16];
            }
            float s = d * qx[b].d;
            acc = acc + s * (float)(dot - 8 * sum);
        }
        out[r] = acc;
    }
}

/* ggml.zig:1277-1294 matvecQ80Int */
static void matvec_q80(float *out, const uint8_t *data, const lo_xblock *qx, size_t rows,
                       size_t cols) {
    size_t nb = cols / LO_QK_0, rb = nb * 34;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = data + r * rb;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * 34;
            float d = f16_at(blk);
            const int8_t *w = (const int8_t *)(blk + 2);
            int32_t dot = 0;
            for (int i = 0; i < 32; i++)
                dot += (int32_t)w[i] * (int32_t)qx[b].q[i];
            float s = d * qx[b].d;
            acc = acc + s * (float)dot;
        }
        out[r] = acc;
    }
}

/* ggml.zig:1545-1551 matvecF32 */
static void matvec_f32(float *out, const uint8_t *data, const float *x, size_t rows, size_t cols) {
    const float *w = (const float *)data;
    for (size_t r = 0; r < rows; r++)
        out[r] = lo_dot_f32(w + r * cols, x, cols);
}

/* F16 rows: widen then dot (the reference's f16 kernel; not on this path's
 * timed configs, kept for dequant/embedding completeness). */
static void matvec_f16(float *out, const uint8_t *data, const float *x, size_t rows, size_t cols) {
    float *tmp = (float *)malloc(cols * sizeof(float));
    for (size_t r = 0; r < rows; r++) {
        lo_dequant_row(LO_F16, tmp, data, r, cols);
        out[r] = lo_dot_f32(tmp, x, cols);
    }
    free(tmp);
}

/* Rows [r0, r1) of one matvec, with the activation already quantized. */
typedef struct {
    int t;
    float *out;
    const uint8_t *data;
    const float *x;
    const void *qx; /* lo_xblock* or lo_xblockk* (per lane when n > 1) */
    size_t n, rows, cols;
} job_t;

static void run_rows(const job_t *j, size_t r0, size_t r1) {
    size_t rb = lo_row_bytes(j->t, j->cols);
    if (j->n > 1) { /* batched kernels: ggml.zig:566-598, 1044-1059 */
        size_t nb = j->cols / lo_block_elems(j->t);
        if (j->t == LO_Q8_0) {
            const lo_xblock *qx = (const lo_xblock *)j->qx; /* [lane][nb] */
            for (size_t r = r0; r < r1; r++) {
                const uint8_t *row = j->data + r * rb;
                float acc[LO_MAX_BATCH] = {0};
                for (size_t b = 0; b < nb; b++) {
                    const uint8_t *blk = row + b * 34;
                    float d = f16_at(blk);
                    const int8_t *w = (const int8_t *)(blk + 2);
                    for (size_t k = 0; k < j->n; k++) {
                        const lo_xblock *xb = &qx[k * nb + b];
                        int32_t dot = 0;
                        for (int i = 0; i < 32; i++)
                            dot += (int32_t)w[i] * (int32_t)xb->q[i];
                        float s = d * xb->d;
                        acc[k] = acc[k] + s * (float)dot;
                    }
                }
                for (size_t k = 0; k < j->n; k++)
                    j->out[k * j->rows + r] = acc[k];
            }
        } else {
            const lo_xblockk *qx = (const lo_xblockk *)j->qx;
            size_t bs = lo_block_bytes(j->t);
            kdec dec;
            for (size_t r = r0; r < r1; r++) {
                const uint8_t *row = j->data + r * rb;
                float acc[LO_MAX_BATCH] = {0};
                for (size_t b = 0; b < nb; b++) {
                    kdecode(j->t, row + b * bs, &dec);
                    for (size_t k = 0; k < j->n; k++)
                        acc[k] = acc[k] + kblock_dot(j->t, &dec, &qx[k * nb + b]);
                }
                for (size_t k = 0; k < j->n; k++)
                    j->out[k * j->rows + r] = acc[k];
            }
        }
        return;
    }
    const uint8_t *d = j->data + r0 * rb;
    float *o = j->out + r0;
    size_t rows = r1 - r0;
    switch (j->t) {
    case LO_Q4_K:
    case LO_Q6_K:
        matvec_k256(j->t, o, d, (const lo_xblockk *)j->qx, rows, j->cols);
        break;
    case LO_Q4_0:
        matvec_q40(o, d, (const lo_xblock *)j->qx, rows, j->cols);
        break;
    case LO_Q8_0:
        matvec_q80(o, d, (const lo_xblock *)j->qx, rows, j->cols);
        break;
    case LO_F32:
        matvec_f32(o, d, j->x, rows, j->cols);
        break;
    case LO_F16:
        matvec_f16(o, d, j->x, rows, j->cols);
        break;
    default:
        break;
    }
}

/* ---- worker pool: ggml.zig:279-399, row split 602-639 --------------------- */

#define MAX_WORKERS 32
#define MIN_ROWS_PER_THREAD 64
#define SPIN_BEFORE_YIELD 40000

static struct {
    int n; /* live workers (excluding the caller) */
    pthread_t threads[MAX_WORKERS];
    atomic_bool quit;
    atomic_ulong seq;
    atomic_ulong active;
    atomic_ulong cursor;
    job_t job;
    size_t chunk;
} pool;

static void run_chunks(void) {
    for (;;) {
        size_t start = atomic_fetch_add(&pool.cursor, pool.chunk);
        if (start >= pool.job.rows)
            return;
        size_t end = start + pool.chunk;
        if (end > pool.job.rows)
            end = pool.job.rows;
        run_rows(&pool.job, start, end);
    }
}

static void *worker(void *arg) {
    (void)arg;
    unsigned long seen = 0;
    unsigned idle = 0;
    for (;;) {
        unsigned long s = atomic_load(&pool.seq);
        if (s == seen) {
            if (atomic_load(&pool.quit))
                return NULL;
            if (++idle >= SPIN_BEFORE_YIELD)
                sched_yield();
            continue;
        }
        idle = 0;
        seen = s;
        if (atomic_load(&pool.quit))
            return NULL;
        run_chunks();
        atomic_fetch_sub(&pool.active, 1);
    }
}

void lo_parallel_begin(int n) {
    if (pool.n != 0)
        return;
    int want = n < MAX_WORKERS ? n : MAX_WORKERS;
    if (want <= 1)
        return;
    atomic_store(&pool.quit, false);
    atomic_store(&pool.seq, 0);
    atomic_store(&pool.active, 0);
    int started = 0;
    while (started + 1 < want) {
        if (pthread_create(&pool.threads[started], NULL, worker, NULL) != 0)
            break;
        started++;
    }
    pool.n = started;
}

void lo_parallel_end(void) {
    if (pool.n == 0)
        return;
    atomic_store(&pool.quit, true);
    atomic_fetch_add(&pool.seq, 1);
    for (int i = 0; i < pool.n; i++)
        pthread_join(pool.threads[i], NULL);
    pool.n = 0;
}

int lo_parallel_threads(void) { return pool.n + 1; }

static void submit(const job_t *j) {
    int workers = pool.n;
    if (workers == 0 || j->rows < 2 * MIN_ROWS_PER_THREAD) {
        run_rows(j, 0, j->rows);
        return;
    }
    size_t parts = (size_t)(workers + 1) * 2;
    size_t per = (j->rows + parts - 1) / parts;
    if (per < MIN_ROWS_PER_THREAD)
        per = MIN_ROWS_PER_THREAD;
    pool.job = *j;
    pool.chunk = per;
    atomic_store(&pool.cursor, 0);
    atomic_store(&pool.active, (unsigned long)workers);
    atomic_fetch_add(&pool.seq, 1);
    run_chunks();
    unsigned spins = 0;
    while (atomic_load(&pool.active) != 0)
        if (++spins >= SPIN_BEFORE_YIELD)
            sched_yield();
}

/* ggml.zig:602-639 matvec: quantize x once, then row-parallel dispatch. */
void lo_matvec(int t, float *out, const uint8_t *w, const float *x, size_t rows, size_t cols) {
    job_t j = {t, out, w, x, NULL, 1, rows, cols};
    void *qx = NULL;
    if (t == LO_Q4_K || t == LO_Q6_K) {
        qx = malloc((cols / LO_QK_K) * sizeof(lo_xblockk));
        lo_quantize_x256(x, cols, (lo_xblockk *)qx);
    } else if (t == LO_Q4_0 || t == LO_Q8_0) {
        qx = malloc((cols / LO_QK_0) * sizeof(lo_xblock));
        lo_quantize_x(x, cols, (lo_xblock *)qx);
    }
    j.qx = qx;
    submit(&j);
    free(qx);
}

/* ggml.zig:504-562 matmul: batched kernels for n <= 8 on the K-quants and
 * Q8_0, otherwise n separate matvecs.  Bit-identical to n matvecs. */
void lo_matmul(int t, float *out, const uint8_t *w, const float *xs, size_t n, size_t rows,
               size_t cols) {
    if (n == 0)
        return;
    int batched = (t == LO_Q4_K || t == LO_Q6_K || t == LO_Q8_0);
    if (n == 1 || !batched || n > LO_MAX_BATCH) {
        for (size_t k = 0; k < n; k++)
            lo_matvec(t, out + k * rows, w, xs + k * cols, rows, cols);
        return;
    }
    void *qx;
    if (t == LO_Q8_0) {
        size_t nb = cols / LO_QK_0;
        qx = malloc(n * nb * sizeof(lo_xblock));
        for (size_t k = 0; k < n; k++)
            lo_quantize_x(xs + k * cols, cols, (lo_xblock *)qx + k * nb);
    } else {
        size_t nb = cols / LO_QK_K;
        qx = malloc(n * nb * sizeof(lo_xblockk));
        for (size_t k = 0; k < n; k++)
            lo_quantize_x256(xs + k * cols, cols, (lo_xblockk *)qx + k * nb);
    }
    job_t j = {t, out, w, xs, qx, n, rows, cols};
    submit(&j);
    free(qx);
}
