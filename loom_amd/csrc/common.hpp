// common.hpp -- shared definitions for libloomhip (gfx950, wave64).
//
// Device weight layout (per [rows][cols] plane, U = rows * blocks_per_row):
//   Q4_K: GGML's native 144-byte blocks (16-byte aligned already).
//   Q6_K: ql[U][128] | qh[U][64] | scales[U][16] | d[U] (f16, padded to 16 B)
//   Q8_0: qs[U][32] | d[U] (f16, padded to 16 B)
//   Q4_0: qs[U][16] | d[U] (f16, padded to 16 B)
// GGML's 210/34/18-byte blocks are only 2-byte aligned; splitting them per
// plane keeps the byte count and makes every lane's load an aligned 16 bytes.
//
// Quantized activations (the reference's XBlock / XBlockK,
// src/gguf/ggml.zig:738-770), per activation vector of `cols` values:
//   q: int8[cols]; d: f32[cols / QB]; s: i32[cols / 16] (K) or [cols / 32]
// with QB = 256 for the K-quants (quantizeX256) and 32 for Q4_0/Q8_0
// (quantizeX).  Vector v lives at q + v*cols, d + v*(cols/QB), s + v*ns.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define LH_F32 0
#define LH_F16 1
#define LH_Q4_0 2
#define LH_Q8_0 8
#define LH_Q4_K 12
#define LH_Q6_K 14

namespace lh {

__host__ __device__ inline constexpr int block_elems(int t) {
    return (t == LH_Q4_0 || t == LH_Q8_0) ? 32 : (t == LH_Q4_K || t == LH_Q6_K) ? 256 : 1;
}
__host__ __device__ inline constexpr int block_bytes(int t) {
    return t == LH_Q4_0 ? 18 : t == LH_Q8_0 ? 34 : t == LH_Q4_K ? 144 : t == LH_Q6_K ? 210
           : t == LH_F16 ? 2 : 4;
}
__host__ __device__ inline constexpr size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

// Bytes of one plane in the device layout.
__host__ __device__ inline size_t plane_bytes(int t, size_t rows, size_t cols) {
    size_t U = rows * (cols / block_elems(t));
    switch (t) {
    case LH_Q4_K:
        return U * 144;
    case LH_Q6_K:
        return U * 208 + align16(U * 2);
    case LH_Q8_0:
        return U * 32 + align16(U * 2);
    case LH_Q4_0:
        return U * 16 + align16(U * 2);
    case LH_F16:
        return rows * cols * 2;
    default:
        return rows * cols * 4;
    }
}
__host__ __device__ inline size_t ggml_bytes(int t, size_t rows, size_t cols) {
    return rows * (cols / block_elems(t)) * block_bytes(t);
}

// Activation block width used by the weight type's int8 kernel.
__host__ __device__ inline constexpr int act_block(int t) {
    return (t == LH_Q4_K || t == LH_Q6_K) ? 256 : 32;
}
// i32 sums per activation vector: per 16 for K-quants, per 32 otherwise.
__host__ __device__ inline size_t act_sums(int t, size_t cols) {
    return (t == LH_Q4_K || t == LH_Q6_K) ? cols / 16 : cols / 32;
}

// ---- device helpers -------------------------------------------------------

__device__ inline float half_bits_to_float(uint32_t bits16) {
    __half_raw r;
    r.x = (unsigned short)(bits16 & 0xffff);
    return __half2float(__half(r));
}

// exp(x) rounded once to f32: the library's double-precision exponential
// (far below half an f32 ulp of error) then one rounding, so the result is
// the correctly rounded f32 exp except when exp(x) lies within a double ulp
// of an f32 rounding midpoint.  The CPU path's expf is itself within 0.502
// ulp, so the two agree on all but a sliver of inputs.
__device__ inline float exp_f32(float x) { return (float)exp((double)x); }

// The same once-rounded exponential in about twenty double operations (a
// tenth of the library's), for the attention softmax, which evaluates it at
// every position: x = k ln2 + r (Cody-Waite: ln 2 split into a double and its
// remainder, both applied by FMA, |r| <= ln2/2), exp(r) by its Taylor series
// through r^13/13! (truncation below 5e-18 relative) in Horner form with FMA,
// scaled by 2^k.  The double result is within about 1e-16 relative, so after
// the f32 rounding it is the correctly rounded f32 exp except within a few
// double ulps of an f32 rounding midpoint; on the host the same steps equal
// (float)exp((double)x) on every f32 input checked (every seventh bit pattern
// in [-110, 90]).  Inputs at or below -104 round to +0, above 88.8 to +inf.
// Its constants take 26 VGPRs where the compiler hoists them, so kernels
// short of registers keep exp_f32.  exp_f32_core evaluates the input clamped
// into [-104, 88.8] with no branch (NaN becomes -104), exp_f32_fix selects
// the special values; a caller with several independent exponentials
// computes their cores together so the dependent FMA chains interleave.
__device__ inline float exp_f32_core(float xf) {
    const double x = (double)__builtin_fminf(__builtin_fmaxf(xf, -104.0f), 88.8f);
    const double kd = __builtin_rint(x * 0x1.71547652b82fep+0); // x / ln 2
    const double r = __builtin_fma(kd, -0x1.abc9e3b39803fp-56, __builtin_fma(kd, -0x1.62e42fefa39efp-1, x));
    double p = 0x1.6124613a86d09p-33; // 1/13!
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);
    p = __builtin_fma(p, r, 0x1p-1);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return (float)__builtin_ldexp(p, (int)kd);
}
__device__ inline float exp_f32_fix(float xf, float y) {
    return xf > 88.8f ? __builtin_inff() : xf > -104.0f ? y : xf != xf ? xf : 0.0f;
}
__device__ inline float exp_f32_poly(float xf) { return exp_f32_fix(xf, exp_f32_core(xf)); }

// Round half away from zero, saturate at +-127, non-finite -> 0
// (src/gguf/ggml.zig:1067-1073 toI8Saturating).
// Branch-free: round, clamp with med3, then select.
__device__ inline int to_i8_sat(float v) {
    const float r = __builtin_amdgcn_fmed3f(__builtin_roundf(v), -127.0f, 127.0f);
    return __builtin_isfinite(v) ? (int)r : 0;
}

__device__ inline int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// DPP reductions inside groups of 2, 4 and 8 lanes (quad_perm xor1/xor2 and
// row_half_mirror).  Integer sums, so the order does not matter.
__device__ inline int dpp_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ inline int dpp_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }
__device__ inline int dpp_hmirror(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); }

template <int LANES>
__device__ inline int group_sum(int v) {
    if constexpr (LANES >= 2)
        v += dpp_xor1(v);
    if constexpr (LANES >= 4)
        v += dpp_xor2(v);
    if constexpr (LANES >= 8)
        v += dpp_hmirror(v);
    return v;
}

// DPP move of a float (disabled rows keep `old`).
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline float dpp_f(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                      ROW_MASK, 0xF, false));
}

// Wave-wide max, returned uniformly: quad xor 1 and 2, half-row and row
// mirrors, then row_bcast 15 / 31 carry the row maxima up to lane 63.
__device__ inline float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    v = fmaxf(v, dpp_f<0x140>(v, v));
    v = fmaxf(v, dpp_f<0x142, 0xA>(v, v));
    v = fmaxf(v, dpp_f<0x143, 0xC>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over aligned groups of 8 lanes, in every lane of the group.
__device__ inline float group8_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    return v;
}

// Max and sum over aligned groups of 16 lanes (a DPP row), in every lane of
// the row: quad xor 1 and 2, then the half-row and row mirrors.  Each step
// adds a lane's value to its partner's, so every lane holds the same result.
__device__ inline float group16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    v = fmaxf(v, dpp_f<0x140>(v, v));
    return v;
}

__device__ inline float group16_sum(float v) {
    v = v + dpp_f<0xB1>(v, v);
    v = v + dpp_f<0x4E>(v, v);
    v = v + dpp_f<0x141>(v, v);
    v = v + dpp_f<0x140>(v, v);
    return v;
}

// sdot4 over the four dwords of two 16-byte vectors.
__device__ inline int dot16(const int4 &w, const int4 &x, int acc) {
    acc = sdot4(w.x, x.x, acc);
    acc = sdot4(w.y, x.y, acc);
    acc = sdot4(w.z, x.z, acc);
    acc = sdot4(w.w, x.w, acc);
    return acc;
}

__device__ inline int4 and4(const int4 &a, int m) { return make_int4(a.x & m, a.y & m, a.z & m, a.w & m); }
__device__ inline int4 shr4(const int4 &a, int s) {
    return make_int4((int)((unsigned)a.x >> s), (int)((unsigned)a.y >> s), (int)((unsigned)a.z >> s),
                     (int)((unsigned)a.w >> s));
}

__device__ inline uint32_t byte_of(const uint4 &v, int i) {
    uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xff;
}

} // namespace lh
