// formats.hip -- activation quantizers, exact dequant, GGML->device repack and
// the synthetic weight generator.
#include "device.hpp"

namespace lh {

// ---- activation quantizers (one wave per item, device.hpp) -----------------------

__global__ __launch_bounds__(64) void quant_act_kernel(int wt, const float *__restrict__ x,
                                                       int cols, int x_stride, QAct qa) {
    quant_item_wave(wt, x + (size_t)blockIdx.y * x_stride, cols, blockIdx.y, blockIdx.x, qa);
}

void launch_quant_act(int wtype, const float *x, int cols, int x_stride, int nvec, QAct qa,
                      hipStream_t st) {
    hipLaunchKernelGGL(quant_act_kernel, dim3(quant_items(wtype, cols), nvec), dim3(64), 0, st,
                       wtype, x, cols, x_stride, qa);
    note_launch();
}

// ---- exact dequant from the device layout ---------------------------------
// One thread per value (dequant_value, device.hpp).

__global__ void dequant_kernel(int t, const uint8_t *__restrict__ w, size_t rows, size_t cols,
                               float *__restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * cols)
        return;
    out[idx] = dequant_value(t, w, rows, cols, idx / cols, idx % cols);
}

void launch_dequant(int t, const void *w, size_t rows, size_t cols, float *out, hipStream_t st) {
    const size_t n = rows * cols;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, t,
                       (const uint8_t *)w, rows, cols, out);
    note_launch();
}

// ---- GGML -> device layout -------------------------------------------------
// One thread per block; planes are independent.

__global__ void repack_kernel(int t, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              size_t U, size_t src_plane, size_t dst_plane, size_t planes) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= U * planes)
        return;
    const size_t p = idx / U, u = idx % U;
    const uint8_t *s = src + p * src_plane + u * block_bytes(t);
    uint8_t *d = dst + p * dst_plane;
    if (t == LH_Q6_K) {
        for (int i = 0; i < 128; i++) d[u * 128 + i] = s[i];
        for (int i = 0; i < 64; i++) d[U * 128 + u * 64 + i] = s[128 + i];
        for (int i = 0; i < 16; i++) d[U * 192 + u * 16 + i] = s[192 + i];
        d[U * 208 + 2 * u] = s[208];
        d[U * 208 + 2 * u + 1] = s[209];
    } else if (t == LH_Q8_0) {
        for (int i = 0; i < 32; i++) d[u * 32 + i] = s[2 + i];
        d[U * 32 + 2 * u] = s[0];
        d[U * 32 + 2 * u + 1] = s[1];
    } else if (t == LH_Q4_0) {
        for (int i = 0; i < 16; i++) d[u * 16 + i] = s[2 + i];
        d[U * 16 + 2 * u] = s[0];
        d[U * 16 + 2 * u + 1] = s[1];
    }
}

void launch_repack(int t, const void *src, void *dst, size_t rows, size_t cols, size_t planes,
                   hipStream_t st) {
    const size_t U = rows * (cols / block_elems(t));
    const size_t sp = ggml_bytes(t, rows, cols), dp = plane_bytes(t, rows, cols);
    if (t == LH_Q4_K || t == LH_F32 || t == LH_F16) {
        (void)hipMemcpyAsync(dst, src, sp * planes, hipMemcpyDeviceToDevice, st);
        return;
    }
    const size_t n = U * planes;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, t,
                       (const uint8_t *)src, (uint8_t *)dst, U, sp, dp, planes);
    note_launch();
}

// Planes whose GGML rows start src_plane bytes apart (a per-head slice of a
// fused tensor): the same per-block copy, plane by plane.
void launch_repack_strided(int t, const void *src, size_t src_plane, void *dst, size_t rows, size_t cols,
                           size_t planes, hipStream_t st) {
    const size_t U = rows * (cols / block_elems(t));
    const size_t sp = ggml_bytes(t, rows, cols), dp = plane_bytes(t, rows, cols);
    if (t == LH_Q4_K || t == LH_F32 || t == LH_F16) {
        (void)hipMemcpy2DAsync(dst, dp, src, src_plane, sp, planes, hipMemcpyDeviceToDevice, st);
        return;
    }
    const size_t n = U * planes;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, t,
                       (const uint8_t *)src, (uint8_t *)dst, U, src_plane, dp, planes);
    note_launch();
}

// ---- synthetic weights ------------------------------------------------------
// Counter-based hash per (seed, plane, unit, word): deterministic and
// independent of launch shape.

__device__ inline uint32_t mix32(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33;
    x *= 0xc4ceb9fe1a85ec53ull;
    x ^= x >> 33;
    return (uint32_t)x;
}

__device__ inline uint16_t f2h_bits(float f) {
    __half h = __float2half(f);
    return __half_raw(h).x;
}

// Blocks are written in GGML layout (the bytes a GGUF file holds); callers
// repack them into the device layout.
__global__ void synth_kernel(int t, uint8_t *__restrict__ dst, size_t U, size_t plane_b,
                             size_t planes, uint64_t seed, float stddev) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= U * planes)
        return;
    const size_t p = idx / U, u = idx % U;
    uint8_t *blk = dst + p * plane_b + u * block_bytes(t);
    const uint64_t key = (seed * 0x9E3779B97F4A7C15ull) ^ (idx * 0xD1B54A32D192ED03ull);
    auto word = [&](int i) { return mix32(key + (uint64_t)i * 0x632BE59BD9B4E019ull); };
    auto put4 = [&](int off, uint32_t r) {
        blk[off] = r & 0xff;
        blk[off + 1] = (r >> 8) & 0xff;
        blk[off + 2] = (r >> 16) & 0xff;
        blk[off + 3] = r >> 24;
    };
    if (t == LH_Q4_K) {
        // value = d*sc*q - dmin*m with q uniform 0..15: std ~ d*sc*4.6
        const float dd = stddev / (4.6f * 52.0f);
        const uint16_t hd = f2h_bits(dd), hm = f2h_bits(dd * 7.5f);
        blk[0] = hd & 0xff; blk[1] = hd >> 8; blk[2] = hm & 0xff; blk[3] = hm >> 8;
        const uint32_t r0 = word(0), r1 = word(1), r2 = word(2);
        for (int j = 0; j < 12; j++) {
            const uint32_t r = j < 4 ? r0 : j < 8 ? r1 : r2;
            blk[4 + j] = (uint8_t)(0x28 | ((r >> (8 * (j & 3))) & 0xD7)); // scales 40..63, mins alike
        }
        for (int i = 0; i < 32; i++)
            put4(16 + 4 * i, word(3 + i));
    } else if (t == LH_Q6_K) {
        for (int i = 0; i < 48; i++) // ql[128] then qh[64]
            put4(4 * i, word(i));
        for (int i = 0; i < 4; i++) {
            const uint32_t r = word(48 + i);
            for (int k = 0; k < 4; k++) { // signed scales with |sc| in 64..127
                const uint8_t b = (r >> (8 * k)) & 0xff;
                const int v = 64 + (b & 63);
                blk[192 + 4 * i + k] = (uint8_t)(int8_t)((b & 0x80) ? -v : v);
            }
        }
        const uint16_t hd = f2h_bits(stddev / (18.5f * 96.0f));
        blk[208] = hd & 0xff;
        blk[209] = hd >> 8;
    } else if (t == LH_Q8_0) {
        const uint16_t hd = f2h_bits(stddev / 73.0f);
        blk[0] = hd & 0xff;
        blk[1] = hd >> 8;
        for (int i = 0; i < 8; i++) {
            const uint32_t r = word(i);
            for (int k = 0; k < 4; k++) {
                const int8_t v = (int8_t)((r >> (8 * k)) & 0xff);
                blk[2 + 4 * i + k] = (uint8_t)(v == -128 ? -127 : v);
            }
        }
    } else if (t == LH_Q4_0) {
        const uint16_t hd = f2h_bits(stddev / 4.6f);
        blk[0] = hd & 0xff;
        blk[1] = hd >> 8;
        for (int i = 0; i < 4; i++) {
            const uint32_t r = word(i);
            for (int k = 0; k < 4; k++)
                blk[2 + 4 * i + k] = (r >> (8 * k)) & 0xff;
        }
    }
}

void launch_synth(int t, void *dst, size_t rows, size_t cols, size_t planes, uint64_t seed,
                  float stddev, hipStream_t st) {
    const size_t U = rows * (cols / block_elems(t));
    const size_t n = U * planes;
    hipLaunchKernelGGL(synth_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, t,
                       (uint8_t *)dst, U, ggml_bytes(t, rows, cols), planes, seed, stddev);
    note_launch();
}

} // namespace lh
