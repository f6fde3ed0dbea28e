// seam_frame.hip -- the compute seam's device K/V cache and frame calls over
// host buffers (src/compute/backend.zig:121-160,186-191): attnInit /
// kvAppend / hasKvCache / releaseKvCache / attnHeads, the recorded dense
// frame of llama.zig:1067-1108 (beginFrame, frameLoadX, layerBlock x
// n_layers, endFrame, frameStoreX), and the GQA+MoE whole token in the shape
// of mlaTokenFrame, with the K/V read-back that keeps the engine's host cache
// authoritative.  Every layer runs through the device frame's own per-layer
// code (frame.hip frame_layer) in PARITY numerics, so one step through the
// seam is the engine's llama.step bit for bit.
//
// Host side: one sequence, one fp16 cache [n_layers][ctx][kvd] on the device,
// a pinned staging area for the per-call inputs and outputs, and a pinned
// mirror of the rows the last frame wrote.
#include "frame_host.hpp"

#include <cstring>
#include <mutex>
#include <vector>

namespace lh {

// kvAppend's conversion: the rounding the frame's own append makes
// (__float2half, round to nearest even).
__global__ __launch_bounds__(256) void kv_put_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                     int kvd, uint16_t *__restrict__ kc_row,
                                                     uint16_t *__restrict__ vc_row) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < kvd) {
        kc_row[i] = __half_raw(__float2half(k[i])).x;
        vc_row[i] = __half_raw(__float2half(v[i])).x;
    }
}

// The exact widening of an IEEE binary16 to binary32.
static float half_bits_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        const float f = (float)m * 0x1p-24f; // subnormal or zero: m * 2^-24, exact
        bits = s | __builtin_bit_cast(uint32_t, f);
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112u) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, bits);
}

namespace {

struct SeamKv {
    size_t layers = 0, ctx = 0, kvd = 0;
    uint16_t *k = nullptr, *v = nullptr; // device [layers][ctx][kvd]
    // the rows of the last frame's position, pinned host [layers][kvd] each
    uint16_t *mk = nullptr, *mv = nullptr;
    size_t mirror_pos = SIZE_MAX;
};

// Pinned staging: the call's inputs go out and its outputs come back
// through here, so every copy is asynchronous on the library's stream.
struct Pinned {
    void *ptr = nullptr;
    size_t cap = 0;
    int reserve(size_t bytes) {
        if (bytes <= cap)
            return LOOMHIP_OK;
        if (ptr) {
            (void)hipStreamSynchronize(g_ctx.compute);
            (void)hipHostFree(ptr);
            ptr = nullptr;
            cap = 0;
        }
        if (hipError_t e = hipHostMalloc(&ptr, bytes); e != hipSuccess) {
            ptr = nullptr;
            return hip_fail(e, "hipHostMalloc seam staging");
        }
        cap = bytes;
        return LOOMHIP_OK;
    }
};

struct SeamFrame {
    bool open = false, loaded = false;
    size_t dim = 0, pos = SIZE_MAX; // the frame's residual width and position
    bool wrote = false;             // a layer ran (its rows go to the mirror at end_frame)
};

std::mutex g_mu;
SeamKv g_kv;
SeamFrame g_sf;
Scratch g_x;      // the frame's residual stream [dim]
Scratch g_io;     // device staging: positions, q, scores, logits
Pinned g_pin_in;  // host -> device
Pinned g_pin_out; // device -> host

int kv_ready(const char *who) {
    if (!g_kv.k)
        return fail(LOOMHIP_DECLINED, "%s: no device K/V cache (attnInit first)", who);
    return LOOMHIP_OK;
}

void release_kv_locked() {
    if (!g_kv.k && !g_kv.mk)
        return;
    if (g_ctx.ready)
        (void)hipStreamSynchronize(g_ctx.compute);
    (void)hipFree(g_kv.k);
    (void)hipFree(g_kv.v);
    (void)hipHostFree(g_kv.mk);
    (void)hipHostFree(g_kv.mv);
    g_kv = SeamKv{};
}

// The rows at pos of every layer, to the pinned mirror (enqueued).
int mirror_rows(size_t pos, hipStream_t st) {
    const size_t rb = g_kv.kvd * 2, pitch = g_kv.ctx * rb;
    hipError_t e = hipMemcpy2DAsync(g_kv.mk, rb, g_kv.k + pos * g_kv.kvd, pitch, rb, g_kv.layers,
                                    hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(g_kv.mv, rb, g_kv.v + pos * g_kv.kvd, pitch, rb, g_kv.layers, hipMemcpyDeviceToHost,
                             st);
    if (e != hipSuccess)
        return hip_fail(e, "kv mirror copy");
    g_kv.mirror_pos = pos;
    return LOOMHIP_OK;
}

bool ref_ok(const loomhip_weight_ref &r, size_t rows, size_t cols, size_t planes = 1) {
    return r.data && r.len == ggml_bytes(r.type, rows, cols) * planes;
}

int upload_ref(const loomhip_weight_ref &r, size_t rows, size_t cols, size_t planes, const void **dev) {
    void *d = nullptr;
    if (int rc = upload_weights(r.type, r.data, rows, cols, planes, &d))
        return rc;
    *dev = d;
    return LOOMHIP_OK;
}

int upload_f32(const float *h, size_t n, const float **dev) {
    void *d = nullptr;
    if (int rc = upload_weights(LH_F32, h, 1, n, 1, &d))
        return rc;
    *dev = (const float *)d;
    return LOOMHIP_OK;
}

// A model shell with the cache's dims for the frame's checks and set-up.
loomhip_model shell(size_t dim, size_t hd, size_t n_heads, size_t n_kv, size_t rope_dim, float rope_base, float eps,
                    int rope_neox) {
    loomhip_model m{};
    m.dim = dim;
    m.head_dim = hd;
    m.n_layers = g_kv.layers;
    m.n_heads = n_heads;
    m.n_kv_heads = n_kv;
    m.ctx_len = g_kv.ctx;
    m.rope_dim = rope_dim;
    m.rope_base = rope_base;
    m.eps = eps;
    m.rope_neox = rope_neox;
    m.numerics = LOOMHIP_NUMERICS_PARITY;
    return m;
}

int put_pos(size_t pos, int32_t **dpos, hipStream_t st) {
    // the position (device int32) from the pinned staging, ordered before
    // the kernels that read it
    if (int rc = g_io.reserve(256))
        return rc;
    if (int rc = g_pin_in.reserve(256))
        return rc;
    *(int32_t *)g_pin_in.ptr = (int32_t)pos;
    *dpos = (int32_t *)g_io.ptr;
    if (hipError_t e = hipMemcpyAsync(*dpos, g_pin_in.ptr, 4, hipMemcpyHostToDevice, st); e != hipSuccess)
        return hip_fail(e, "position upload");
    return LOOMHIP_OK;
}

} // namespace

void seam_release() {
    std::lock_guard<std::mutex> lk(g_mu);
    release_kv_locked();
    g_sf = SeamFrame{};
    g_x.release();
    g_io.release();
    for (Pinned *p : {&g_pin_in, &g_pin_out}) {
        (void)hipHostFree(p->ptr);
        *p = Pinned{};
    }
}

} // namespace lh

using namespace lh;

extern "C" {

int loomhip_attn_init(size_t layers, size_t ctx_len, size_t kvd) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (layers == 0 || kvd == 0 || ctx_len == 0 || ctx_len > (size_t)EXACT_MAX_CTX)
        return fail(LOOMHIP_DECLINED, "attn_init: %zu layers x %zu positions x %zu not served (contexts up to %d)",
                    layers, ctx_len, kvd, EXACT_MAX_CTX);
    if (g_sf.open)
        return fail(LOOMHIP_ERR_ARG, "attn_init: a frame is open");
    release_kv_locked();
    const size_t bytes = layers * ctx_len * kvd * 2;
    void *k = nullptr, *v = nullptr;
    hipError_t e = hipMalloc(&k, bytes);
    if (e == hipSuccess)
        e = hipMalloc(&v, bytes);
    if (e == hipSuccess)
        e = hipMemsetAsync(k, 0, bytes, g_ctx.compute);
    if (e == hipSuccess)
        e = hipMemsetAsync(v, 0, bytes, g_ctx.compute);
    void *mk = nullptr, *mv = nullptr;
    if (e == hipSuccess)
        e = hipHostMalloc(&mk, layers * kvd * 2);
    if (e == hipSuccess)
        e = hipHostMalloc(&mv, layers * kvd * 2);
    if (e == hipSuccess)
        e = hipStreamSynchronize(g_ctx.compute);
    if (e != hipSuccess) {
        (void)hipFree(k);
        (void)hipFree(v);
        (void)hipHostFree(mk);
        (void)hipHostFree(mv);
        return hip_fail(e, "attn_init");
    }
    g_kv.layers = layers;
    g_kv.ctx = ctx_len;
    g_kv.kvd = kvd;
    g_kv.k = (uint16_t *)k;
    g_kv.v = (uint16_t *)v;
    g_kv.mk = (uint16_t *)mk;
    g_kv.mv = (uint16_t *)mv;
    g_kv.mirror_pos = SIZE_MAX;
    return LOOMHIP_OK;
}

int loomhip_has_kv_cache(void) { return g_kv.k != nullptr; }

void loomhip_release_kv_cache(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_sf.open)
        release_kv_locked();
}

int loomhip_kv_append(size_t li, size_t pos, const float *k_new, const float *v_new, size_t kvd) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = kv_ready("kv_append"))
        return rc;
    if (!k_new || !v_new || li >= g_kv.layers || pos >= g_kv.ctx || kvd != g_kv.kvd)
        return fail(LOOMHIP_DECLINED, "kv_append: layer %zu / position %zu / %zu values outside the cache", li,
                    pos, kvd);
    if (g_sf.open) // the frame writes its own rows; its staging is in use
        return fail(LOOMHIP_ERR_ARG, "kv_append: a frame is open");
    hipStream_t st = g_ctx.compute;
    if (int rc = g_pin_in.reserve(kvd * 8))
        return rc;
    if (int rc = g_io.reserve(kvd * 8))
        return rc;
    // the previous call's copies out of the staging have finished (every
    // seam call but the frame's layers ends synchronised)
    memcpy(g_pin_in.ptr, k_new, kvd * 4);
    memcpy((float *)g_pin_in.ptr + kvd, v_new, kvd * 4);
    float *d = (float *)g_io.ptr;
    hipError_t e = hipMemcpyAsync(d, g_pin_in.ptr, kvd * 8, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "kv_append upload");
    const size_t row = (li * g_kv.ctx + pos) * kvd;
    hipLaunchKernelGGL(kv_put_kernel, dim3((kvd + 255) / 256), dim3(256), 0, st, d, d + kvd, (int)kvd, g_kv.k + row,
                       g_kv.v + row);
    note_launch();
    if (pos == g_kv.mirror_pos)
        g_kv.mirror_pos = SIZE_MAX; // the mirror no longer holds this position's rows
    e = hipStreamSynchronize(st);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "kv_append");
}

int loomhip_read_kv(size_t li, size_t pos, float *k_out, float *v_out, size_t kvd) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = kv_ready("read_kv"))
        return rc;
    if (!k_out || !v_out || li >= g_kv.layers || pos >= g_kv.ctx || kvd != g_kv.kvd)
        return fail(LOOMHIP_DECLINED, "read_kv: layer %zu / position %zu / %zu values outside the cache", li, pos,
                    kvd);
    if (g_sf.open)
        return fail(LOOMHIP_ERR_ARG, "read_kv: a frame is open (its rows exist after end_frame)");
    const uint16_t *hk, *hv;
    if (pos == g_kv.mirror_pos) {
        hk = g_kv.mk + li * kvd;
        hv = g_kv.mv + li * kvd;
    } else {
        if (int rc = g_pin_out.reserve(kvd * 4))
            return rc;
        uint16_t *b = (uint16_t *)g_pin_out.ptr;
        const size_t row = (li * g_kv.ctx + pos) * kvd;
        hipError_t e = hipMemcpyAsync(b, g_kv.k + row, kvd * 2, hipMemcpyDeviceToHost, g_ctx.compute);
        if (e == hipSuccess)
            e = hipMemcpyAsync(b + kvd, g_kv.v + row, kvd * 2, hipMemcpyDeviceToHost, g_ctx.compute);
        if (e == hipSuccess)
            e = hipStreamSynchronize(g_ctx.compute);
        if (e != hipSuccess)
            return hip_fail(e, "read_kv");
        hk = b;
        hv = b + kvd;
    }
    for (size_t i = 0; i < kvd; i++) {
        k_out[i] = half_bits_to_f32(hk[i]);
        v_out[i] = half_bits_to_f32(hv[i]);
    }
    return LOOMHIP_OK;
}

int loomhip_attn_heads(size_t li, size_t pos, const float *q, float *out, size_t n_heads, size_t n_kv_heads,
                       size_t hd, float scale) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = kv_ready("attn_heads"))
        return rc;
    if (!q || !out || li >= g_kv.layers || pos >= g_kv.ctx || n_kv_heads == 0 || n_heads % n_kv_heads ||
        n_heads / n_kv_heads > (size_t)MAX_G || n_kv_heads * hd != g_kv.kvd || (hd != 48 && hd != 64 && hd != 128))
        return fail(LOOMHIP_DECLINED, "attn_heads: heads %zu/%zu x %zu at layer %zu, position %zu not served",
                    n_heads, n_kv_heads, hd, li, pos);
    if (g_sf.open)
        return fail(LOOMHIP_ERR_ARG, "attn_heads: a frame is open");
    hipStream_t st = g_ctx.compute;
    FrameDims D{};
    D.hd = (int)hd;
    D.n_heads = (int)n_heads;
    D.n_kv = (int)n_kv_heads;
    D.qd = (int)(n_heads * hd);
    D.kvd = (int)g_kv.kvd;
    D.ctx = (int)g_kv.ctx;
    D.n_layers = (int)g_kv.layers;
    D.scale = scale;
    const int s_stride = (int)((g_kv.ctx + 63) / 64 * 64);
    const size_t qd = n_heads * hd;
    // device staging: pos | q | S | att
    const size_t o_q = 256, o_s = o_q + align16(qd * 4), o_a = o_s + align16(n_heads * (size_t)s_stride * 4);
    if (int rc = g_io.reserve(o_a + qd * 4))
        return rc;
    if (int rc = g_pin_in.reserve(256 + qd * 4))
        return rc;
    if (int rc = g_pin_out.reserve(qd * 4))
        return rc;
    char *io = (char *)g_io.ptr;
    *(int32_t *)g_pin_in.ptr = (int32_t)pos;
    memcpy((char *)g_pin_in.ptr + 256, q, qd * 4);
    hipError_t e = hipMemcpyAsync(io, g_pin_in.ptr, 256 + qd * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "attn_heads upload");
    // the rotated queries and the appended row are in place: no fused
    // prologue; one lane, so the softmax runs inside the P.V launch
    if (!launch_attn_exact(D, (const float *)(io + o_q), nullptr, nullptr, nullptr, nullptr, nullptr, g_kv.k, g_kv.v,
                           (const int32_t *)io, (int)li, false, (float *)(io + o_s), s_stride, (float *)(io + o_a), 1,
                           -1, QAct{}, st))
        return fail(LOOMHIP_DECLINED, "attn_heads: head size %zu not served", hd);
    e = hipMemcpyAsync(g_pin_out.ptr, io + o_a, qd * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "attn_heads");
    memcpy(out, g_pin_out.ptr, qd * 4);
    return LOOMHIP_OK;
}

// ---- the recorded dense frame (llama.zig:1067-1108 stepRecorded) ----------------

int loomhip_begin_frame(void) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_sf.open)
        return fail(LOOMHIP_ERR_ARG, "begin_frame: a frame is already open");
    g_sf = SeamFrame{};
    g_sf.open = true;
    return LOOMHIP_OK;
}

int loomhip_frame_open(void) { return g_sf.open ? 1 : 0; }

int loomhip_frame_load_x(const float *x, size_t dim) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_sf.open || !x || dim == 0)
        return fail(LOOMHIP_DECLINED, "frame_load_x: no open frame or no input");
    if (int rc = g_x.reserve(dim * 4))
        return rc;
    if (int rc = g_pin_in.reserve(dim * 4))
        return rc;
    memcpy(g_pin_in.ptr, x, dim * 4);
    hipError_t e = hipMemcpyAsync(g_x.ptr, g_pin_in.ptr, dim * 4, hipMemcpyHostToDevice, g_ctx.compute);
    if (e != hipSuccess)
        return hip_fail(e, "frame_load_x");
    // the staging is reused by the first layer's position: drain this copy
    if ((e = hipStreamSynchronize(g_ctx.compute)) != hipSuccess)
        return hip_fail(e, "frame_load_x");
    g_sf.dim = dim;
    g_sf.loaded = true;
    return LOOMHIP_OK;
}

int loomhip_layer_block(const loomhip_layer_spec *s) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!s || !g_sf.open || !g_sf.loaded || s->dim != g_sf.dim)
        return fail(LOOMHIP_DECLINED, "layer_block: no open frame holding a residual of this width");
    if (int rc = kv_ready("layer_block"))
        return rc;
    if (s->li >= g_kv.layers || s->pos >= g_kv.ctx || s->n_kv_heads * s->hd != g_kv.kvd ||
        (g_sf.pos != SIZE_MAX && s->pos != g_sf.pos))
        return fail(LOOMHIP_DECLINED, "layer_block: layer %zu / position %zu / kv width outside the cache", s->li,
                    s->pos);
    const size_t dim = s->dim, qd = s->n_heads * s->hd, kvd = g_kv.kvd;
    loomhip_model m = shell(dim, s->hd, s->n_heads, s->n_kv_heads, s->rope_dim, s->rope_base, s->eps, s->rope_neox);
    if (int rc = frame_dims_check(&m, 1))
        return rc;
    if (!s->attn_norm || !s->ffn_norm || !ref_ok(s->wq, qd, dim) || !ref_ok(s->wk, kvd, dim) ||
        !ref_ok(s->wv, kvd, dim) || !ref_ok(s->wo, dim, qd) || !ref_ok(s->gate, s->ffn, dim) ||
        !ref_ok(s->up, s->ffn, dim) || !ref_ok(s->down, dim, s->ffn))
        return fail(LOOMHIP_DECLINED, "layer_block: layer %zu misses a tensor or a length its shape implies", s->li);
    loomhip_layer l{};
    l.attn_norm = s->attn_norm; // host pointers for the checks; device ones below
    l.ffn_norm = s->ffn_norm;
    l.wq_t = s->wq.type;
    l.wk_t = s->wk.type;
    l.wv_t = s->wv.type;
    l.wo_t = s->wo.type;
    l.wq = s->wq.data;
    l.wk = s->wk.data;
    l.wv = s->wv.data;
    l.wo = s->wo.data;
    l.is_moe = 0;
    l.ffn_gate_t = s->gate.type;
    l.ffn_up_t = s->up.type;
    l.ffn_down_t = s->down.type;
    l.ffn_gate = s->gate.data;
    l.ffn_up = s->up.data;
    l.ffn_down = s->down.data;
    l.ffn = s->ffn;
    size_t ffn_max = 0;
    if (int rc = frame_layer_check(&m, l, s->li, 1, &ffn_max))
        return rc;
    int rc;
    if ((rc = upload_f32(s->attn_norm, dim, &l.attn_norm)) || (rc = upload_f32(s->ffn_norm, dim, &l.ffn_norm)) ||
        (rc = upload_ref(s->wq, qd, dim, 1, &l.wq)) || (rc = upload_ref(s->wk, kvd, dim, 1, &l.wk)) ||
        (rc = upload_ref(s->wv, kvd, dim, 1, &l.wv)) || (rc = upload_ref(s->wo, dim, qd, 1, &l.wo)) ||
        (rc = upload_ref(s->gate, s->ffn, dim, 1, &l.ffn_gate)) || (rc = upload_ref(s->up, s->ffn, dim, 1, &l.ffn_up)) ||
        (rc = upload_ref(s->down, dim, s->ffn, 1, &l.ffn_down)))
        return rc;
    hipStream_t st = g_ctx.compute;
    int32_t *dpos = nullptr;
    if (g_sf.pos == SIZE_MAX) { // the frame's position, once (every layer reads the same)
        if ((rc = put_pos(s->pos, &dpos, st)))
            return rc;
        g_sf.pos = s->pos;
    }
    dpos = (int32_t *)g_io.ptr;
    FrameCall c;
    if ((rc = frame_setup(&m, 1, ffn_max, s->attn_scale, dpos, g_kv.k, g_kv.v, st, c)))
        return rc;
    c.w.x = (float *)g_x.ptr; // the frame's residual, loaded by frame_load_x
    if ((rc = frame_layer(c, l, s->li, nullptr)))
        return rc;
    g_sf.wrote = true;
    return LOOMHIP_OK;
}

int loomhip_end_frame(void) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_sf.open)
        return LOOMHIP_OK;
    int rc = LOOMHIP_OK;
    if (g_sf.wrote)
        rc = mirror_rows(g_sf.pos, g_ctx.compute);
    const hipError_t e = hipStreamSynchronize(g_ctx.compute);
    g_sf.open = false;
    if (rc)
        return rc;
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "end_frame");
}

int loomhip_frame_store_x(float *x, size_t dim) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_sf.open || !g_sf.loaded || !x || dim != g_sf.dim)
        return fail(LOOMHIP_DECLINED, "frame_store_x: no finished frame of this width");
    hipError_t e = hipMemcpy(x, g_x.ptr, dim * 4, hipMemcpyDeviceToHost);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "frame_store_x");
}

// ---- the GQA+MoE whole token (the qwen3moe form of mlaTokenFrame) ----------------

int loomhip_gqa_token_frame(const loomhip_gqa_layer_desc *descs, size_t n_layers, const loomhip_gqa_frame_cfg *fc,
                            float *x, size_t pos, const float *out_norm, loomhip_weight_ref lm_head, float *logits,
                            size_t vocab) {
    if (int rc = require_ready())
        return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!descs || !fc || !x || !out_norm || !logits || vocab == 0 || n_layers == 0)
        return fail(LOOMHIP_ERR_ARG, "gqa_token_frame: null argument");
    if (g_sf.open)
        return fail(LOOMHIP_ERR_ARG, "gqa_token_frame: a frame is open");
    if (int rc = kv_ready("gqa_token_frame"))
        return rc;
    const size_t dim = fc->dim, hd = fc->head_dim, qd = fc->n_heads * hd, kvd = fc->n_kv_heads * hd;
    if (n_layers != g_kv.layers || kvd != g_kv.kvd || pos >= g_kv.ctx)
        return fail(LOOMHIP_DECLINED, "gqa_token_frame: %zu layers x %zu at position %zu do not match the cache",
                    n_layers, kvd, pos);
    loomhip_model m = shell(dim, hd, fc->n_heads, fc->n_kv_heads, fc->rope_dim, fc->rope_base, fc->eps,
                            fc->rope_neox);
    m.vocab = vocab;
    m.output_t = lm_head.type;
    m.output = lm_head.data;
    m.out_norm = out_norm;
    if (!ref_ok(lm_head, vocab, dim))
        return fail(LOOMHIP_DECLINED, "gqa_token_frame: lm_head of %zu bytes is not [%zu][%zu]", lm_head.len, vocab,
                    dim);
    // every layer resolved and checked (host pointers), then uploaded,
    // before the first launch
    std::vector<loomhip_layer> L(n_layers);
    for (size_t li = 0; li < n_layers; li++) {
        const loomhip_gqa_layer_desc &d = descs[li];
        loomhip_layer &l = L[li];
        if (!ref_ok(d.wq, qd, dim) || !ref_ok(d.wk, kvd, dim) || !ref_ok(d.wv, kvd, dim) || !ref_ok(d.wo, dim, qd))
            return fail(LOOMHIP_DECLINED, "gqa_token_frame: layer %zu attention weights do not match their shapes",
                        li);
        l.attn_norm = d.attn_norm;
        l.ffn_norm = d.ffn_norm;
        l.q_norm = d.q_norm;
        l.k_norm = d.k_norm;
        l.wq_t = d.wq.type;
        l.wk_t = d.wk.type;
        l.wv_t = d.wv.type;
        l.wo_t = d.wo.type;
        l.wq = d.wq.data;
        l.wk = d.wk.data;
        l.wv = d.wv.data;
        l.wo = d.wo.data;
        l.is_moe = d.is_moe ? 1 : 0;
        if (d.is_moe) {
            const size_t E = fc->n_expert;
            const bool sh = d.shexp_gate.data != nullptr;
            if (d.router.type != LH_F32 || !ref_ok(d.router, E, dim) || !ref_ok(d.gate, d.ffn, dim, E) ||
                !ref_ok(d.up, d.ffn, dim, E) || !ref_ok(d.down, dim, d.ffn, E) ||
                (sh && (!ref_ok(d.shexp_gate, d.shexp_ffn, dim) || !ref_ok(d.shexp_up, d.shexp_ffn, dim) ||
                        !ref_ok(d.shexp_down, dim, d.shexp_ffn))))
                return fail(LOOMHIP_DECLINED, "gqa_token_frame: layer %zu MoE weights do not match their shapes", li);
            loomhip_moe_layer &e = l.moe;
            e.dim = dim;
            e.ffn = d.ffn;
            e.n_expert = E;
            e.n_used = fc->n_used;
            e.gating = fc->gating;
            e.weights_norm = fc->weights_norm;
            e.weights_scale = fc->weights_scale;
            e.router = (const float *)d.router.data;
            e.router_bias = d.router_bias;
            e.sel_bias = d.sel_bias;
            e.gate_t = d.gate.type;
            e.up_t = d.up.type;
            e.down_t = d.down.type;
            e.gate = d.gate.data;
            e.up = d.up.data;
            e.down = d.down.data;
            if (sh) {
                e.shexp_gate_t = d.shexp_gate.type;
                e.shexp_up_t = d.shexp_up.type;
                e.shexp_down_t = d.shexp_down.type;
                e.shexp_gate = d.shexp_gate.data;
                e.shexp_up = d.shexp_up.data;
                e.shexp_down = d.shexp_down.data;
                e.shexp_ffn = d.shexp_ffn;
            }
        } else {
            if (!ref_ok(d.dgate, d.dffn, dim) || !ref_ok(d.dup, d.dffn, dim) || !ref_ok(d.ddown, dim, d.dffn))
                return fail(LOOMHIP_DECLINED, "gqa_token_frame: layer %zu FFN weights do not match their shapes", li);
            l.ffn_gate_t = d.dgate.type;
            l.ffn_up_t = d.dup.type;
            l.ffn_down_t = d.ddown.type;
            l.ffn_gate = d.dgate.data;
            l.ffn_up = d.dup.data;
            l.ffn_down = d.ddown.data;
            l.ffn = d.dffn;
        }
    }
    m.layers = L.data();
    size_t ffn_max = 0;
    if (int rc = frame_check(&m, 1, &ffn_max))
        return rc;
    int rc;
    for (size_t li = 0; li < n_layers; li++) {
        const loomhip_gqa_layer_desc &d = descs[li];
        loomhip_layer &l = L[li];
        if ((rc = upload_f32(d.attn_norm, dim, &l.attn_norm)) || (rc = upload_f32(d.ffn_norm, dim, &l.ffn_norm)) ||
            (d.q_norm && (rc = upload_f32(d.q_norm, hd, &l.q_norm))) ||
            (d.k_norm && (rc = upload_f32(d.k_norm, hd, &l.k_norm))) || (rc = upload_ref(d.wq, qd, dim, 1, &l.wq)) ||
            (rc = upload_ref(d.wk, kvd, dim, 1, &l.wk)) || (rc = upload_ref(d.wv, kvd, dim, 1, &l.wv)) ||
            (rc = upload_ref(d.wo, dim, qd, 1, &l.wo)))
            return rc;
        if (d.is_moe) {
            loomhip_moe_layer &e = l.moe;
            const size_t E = fc->n_expert;
            if ((rc = upload_f32((const float *)d.router.data, E * dim, &e.router)) ||
                (d.router_bias && (rc = upload_f32(d.router_bias, E, &e.router_bias))) ||
                (d.sel_bias && (rc = upload_f32(d.sel_bias, E, &e.sel_bias))) ||
                (rc = upload_ref(d.gate, d.ffn, dim, E, &e.gate)) || (rc = upload_ref(d.up, d.ffn, dim, E, &e.up)) ||
                (rc = upload_ref(d.down, dim, d.ffn, E, &e.down)))
                return rc;
            if (d.shexp_gate.data &&
                ((rc = upload_ref(d.shexp_gate, d.shexp_ffn, dim, 1, &e.shexp_gate)) ||
                 (rc = upload_ref(d.shexp_up, d.shexp_ffn, dim, 1, &e.shexp_up)) ||
                 (rc = upload_ref(d.shexp_down, dim, d.shexp_ffn, 1, &e.shexp_down))))
                return rc;
        } else if ((rc = upload_ref(d.dgate, d.dffn, dim, 1, &l.ffn_gate)) ||
                   (rc = upload_ref(d.dup, d.dffn, dim, 1, &l.ffn_up)) ||
                   (rc = upload_ref(d.ddown, dim, d.dffn, 1, &l.ffn_down)))
            return rc;
    }
    if ((rc = upload_f32(out_norm, dim, &m.out_norm)) || (rc = upload_ref(lm_head, vocab, dim, 1, &m.output)))
        return rc;
    hipStream_t st = g_ctx.compute;
    // device staging: pos | logits; pinned: pos | x in, x | logits out
    const size_t o_l = 256;
    if ((rc = g_io.reserve(o_l + vocab * 4)) || (rc = g_pin_in.reserve(256 + dim * 4)) ||
        (rc = g_pin_out.reserve((dim + vocab) * 4)))
        return rc;
    char *io = (char *)g_io.ptr;
    *(int32_t *)g_pin_in.ptr = (int32_t)pos;
    memcpy((char *)g_pin_in.ptr + 256, x, dim * 4);
    FrameCall c;
    if ((rc = frame_setup(&m, 1, ffn_max, fc->scale, (int32_t *)io, g_kv.k, g_kv.v, st, c)))
        return rc;
    hipError_t e = hipMemcpyAsync(io, g_pin_in.ptr, 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(c.w.x, (char *)g_pin_in.ptr + 256, dim * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "gqa_token_frame upload");
    for (size_t li = 0; li < n_layers; li++)
        if ((rc = frame_layer(c, L[li], li, nullptr)))
            return rc;
    float *dlog = (float *)(io + o_l);
    if ((rc = frame_head(c, &m, dlog)))
        return rc;
    float *px = (float *)g_pin_out.ptr, *pl = px + dim;
    e = hipMemcpyAsync(px, c.w.x, dim * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(pl, dlog, vocab * 4, hipMemcpyDeviceToHost, st);
    if (e != hipSuccess)
        return hip_fail(e, "gqa_token_frame download");
    if ((rc = mirror_rows(pos, st)))
        return rc;
    if ((e = hipStreamSynchronize(st)) != hipSuccess)
        return hip_fail(e, "gqa_token_frame");
    memcpy(x, px, dim * 4);
    memcpy(logits, pl, vocab * 4);
    return LOOMHIP_OK;
}

} // extern "C"
