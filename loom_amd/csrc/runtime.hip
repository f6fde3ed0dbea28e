// runtime.hip -- host side of libloomhip: device/stream lifecycle, the
// pointer-keyed weight cache, grow-only scratch, and the C ABI of
// include/loomhip.h.  The MoE layer and expert cache entry points live in
// moe_host.hip and expert_cache.hip.
#include "runtime.hpp"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace lh {

static std::atomic<uint64_t> g_launches{0};
static thread_local char g_err[512] = "";
Ctx g_ctx;

void note_launch() { g_launches.fetch_add(1, std::memory_order_relaxed); }

// ---- kernel timing -------------------------------------------------------------
struct ProfRec {
    hipEvent_t a, b;
    int tag;
};
static bool g_prof = false;
static std::vector<ProfRec> g_prof_recs;
static std::vector<hipEvent_t> g_prof_pool;
static double g_prof_ms[LOOMHIP_KT_COUNT];
static uint64_t g_prof_n[LOOMHIP_KT_COUNT];

static hipEvent_t prof_event() {
    if (!g_prof_pool.empty()) {
        hipEvent_t e = g_prof_pool.back();
        g_prof_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

int prof_begin(int tag, hipStream_t st) {
    if (!g_prof || tag < 0 || tag >= LOOMHIP_KT_COUNT)
        return -1;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return -1;
    ProfRec r{prof_event(), prof_event(), tag};
    if (!r.a || !r.b || hipEventRecord(r.a, st) != hipSuccess)
        return -1;
    g_prof_recs.push_back(r);
    return (int)g_prof_recs.size() - 1;
}

void prof_end(int handle, hipStream_t st) {
    if (handle < 0 || handle >= (int)g_prof_recs.size())
        return;
    (void)hipEventRecord(g_prof_recs[handle].b, st);
}

static void prof_drain() {
    for (auto &r : g_prof_recs) {
        float ms = 0.0f;
        if (hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
            g_prof_ms[r.tag] += ms;
            g_prof_n[r.tag] += 1;
        }
        g_prof_pool.push_back(r.a);
        g_prof_pool.push_back(r.b);
    }
    g_prof_recs.clear();
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(LOOMHIP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t stream_of(void *s) { return (hipStream_t)s; } // NULL: the null stream

int Scratch::reserve(size_t bytes) {
    if (bytes <= cap)
        return LOOMHIP_OK;
    if (ptr) {
        (void)hipStreamSynchronize(g_ctx.compute);
        (void)hipFree(ptr);
        ptr = nullptr;
        cap = 0;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    want += want / 4; // grow geometrically
    hipError_t e = hipMalloc(&ptr, want);
    if (e != hipSuccess) {
        ptr = nullptr;
        return hip_fail(e, "hipMalloc scratch");
    }
    cap = want;
    return LOOMHIP_OK;
}

// ---- weight cache (src/vulkan/backend.zig:244-261 semantics) ---------------

struct CachedWeight {
    void *dev;
    size_t len; // GGML bytes of the host tensor
    int type;
    size_t rows, cols, planes;
};
static std::mutex g_wmu;
static std::unordered_map<const void *, CachedWeight> g_wcache;
static size_t g_resident = 0;

int upload_weights(int t, const void *host, size_t rows, size_t cols, size_t planes, void **dev) {
    const size_t glen = ggml_bytes(t, rows, cols) * planes;
    std::lock_guard<std::mutex> lk(g_wmu);
    auto it = g_wcache.find(host);
    if (it != g_wcache.end() && it->second.len == glen && it->second.type == t &&
        it->second.rows == rows && it->second.cols == cols) {
        *dev = it->second.dev;
        return LOOMHIP_OK;
    }
    if (it != g_wcache.end()) { // same pointer, different tensor: re-upload
        (void)hipFree(it->second.dev);
        g_resident -= plane_bytes(it->second.type, it->second.rows, it->second.cols) * it->second.planes;
        g_wcache.erase(it);
    }
    const size_t dlen = plane_bytes(t, rows, cols) * planes;
    void *d = nullptr, *tmp = nullptr;
    hipError_t e = hipMalloc(&d, dlen);
    if (e != hipSuccess)
        return hip_fail(e, "hipMalloc weights");
    if (t == LH_Q4_K || t == LH_F32 || t == LH_F16) {
        e = hipMemcpy(d, host, glen, hipMemcpyHostToDevice);
    } else {
        e = hipMalloc(&tmp, glen);
        if (e == hipSuccess)
            e = hipMemcpy(tmp, host, glen, hipMemcpyHostToDevice);
        if (e == hipSuccess) {
            launch_repack(t, tmp, d, rows, cols, planes, g_ctx.compute);
            e = hipStreamSynchronize(g_ctx.compute);
        }
        if (tmp)
            (void)hipFree(tmp);
    }
    if (e != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "upload weights");
    }
    g_wcache[host] = CachedWeight{d, glen, t, rows, cols, planes};
    g_resident += dlen;
    *dev = d;
    return LOOMHIP_OK;
}

void clear_weight_cache() {
    std::lock_guard<std::mutex> lk(g_wmu);
    if (g_ctx.ready)
        (void)hipDeviceSynchronize();
    for (auto &kv : g_wcache)
        (void)hipFree(kv.second.dev);
    g_wcache.clear();
    g_resident = 0;
}

// ---- dense grouped-matvec plumbing ---------------------------------------------

// Device group table for n dense vectors against plane 0 (cached per n).
const DmmvGroup *dense_groups(int n, int nt, int *count) {
    const int ng = (n + nt - 1) / nt;
    *count = ng;
    const int key = n * 16 + nt;
    auto it = g_ctx.dense_tables.find(key);
    if (it != g_ctx.dense_tables.end())
        return (const DmmvGroup *)it->second;
    DmmvGroup *h = new DmmvGroup[ng];
    for (int i = 0; i < ng; i++) {
        h[i].plane = 0;
        h[i].first = i * nt;
        h[i].n = (n - i * nt) < nt ? (n - i * nt) : nt;
    }
    void *d = nullptr;
    if (hipMalloc(&d, sizeof(DmmvGroup) * ng) != hipSuccess) {
        delete[] h;
        return nullptr;
    }
    (void)hipMemcpy(d, h, sizeof(DmmvGroup) * ng, hipMemcpyHostToDevice);
    delete[] h;
    g_ctx.dense_tables[key] = d;
    return (const DmmvGroup *)d;
}

int pick_nt(int n) { return n >= 8 ? 8 : n >= 4 ? 4 : n >= 2 ? 2 : 1; }

// Quantize n vectors and run the grouped matvec against one plane.
int matvec_dev_impl(int t, float *out, const void *w, const float *x, size_t n, size_t rows,
                    size_t cols, hipStream_t st) {
    if (n == 0)
        return LOOMHIP_OK;
    if (t == LH_F32) {
        launch_router_gemv((const float *)w, nullptr, x, (int)rows, (int)cols, (int)n, out, st);
        // router gemv writes logits[t][e] = out[k*rows + r]: same layout
        return LOOMHIP_OK;
    }
    if (!dmmv_supported(t, (int)cols))
        return fail(LOOMHIP_DECLINED, "dmmv: type %d with %zu columns not served", t, cols);
    if (n > IOTA_LEN)
        return fail(LOOMHIP_DECLINED, "dmmv: %zu vectors exceed %d", n, IOTA_LEN);
    const size_t qbytes = align16(n * cols) + align16(n * cols / 32 * 4) + align16(n * cols / 16 * 4);
    int rc = g_ctx.act.reserve(qbytes);
    if (rc)
        return rc;
    QAct qa;
    qa.q = (int8_t *)g_ctx.act.ptr;
    qa.d = (float *)((char *)g_ctx.act.ptr + align16(n * cols));
    qa.s = (int32_t *)((char *)qa.d + align16(n * cols / 32 * 4));
    launch_quant_act(t, x, (int)cols, (int)cols, (int)n, qa, st);
    const bool mq = use_mmq(t, (int)cols, (int)n, 32, false);
    const int nt = mq ? 32 : pick_nt((int)n);
    int ng = 0;
    const DmmvGroup *groups = dense_groups((int)n, nt, &ng);
    if (!groups)
        return fail(LOOMHIP_ERR_HIP, "dense group table");
    DmmvParams p{};
    p.w = (const uint8_t *)w;
    p.w2 = nullptr;
    p.plane_bytes = plane_bytes(t, rows, cols);
    p.rows = (int)rows;
    p.cols = (int)cols;
    p.xq = qa.q;
    p.xd = qa.d;
    p.xs = qa.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = groups;
    p.n_groups_dev = nullptr;
    p.n_groups = ng;
    p.out = out;
    p.out_stride = (int)rows;
    p.rpw = mq ? 0 : dmmv_pick_rpw(t, (int)cols, (int)rows, ng, nt, false);
    p.ident_n = mq ? (int)n : 0;
    const int ph = prof_begin(LOOMHIP_KT_DENSE, st);
    const bool launched = mq ? launch_mmq(t, nt, false, p, st) : launch_dmmv(t, nt, false, p, st);
    prof_end(ph, st);
    if (!launched)
        return fail(LOOMHIP_DECLINED, "dmmv: partials exceed LDS for %zu columns", cols);
    return LOOMHIP_OK;
}

int require_ready() {
    if (!g_ctx.ready)
        return fail(LOOMHIP_ERR_INIT, "loomhip_init has not succeeded");
    return LOOMHIP_OK;
}

} // namespace lh

using namespace lh;

extern "C" {

int loomhip_init(int device) {
    if (g_ctx.ready)
        return g_ctx.device == device ? LOOMHIP_OK : fail(LOOMHIP_ERR_ARG, "already initialised on device %d", g_ctx.device);
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= device || device < 0)
        return fail(LOOMHIP_ERR_INIT, "no HIP device %d (count %d)", device, count);
    if ((e = hipSetDevice(device)) != hipSuccess)
        return hip_fail(e, "hipSetDevice");
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return hip_fail(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(LOOMHIP_ERR_INIT, "device %d is %s, this build targets gfx950", device, prop.gcnArchName);
    // default-priority streams only
    if ((e = hipStreamCreateWithFlags(&g_ctx.compute, hipStreamNonBlocking)) != hipSuccess)
        return hip_fail(e, "hipStreamCreate compute");
    if ((e = hipStreamCreateWithFlags(&g_ctx.copy, hipStreamNonBlocking)) != hipSuccess)
        return hip_fail(e, "hipStreamCreate copy");
    int *iota = new int[IOTA_LEN];
    for (int i = 0; i < IOTA_LEN; i++)
        iota[i] = i;
    void *d = nullptr;
    if ((e = hipMalloc(&d, sizeof(int) * IOTA_LEN)) != hipSuccess) {
        delete[] iota;
        return hip_fail(e, "hipMalloc iota");
    }
    e = hipMemcpy(d, iota, sizeof(int) * IOTA_LEN, hipMemcpyHostToDevice);
    delete[] iota;
    if (e != hipSuccess)
        return hip_fail(e, "iota upload");
    g_ctx.iota = (const int *)d;
    void *sy = nullptr;
    if ((e = hipMalloc(&sy, sizeof(int) * SYNC_INTS)) != hipSuccess)
        return hip_fail(e, "hipMalloc sync");
    if ((e = hipMemset(sy, 0, sizeof(int) * SYNC_INTS)) != hipSuccess)
        return hip_fail(e, "hipMemset sync");
    g_ctx.sync = (int *)sy;
    if (int rc = moe_noalloc_setup(device))
        return rc;
    g_ctx.device = device;
    g_ctx.ready = true;
    return LOOMHIP_OK;
}

void loomhip_shutdown(void) {
    if (!g_ctx.ready)
        return;
    (void)hipDeviceSynchronize();
    clear_weight_cache();
    for (auto &kv : g_ctx.dense_tables)
        (void)hipFree(kv.second);
    g_ctx.dense_tables.clear();
    g_ctx.act.release();
    g_ctx.xstage.release();
    g_ctx.ostage.release();
    moe_release_scratch();
    ec_release_scratch();
    block_release_cache();
    mla_release();
    seam_release();
    prof_drain();
    for (hipEvent_t e : g_prof_pool)
        (void)hipEventDestroy(e);
    g_prof_pool.clear();
    g_prof = false;
    (void)hipFree((void *)g_ctx.iota);
    (void)hipFree(g_ctx.sync);
    g_ctx.sync = nullptr;
    (void)hipStreamDestroy(g_ctx.compute);
    (void)hipStreamDestroy(g_ctx.copy);
    g_ctx.ready = false;
}

const char *loomhip_last_error(void) { return g_err; }

void loomhip_profile_kernels(int enable) {
    prof_drain();
    for (int i = 0; i < LOOMHIP_KT_COUNT; i++) {
        g_prof_ms[i] = 0.0;
        g_prof_n[i] = 0;
    }
    g_prof = enable != 0;
}

int loomhip_kernel_time(int tag, double *total_ms, uint64_t *launches) {
    if (tag < 0 || tag >= LOOMHIP_KT_COUNT || !total_ms || !launches)
        return fail(LOOMHIP_ERR_ARG, "kernel_time: bad tag %d", tag);
    prof_drain();
    *total_ms = g_prof_ms[tag];
    *launches = g_prof_n[tag];
    return LOOMHIP_OK;
}

uint64_t loomhip_take_launch_count(void) { return g_launches.exchange(0); }

const char *loomhip_version(void) { return "loomhip 0.1 gfx950"; }

size_t loomhip_plane_bytes(int t, size_t rows, size_t cols) { return plane_bytes(t, rows, cols); }
size_t loomhip_ggml_bytes(int t, size_t rows, size_t cols) { return ggml_bytes(t, rows, cols); }

int loomhip_register_weights(int t, const void *host, size_t rows, size_t cols, size_t planes,
                             void **dev_out) {
    if (int rc = require_ready())
        return rc;
    if (!host || !dev_out || planes == 0 || cols % block_elems(t))
        return fail(LOOMHIP_ERR_ARG, "register_weights: bad arguments");
    return upload_weights(t, host, rows, cols, planes, dev_out);
}

void loomhip_clear_weight_cache(void) {
    clear_weight_cache();
    block_release_cache();
}

size_t loomhip_resident_bytes(void) { return g_resident; }

int loomhip_repack_dev(int t, void *dst, const void *src, size_t rows, size_t cols, size_t planes,
                       void *stream) {
    if (int rc = require_ready())
        return rc;
    if (cols % block_elems(t))
        return fail(LOOMHIP_ERR_ARG, "repack: cols %% block");
    launch_repack(t, src, dst, rows, cols, planes, stream_of(stream));
    return LOOMHIP_OK;
}

int loomhip_synth_weights_dev(int t, void *dst, size_t rows, size_t cols, size_t planes,
                              uint64_t seed, float stddev, void *stream) {
    if (int rc = require_ready())
        return rc;
    if (t != LH_Q4_K && t != LH_Q6_K && t != LH_Q8_0 && t != LH_Q4_0)
        return fail(LOOMHIP_DECLINED, "synth: type %d", t);
    if (cols % block_elems(t))
        return fail(LOOMHIP_ERR_ARG, "synth: cols %% block");
    launch_synth(t, dst, rows, cols, planes, seed, stddev, stream_of(stream));
    return LOOMHIP_OK;
}

int loomhip_matvec_dev(int t, float *out, const void *w, const float *x, size_t n, size_t rows,
                       size_t cols, void *stream) {
    if (int rc = require_ready())
        return rc;
    return matvec_dev_impl(t, out, w, x, n, rows, cols, stream_of(stream));
}

int loomhip_dequant_dev(int t, float *out, const void *w, size_t rows, size_t cols, void *stream) {
    if (int rc = require_ready())
        return rc;
    if (cols % block_elems(t))
        return fail(LOOMHIP_ERR_ARG, "dequant: cols %% block");
    launch_dequant(t, w, rows, cols, out, stream_of(stream));
    return LOOMHIP_OK;
}

// ---- seam calls ----------------------------------------------------------------

static bool served_type(int t) {
    return t == LH_Q4_K || t == LH_Q6_K || t == LH_Q8_0 || t == LH_Q4_0 || t == LH_F32;
}

int loomhip_matmul(int t, float *out, const uint8_t *w, const float *xs, size_t n, size_t rows,
                   size_t cols) {
    if (int rc = require_ready())
        return rc;
    if (!served_type(t))
        return fail(LOOMHIP_DECLINED, "matmul: type %d not served", t);
    if (t != LH_F32 && !dmmv_supported(t, (int)cols))
        return fail(LOOMHIP_DECLINED, "matmul: %zu columns not served for type %d", cols, t);
    if (n == 0)
        return LOOMHIP_OK;
    void *dw = nullptr;
    int rc = upload_weights(t, w, rows, cols, 1, &dw);
    if (rc)
        return rc;
    if ((rc = g_ctx.xstage.reserve(n * cols * 4)) || (rc = g_ctx.ostage.reserve(n * rows * 4)))
        return rc;
    hipStream_t st = g_ctx.compute;
    hipError_t e = hipMemcpyAsync(g_ctx.xstage.ptr, xs, n * cols * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "stage x");
    rc = matvec_dev_impl(t, (float *)g_ctx.ostage.ptr, dw, (const float *)g_ctx.xstage.ptr, n, rows,
                         cols, st);
    if (rc)
        return rc;
    e = hipMemcpyAsync(out, g_ctx.ostage.ptr, n * rows * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "matmul readback");
    return LOOMHIP_OK;
}

int loomhip_matvec(int t, float *out, const uint8_t *w, const float *x, size_t rows, size_t cols) {
    return loomhip_matmul(t, out, w, x, 1, rows, cols);
}

int loomhip_dequant_row(int t, float *out, const uint8_t *w, size_t r, size_t cols) {
    if (int rc = require_ready())
        return rc;
    if (!served_type(t) && t != LH_F16)
        return fail(LOOMHIP_DECLINED, "dequant_row: type %d not served", t);
    if (cols % block_elems(t))
        return fail(LOOMHIP_ERR_ARG, "dequant_row: cols %% block");
    // One row is its own plane: upload just that row (the embedding lookup).
    const uint8_t *row = w + r * ggml_bytes(t, 1, cols);
    void *dw = nullptr;
    int rc = upload_weights(t, row, 1, cols, 1, &dw);
    if (rc)
        return rc;
    if ((rc = g_ctx.ostage.reserve(cols * 4)))
        return rc;
    hipStream_t st = g_ctx.compute;
    launch_dequant(t, dw, 1, cols, (float *)g_ctx.ostage.ptr, st);
    hipError_t e = hipMemcpyAsync(out, g_ctx.ostage.ptr, cols * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "dequant readback");
    return LOOMHIP_OK;
}

} // extern "C"
