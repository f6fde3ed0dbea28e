// expert_block.hip -- backend.moeFfnBlock (src/compute/cpu.zig:23-30; the
// Metal form src/metal/backend.zig:2322-2410): one MoE layer's selected
// experts, and the shared one, handed over as host tensor slices with their
// router weights; out = the sum, in list order, of weight * FFN(normed).  The
// caller (src/gguf/deepseek.zig:1405-1440) builds the list from its expert
// Source (src/p2p/expert_fetch.zig:91-400), whose slices stay valid for the
// call (stablePointers).
//
// The HBM tier in front of that Source.  Each tensor slice resolves to a slot
// of an LRU in HBM: a hit uses the slot as is; a miss copies the GGML bytes
// into the slot (Q4_K keeps GGML's layout) or through a staging buffer and
// the device-layout repack (Q6_K, Q8_0, Q4_0).  Only slices inside a
// registered arena (backend.registerArena: the model's mapping, whose bytes
// never change, src/gguf/deepseek.zig:466-473) are kept across calls, keyed
// by (pointer, length, type, shape); any other slice -- a RAM-cache slot of
// the Source, whose bytes change when it refills -- is copied in on every
// call and its slot freed afterwards.  prefetch is the tier's prefetchAsync
// (expert_fetch.zig:390-400): arena slices not resident start their fills on
// the copy stream, and the call that uses them waits for each fill.  The
// slots are sized by the largest tensor seen; a larger one empties the cache
// and re-sizes it.  Then, per expert, the fused gate/up SwiGLU matvec, the
// activations' quantization and the down matvec (all bit-identical to the
// CPU kernels), and one weighted combine in list order.  One stream-ordered
// submission; synchronous at the seam, like the reference's.
#include "runtime.hpp"

#include <list>
#include <unordered_map>
#include <vector>

namespace lh {

constexpr size_t BLOCK_MAX_EXPERTS = 16; // the Metal form's MAX_MOE_EXPERTS
constexpr size_t BLOCK_LRU_SLOTS = 192;  // 64 experts of three tensors

struct SliceKey {
    const void *ptr;
    size_t len;
    int t;
    size_t rows, cols;
    bool operator==(const SliceKey &o) const {
        return ptr == o.ptr && len == o.len && t == o.t && rows == o.rows && cols == o.cols;
    }
};
struct SliceHash {
    size_t operator()(const SliceKey &k) const {
        return std::hash<const void *>()(k.ptr) ^ (k.len * 0x9E3779B97F4A7C15ull) ^ ((size_t)k.t << 48);
    }
};

// Registered arenas (backend.registerArena): read-only host regions whose
// bytes stay fixed while registered, page-aligned outward like the Metal form.
constexpr int MAX_ARENAS = 16;
struct Arena {
    uintptr_t base = 0;
    size_t len = 0;
};
static Arena g_arenas[MAX_ARENAS];
static int g_n_arenas = 0;

static bool in_arena(const void *p, size_t len) {
    const uintptr_t a = (uintptr_t)p;
    for (int i = 0; i < g_n_arenas; i++)
        if (a >= g_arenas[i].base && a + len <= g_arenas[i].base + g_arenas[i].len)
            return true;
    return false;
}

struct BlockLru {
    uint8_t *slab = nullptr, *staging = nullptr, *staging_copy = nullptr;
    size_t slot_bytes = 0, n_slots = 0;
    std::vector<size_t> free_slots;
    std::vector<hipEvent_t> fill; // per slot: the prefetch fill on the copy stream
    std::vector<char> fill_pending;
    std::list<SliceKey> order; // front = most recent
    struct Entry {
        size_t slot;
        std::list<SliceKey>::iterator it;
    };
    std::unordered_map<SliceKey, Entry, SliceHash> map;
    std::vector<size_t> transient; // this call's slots of slices outside the arenas
    uint64_t hits = 0, misses = 0, bytes_read = 0, prefetched = 0;

    void release() {
        if (slab || staging)
            (void)hipDeviceSynchronize();
        if (slab)
            (void)hipFree(slab);
        if (staging)
            (void)hipFree(staging);
        if (staging_copy)
            (void)hipFree(staging_copy);
        for (hipEvent_t e : fill)
            (void)hipEventDestroy(e);
        slab = staging = staging_copy = nullptr;
        slot_bytes = n_slots = 0;
        free_slots.clear();
        fill.clear();
        fill_pending.clear();
        order.clear();
        map.clear();
        transient.clear();
    }
    int reserve(size_t bytes) {
        if (bytes <= slot_bytes)
            return LOOMHIP_OK;
        release();
        hipError_t e = hipMalloc((void **)&slab, bytes * BLOCK_LRU_SLOTS);
        if (e == hipSuccess)
            e = hipMalloc((void **)&staging, bytes);
        if (e == hipSuccess)
            e = hipMalloc((void **)&staging_copy, bytes);
        fill.assign(BLOCK_LRU_SLOTS, nullptr);
        fill_pending.assign(BLOCK_LRU_SLOTS, 0);
        for (size_t i = 0; e == hipSuccess && i < BLOCK_LRU_SLOTS; i++)
            e = hipEventCreateWithFlags(&fill[i], hipEventDisableTiming);
        if (e != hipSuccess) {
            release();
            return hip_fail(e, "moe_ffn_block: HBM cache");
        }
        slot_bytes = bytes;
        n_slots = BLOCK_LRU_SLOTS;
        for (size_t i = n_slots; i-- > 0;)
            free_slots.push_back(i);
        return LOOMHIP_OK;
    }
    // A slot for new contents: a free one, else the least recently used
    // cached slice's.  Work on st that follows waits for any fill still
    // writing the slot on the copy stream.
    size_t take_slot(hipStream_t st) {
        size_t s;
        if (!free_slots.empty()) {
            s = free_slots.back();
            free_slots.pop_back();
        } else {
            const SliceKey victim = order.back();
            s = map[victim].slot;
            map.erase(victim);
            order.pop_back();
        }
        if (fill_pending[s]) {
            (void)hipStreamWaitEvent(st, fill[s], 0);
            fill_pending[s] = 0;
        }
        return s;
    }
    hipError_t copy_in(const SliceKey &k, uint8_t *dst, uint8_t *stage, hipStream_t st) {
        if (k.t == LH_Q4_K)
            return hipMemcpyAsync(dst, k.ptr, k.len, hipMemcpyHostToDevice, st);
        hipError_t e = hipMemcpyAsync(stage, k.ptr, k.len, hipMemcpyHostToDevice, st);
        if (e == hipSuccess)
            launch_repack(k.t, stage, dst, k.rows, k.cols, 1, st);
        return e;
    }
    // The device-layout copy of a host tensor slice for work on st.
    int get(const SliceKey &k, hipStream_t st, const void **dev) {
        const bool keep = in_arena(k.ptr, k.len);
        if (keep) {
            auto f = map.find(k);
            if (f != map.end()) {
                hits++;
                order.splice(order.begin(), order, f->second.it);
                const size_t s = f->second.slot;
                if (fill_pending[s]) { // a prefetch still copying it in
                    (void)hipStreamWaitEvent(st, fill[s], 0);
                    fill_pending[s] = 0;
                }
                *dev = slab + s * slot_bytes;
                return LOOMHIP_OK;
            }
        }
        const size_t s = take_slot(st);
        uint8_t *dst = slab + s * slot_bytes;
        if (hipError_t e = copy_in(k, dst, staging, st); e != hipSuccess) {
            free_slots.push_back(s);
            return hip_fail(e, "moe_ffn_block: fill");
        }
        if (keep) {
            order.push_front(k);
            map[k] = Entry{s, order.begin()};
        } else {
            transient.push_back(s); // freed when the call's work is done
        }
        misses++;
        bytes_read += k.len;
        *dev = dst;
        return LOOMHIP_OK;
    }
    // prefetchAsync for one arena slice: start its fill on the copy stream.
    int prefetch(const SliceKey &k, hipStream_t copy) {
        if (!in_arena(k.ptr, k.len) || map.count(k))
            return LOOMHIP_OK;
        const size_t s = take_slot(copy);
        uint8_t *dst = slab + s * slot_bytes;
        if (hipError_t e = copy_in(k, dst, staging_copy, copy); e != hipSuccess) {
            free_slots.push_back(s);
            return hip_fail(e, "moe_ffn_block: prefetch");
        }
        (void)hipEventRecord(fill[s], copy);
        fill_pending[s] = 1;
        order.push_front(k);
        map[k] = Entry{s, order.begin()};
        prefetched++;
        bytes_read += k.len;
        return LOOMHIP_OK;
    }
    void end_call() { // after the call's stream is synchronised
        for (size_t s : transient)
            free_slots.push_back(s);
        transient.clear();
    }
};

static BlockLru g_block;
static Scratch g_block_ws;

void block_release_cache() {
    g_block.release();
    g_block_ws.release();
    g_n_arenas = 0;
}

// out[i] = sum over r in order of w[r] * y[r][i], from +0 (the reference's
// acc += gate * ffn_out, deepseek.zig:1485-1487)
__global__ __launch_bounds__(256) void block_combine_kernel(const float *__restrict__ y, int n, int dim,
                                                            const float *__restrict__ w, float *__restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim)
        return;
    float acc = 0.0f;
    for (int r = 0; r < n; r++) {
        const float p = w[r] * y[(size_t)r * dim + i];
        acc = acc + p;
    }
    out[i] = acc;
}

} // namespace lh

using namespace lh;

extern "C" {

int loomhip_moe_ffn_block(const float *normed, size_t dim, const loomhip_expert_ref *experts, size_t n_experts,
                          float *out) {
    if (int rc = require_ready())
        return rc;
    if (!normed || !out || (n_experts && !experts))
        return fail(LOOMHIP_ERR_ARG, "moe_ffn_block: null argument");
    if (n_experts == 0 || n_experts > BLOCK_MAX_EXPERTS)
        return fail(LOOMHIP_DECLINED, "moe_ffn_block: %zu experts (1..%zu served)", n_experts, BLOCK_MAX_EXPERTS);
    // resolve everything before recording anything (src/metal/backend.zig:2337-2353)
    size_t widest = 0, biggest = 0;
    for (size_t r = 0; r < n_experts; r++) {
        const loomhip_expert_ref &x = experts[r];
        if (!x.gate || !x.up || !x.down)
            return fail(LOOMHIP_ERR_ARG, "moe_ffn_block: expert %zu has a null tensor", r);
        const DenseFfn probe{x.gate_t, x.up_t, x.down_t, x.gate, x.up, x.down, x.ffn};
        if (int rc = dense_ffn_check(probe, dim))
            return rc;
        widest = x.ffn > widest ? x.ffn : widest;
        const size_t gb = plane_bytes(x.gate_t, x.ffn, dim), db = plane_bytes(x.down_t, dim, x.ffn);
        biggest = gb > biggest ? gb : biggest;
        biggest = db > biggest ? db : biggest;
    }
    hipStream_t st = g_ctx.compute;
    if (int rc = g_block.reserve(align16(biggest)))
        return rc;
    const size_t xb = align16(dim * 4), yb = align16(n_experts * dim * 4), wb = align16(n_experts * 4);
    if (int rc = g_block_ws.reserve(xb + yb + wb + xb))
        return rc;
    char *base = (char *)g_block_ws.ptr;
    float *dx = (float *)base, *dy = (float *)(base + xb), *dw = (float *)(base + xb + yb);
    float *dout = (float *)(base + xb + yb + wb);
    float hw[BLOCK_MAX_EXPERTS];
    for (size_t r = 0; r < n_experts; r++)
        hw[r] = experts[r].weight;
    hipError_t e = hipMemcpyAsync(dx, normed, dim * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dw, hw, n_experts * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_ffn_block: staging");
    for (size_t r = 0; r < n_experts; r++) {
        const loomhip_expert_ref &x = experts[r];
        const size_t gl = ggml_bytes(x.gate_t, x.ffn, dim), ul = ggml_bytes(x.up_t, x.ffn, dim);
        const size_t dl = ggml_bytes(x.down_t, dim, x.ffn);
        DenseFfn f{x.gate_t, x.up_t, x.down_t, nullptr, nullptr, nullptr, x.ffn};
        int rc;
        if ((rc = g_block.get(SliceKey{x.gate, gl, x.gate_t, x.ffn, dim}, st, &f.gate)) ||
            (rc = g_block.get(SliceKey{x.up, ul, x.up_t, x.ffn, dim}, st, &f.up)) ||
            (rc = g_block.get(SliceKey{x.down, dl, x.down_t, dim, x.ffn}, st, &f.down)) ||
            (rc = dense_ffn_add(f, dx, 1, dim, dy + r * dim, st, false))) {
            (void)hipStreamSynchronize(st); // what was enqueued finishes before its slots are reused
            g_block.end_call();
            return rc;
        }
    }
    hipLaunchKernelGGL(block_combine_kernel, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, st, dy,
                       (int)n_experts, (int)dim, dw, dout);
    note_launch();
    e = hipMemcpyAsync(out, dout, dim * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    g_block.end_call();
    if (e != hipSuccess)
        return hip_fail(e, "moe_ffn_block: readback");
    return LOOMHIP_OK;
}

int loomhip_moe_ffn_block_prefetch(size_t dim, const loomhip_expert_ref *experts, size_t n_experts) {
    if (int rc = require_ready())
        return rc;
    if (n_experts && !experts)
        return fail(LOOMHIP_ERR_ARG, "moe_ffn_block_prefetch: null argument");
    size_t biggest = 0;
    for (size_t r = 0; r < n_experts; r++) {
        const loomhip_expert_ref &x = experts[r];
        if (!x.gate || !x.up || !x.down)
            return fail(LOOMHIP_ERR_ARG, "moe_ffn_block_prefetch: expert %zu has a null tensor", r);
        const DenseFfn probe{x.gate_t, x.up_t, x.down_t, x.gate, x.up, x.down, x.ffn};
        if (int rc = dense_ffn_check(probe, dim))
            return rc;
        const size_t gb = plane_bytes(x.gate_t, x.ffn, dim), db = plane_bytes(x.down_t, dim, x.ffn);
        biggest = std::max(biggest, std::max(gb, db));
    }
    if (biggest > g_block.slot_bytes) // the cache re-sizes (and empties) on the call that needs it
        return LOOMHIP_OK;
    hipStream_t cp = g_ctx.copy;
    for (size_t r = 0; r < n_experts; r++) {
        const loomhip_expert_ref &x = experts[r];
        const size_t gl = ggml_bytes(x.gate_t, x.ffn, dim), ul = ggml_bytes(x.up_t, x.ffn, dim);
        const size_t dl = ggml_bytes(x.down_t, dim, x.ffn);
        int rc;
        if ((rc = g_block.prefetch(SliceKey{x.gate, gl, x.gate_t, x.ffn, dim}, cp)) ||
            (rc = g_block.prefetch(SliceKey{x.up, ul, x.up_t, x.ffn, dim}, cp)) ||
            (rc = g_block.prefetch(SliceKey{x.down, dl, x.down_t, dim, x.ffn}, cp)))
            return rc;
    }
    return LOOMHIP_OK;
}

int loomhip_register_arena(const void *mem, size_t len) {
    if (!mem || !len)
        return fail(LOOMHIP_ERR_ARG, "register_arena: empty region");
    const uintptr_t page = 4096;
    const uintptr_t base = (uintptr_t)mem & ~(page - 1);
    const uintptr_t end = ((uintptr_t)mem + len + page - 1) & ~(page - 1);
    for (int i = 0; i < g_n_arenas; i++) // already covered: not an error
        if (base >= g_arenas[i].base && end <= g_arenas[i].base + g_arenas[i].len)
            return LOOMHIP_OK;
    if (g_n_arenas == MAX_ARENAS)
        return fail(LOOMHIP_DECLINED, "register_arena: %d regions registered", MAX_ARENAS);
    g_arenas[g_n_arenas++] = Arena{base, (size_t)(end - base)};
    return LOOMHIP_OK;
}

size_t loomhip_materialize_arenas(void) {
    size_t total = 0;
    for (int i = 0; i < g_n_arenas; i++)
        total += g_arenas[i].len;
    return total;
}

int loomhip_moe_ffn_block_stats(uint64_t *hits, uint64_t *misses, uint64_t *bytes_read) {
    if (!hits || !misses || !bytes_read)
        return fail(LOOMHIP_ERR_ARG, "moe_ffn_block_stats: null argument");
    *hits = g_block.hits;
    *misses = g_block.misses;
    *bytes_read = g_block.bytes_read;
    return LOOMHIP_OK;
}

} // extern "C"
