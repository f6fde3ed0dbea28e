// expert_block.hip -- backend.moeFfnBlock (src/compute/cpu.zig:23-30; the
// Metal form src/metal/backend.zig:2322-2410): one MoE layer's selected
// experts, and the shared one, handed over as host tensor slices with their
// router weights; out = the sum, in list order, of weight * FFN(normed).  The
// caller (src/gguf/deepseek.zig:1405-1440) builds the list from its expert
// Source, whose slices stay valid for the call (stablePointers).
//
// Residency: each tensor slice resolves to a slot of an HBM LRU keyed by the
// slice (host pointer, length, type, shape): a hit uses the slot as is; a miss
// copies the GGML bytes into the slot (Q4_K keeps GGML's layout) or through a
// staging buffer and the device-layout repack (Q6_K, Q8_0, Q4_0).  The slots
// are sized by the largest tensor seen; a larger one empties the cache and
// re-sizes it.  Then, per expert, the fused gate/up SwiGLU matvec, the
// activations' quantization and the down matvec (all bit-identical to the CPU
// kernels), and one weighted combine in list order.  One stream-ordered
// submission; synchronous at the seam, like the reference's.
#include "runtime.hpp"

#include <list>
#include <unordered_map>

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

struct BlockLru {
    uint8_t *slab = nullptr, *staging = nullptr;
    size_t slot_bytes = 0, n_slots = 0, used = 0;
    std::list<SliceKey> order; // front = most recent
    struct Entry {
        size_t slot;
        std::list<SliceKey>::iterator it;
    };
    std::unordered_map<SliceKey, Entry, SliceHash> map;
    uint64_t hits = 0, misses = 0, bytes_read = 0;

    void release() {
        if (slab)
            (void)hipFree(slab);
        if (staging)
            (void)hipFree(staging);
        slab = staging = nullptr;
        slot_bytes = n_slots = used = 0;
        order.clear();
        map.clear();
    }
    int reserve(size_t bytes, hipStream_t st) {
        if (bytes <= slot_bytes)
            return LOOMHIP_OK;
        (void)hipStreamSynchronize(st);
        release();
        hipError_t e = hipMalloc((void **)&slab, bytes * BLOCK_LRU_SLOTS);
        if (e == hipSuccess)
            e = hipMalloc((void **)&staging, bytes);
        if (e != hipSuccess) {
            release();
            return hip_fail(e, "moe_ffn_block: HBM cache");
        }
        slot_bytes = bytes;
        n_slots = BLOCK_LRU_SLOTS;
        return LOOMHIP_OK;
    }
    // The device-layout copy of a host tensor slice; misses fill on st.
    int get(const SliceKey &k, hipStream_t st, const void **dev) {
        auto f = map.find(k);
        if (f != map.end()) {
            hits++;
            order.splice(order.begin(), order, f->second.it);
            *dev = slab + f->second.slot * slot_bytes;
            return LOOMHIP_OK;
        }
        size_t s;
        if (used < n_slots) {
            s = used++;
        } else { // evict the least recently used; earlier work on st is ordered before the refill
            const SliceKey victim = order.back();
            s = map[victim].slot;
            map.erase(victim);
            order.pop_back();
        }
        uint8_t *dst = slab + s * slot_bytes;
        hipError_t e;
        if (k.t == LH_Q4_K) {
            e = hipMemcpyAsync(dst, k.ptr, k.len, hipMemcpyHostToDevice, st);
        } else {
            e = hipMemcpyAsync(staging, k.ptr, k.len, hipMemcpyHostToDevice, st);
            if (e == hipSuccess)
                launch_repack(k.t, staging, dst, k.rows, k.cols, 1, st);
        }
        if (e != hipSuccess)
            return hip_fail(e, "moe_ffn_block: fill");
        order.push_front(k);
        map[k] = Entry{s, order.begin()};
        misses++;
        bytes_read += k.len;
        *dev = dst;
        return LOOMHIP_OK;
    }
};

static BlockLru g_block;
static Scratch g_block_ws;

void block_release_cache() {
    g_block.release();
    g_block_ws.release();
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
    if (int rc = g_block.reserve(align16(biggest), st))
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
            (rc = g_block.get(SliceKey{x.down, dl, x.down_t, dim, x.ffn}, st, &f.down)))
            return rc;
        if ((rc = dense_ffn_add(f, dx, 1, dim, dy + r * dim, st, false)))
            return rc;
    }
    hipLaunchKernelGGL(block_combine_kernel, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, st, dy,
                       (int)n_experts, (int)dim, dw, dout);
    note_launch();
    e = hipMemcpyAsync(out, dout, dim * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_ffn_block: readback");
    return LOOMHIP_OK;
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
