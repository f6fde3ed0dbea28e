// expert_cache.hip -- the HBM tier of Loom's expert cache and the routed MoE
// layer that reads its experts through it.
//
// Bookkeeping (host): ExpertCache of src/engine/expert_cache.zig:150-249 --
// a pinned set, then an intrusive LRU over `capacity` slots (Lru, 39-148),
// then the backing block.  Storage: one HBM slab of (capacity + pin_slots)
// slots of slot_bytes; slots [0, capacity) belong to the LRU, the rest to
// the pinned set.  The backing store is pinned host memory, read by
// hipMemcpyAsync on the library's copy stream.
//
// Ordering.  A fill is the copy stream's work; the consumer's stream waits
// on an event recorded after the fill.  Each slot also keeps the event of
// its last use: loomhip_ec_release records it precisely after the kernels
// that read the slot; a slot evicted while still marked "in use, not
// released" gets an event recorded on its consumer stream at eviction time
// (everything enqueued there so far).  The refill copy waits on that event,
// so a slot is never overwritten under a kernel still reading it.
#include "runtime.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

namespace lh {

constexpr size_t EC_NIL = (size_t)-1;

struct EcSlot {
    size_t id = EC_NIL;
    size_t prev = EC_NIL, next = EC_NIL;
    hipEvent_t last_use = nullptr; // recorded after the slot's latest released use
    bool has_use = false;          // last_use has been recorded at least once
    bool open = false;                 // handed out, not yet released
    hipStream_t open_stream = nullptr; // ... on this stream (may be the null stream)
    hipEvent_t fill = nullptr;         // recorded on the copy stream after the slot's latest fill
    bool fill_pending = false;         // that fill may still be in flight
};

} // namespace lh

struct loomhip_ec {
    size_t capacity = 0, pin_slots = 0, slot_bytes = 0, n_ids = 0;
    uint8_t *slab = nullptr;
    std::vector<lh::EcSlot> slot;   // capacity + pin_slots
    std::vector<size_t> map;        // id -> LRU slot or EC_NIL
    std::vector<size_t> pin_of;     // id -> pinned slot or EC_NIL
    size_t head = lh::EC_NIL, tail = lh::EC_NIL, free_top = 0, n_pinned = 0;
    std::vector<const void *> src;
    std::vector<size_t> src_len;
    std::vector<uint64_t> access;
    std::vector<size_t> open; // slots handed out since the last release
    loomhip_ec_stats stats{};
};

namespace lh {

// ---- Lru (expert_cache.zig:39-148) -------------------------------------------------

static void lru_unlink(loomhip_ec *c, size_t s) {
    const size_t p = c->slot[s].prev, n = c->slot[s].next;
    if (p != EC_NIL)
        c->slot[p].next = n;
    else
        c->head = n;
    if (n != EC_NIL)
        c->slot[n].prev = p;
    else
        c->tail = p;
}

static void lru_push_front(loomhip_ec *c, size_t s) {
    c->slot[s].prev = EC_NIL;
    c->slot[s].next = c->head;
    if (c->head != EC_NIL)
        c->slot[c->head].prev = s;
    c->head = s;
    if (c->tail == EC_NIL)
        c->tail = s;
}

// find (97-103): a hit becomes the most recently used.
static size_t lru_find(loomhip_ec *c, size_t id) {
    const size_t s = c->map[id];
    if (s == EC_NIL)
        return EC_NIL;
    if (c->head != s) {
        lru_unlink(c, s);
        lru_push_front(c, s);
    }
    return s;
}

// reserve (107-123): a never-used slot first, else evict the tail.
// *evicted = the slot's previous id, or EC_NIL.
static size_t lru_reserve(loomhip_ec *c, size_t id, size_t *evicted) {
    *evicted = EC_NIL;
    if (c->capacity == 0)
        return EC_NIL;
    size_t s;
    if (c->free_top < c->capacity) {
        s = c->free_top++;
    } else {
        s = c->tail;
        lru_unlink(c, s);
        *evicted = c->slot[s].id;
        c->map[c->slot[s].id] = EC_NIL;
    }
    c->slot[s].id = id;
    c->map[id] = s;
    lru_push_front(c, s);
    return s;
}

// abort (138-147): unpublish a failed fill.
static void lru_abort(loomhip_ec *c, size_t id) {
    const size_t s = c->map[id];
    if (s == EC_NIL)
        return;
    c->map[id] = EC_NIL;
    lru_unlink(c, s);
    c->slot[s].id = EC_NIL;
    if (s + 1 == c->free_top)
        c->free_top--;
}

static uint8_t *slot_ptr(const loomhip_ec *c, size_t s) { return c->slab + s * c->slot_bytes; }

// The fill of slot s from id's source on the copy stream, after the slot's
// previous uses; when `wait`, `consumer` (may be the null stream) then
// waits for the fill.
static int fill_slot(loomhip_ec *c, size_t s, size_t id, bool wait, hipStream_t consumer) {
    EcSlot &sl = c->slot[s];
    hipError_t e = hipSuccess;
    if (sl.open) { // handed out and not released: everything enqueued there so far
        e = hipEventRecord(sl.last_use, sl.open_stream);
        sl.has_use = e == hipSuccess;
        sl.open = false;
    }
    if (e == hipSuccess && sl.has_use)
        e = hipStreamWaitEvent(g_ctx.copy, sl.last_use, 0);
    if (e == hipSuccess)
        e = hipMemcpyAsync(slot_ptr(c, s), c->src[id], c->src_len[id], hipMemcpyHostToDevice, g_ctx.copy);
    if (e == hipSuccess)
        e = hipEventRecord(sl.fill, g_ctx.copy);
    sl.fill_pending = e == hipSuccess;
    if (e == hipSuccess && wait)
        e = hipStreamWaitEvent(consumer, sl.fill, 0);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "expert cache fill");
}

// A hit on a slot whose fill (a prefetch, or a miss taken on another stream)
// may still be in flight: the consumer's stream waits for that fill.
static int wait_fill(EcSlot &sl, hipStream_t consumer) {
    if (!sl.fill_pending)
        return LOOMHIP_OK;
    hipError_t e = hipEventQuery(sl.fill);
    if (e == hipSuccess) {
        sl.fill_pending = false;
        return LOOMHIP_OK;
    }
    if (e != hipErrorNotReady)
        return hip_fail(e, "expert cache fill query");
    e = hipStreamWaitEvent(consumer, sl.fill, 0);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "expert cache fill wait");
}

static void mark_open(loomhip_ec *c, size_t s, hipStream_t st) {
    EcSlot &sl = c->slot[s];
    if (!sl.open)
        c->open.push_back(s);
    sl.open = true;
    sl.open_stream = st;
}

static int ec_get(loomhip_ec *c, size_t id, hipStream_t st, size_t *slot_out) {
    c->access[id] += 1;
    if (c->pin_of[id] != EC_NIL) {
        c->stats.pin_hits += 1;
        *slot_out = c->pin_of[id];
        return LOOMHIP_OK;
    }
    size_t s = lru_find(c, id);
    if (s != EC_NIL) {
        c->stats.lru_hits += 1;
        if (int rc = wait_fill(c->slot[s], st))
            return rc;
        mark_open(c, s, st);
        *slot_out = s;
        return LOOMHIP_OK;
    }
    size_t evicted;
    s = lru_reserve(c, id, &evicted);
    if (s == EC_NIL)
        return fail(LOOMHIP_ERR_ARG, "expert cache: no capacity");
    if (!c->src[id]) {
        lru_abort(c, id);
        return fail(LOOMHIP_ERR_ARG, "expert cache: expert %zu has no backing block", id);
    }
    if (int rc = fill_slot(c, s, id, true, st)) {
        lru_abort(c, id);
        return rc;
    }
    c->stats.misses += 1;
    c->stats.bytes_read += c->src_len[id];
    mark_open(c, s, st);
    *slot_out = s;
    return LOOMHIP_OK;
}

static int ec_release(loomhip_ec *c, hipStream_t st) {
    for (size_t s : c->open) {
        EcSlot &sl = c->slot[s];
        if (!sl.open)
            continue;
        const hipError_t e = hipEventRecord(sl.last_use, st);
        if (e != hipSuccess)
            return hip_fail(e, "expert cache release");
        sl.has_use = true;
        sl.open = false;
    }
    c->open.clear();
    return LOOMHIP_OK;
}

// ---- the cached MoE layer -----------------------------------------------------------

// out[t] = (init ? +0 : out[t]) + sum over the token's entries, in list
// order, of gate * y[pair] (tensor.zig add order: acc = acc + g * v).
__global__ __launch_bounds__(256) void ec_combine_kernel(const float *__restrict__ y,
                                                         const int *__restrict__ first,
                                                         const int *__restrict__ pair,
                                                         const float *__restrict__ gate, int dim,
                                                         int init, float *__restrict__ out) {
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim)
        return;
    float *o = out + (size_t)t * dim + i;
    float acc = init ? 0.0f : *o;
    for (int j = first[t]; j < first[t + 1]; j++) {
        const float pr = gate[j] * y[(size_t)pair[j] * dim + i];
        acc = acc + pr;
    }
    *o = acc;
}

static Scratch g_ec_dev;                 // device workspace of the cached layer
static void *g_ec_host = nullptr;        // pinned staging: ids/gates back, tables out
static size_t g_ec_host_cap = 0;
static hipEvent_t g_ec_tables_done = nullptr; // the last table upload has been consumed

static int ec_host_reserve(size_t bytes) {
    if (bytes <= g_ec_host_cap)
        return LOOMHIP_OK;
    if (g_ec_tables_done)
        (void)hipEventSynchronize(g_ec_tables_done);
    if (g_ec_host)
        (void)hipHostFree(g_ec_host);
    g_ec_host = nullptr;
    g_ec_host_cap = 0;
    const hipError_t e = hipHostMalloc(&g_ec_host, bytes, hipHostMallocDefault);
    if (e != hipSuccess)
        return hip_fail(e, "expert cache staging");
    g_ec_host_cap = bytes;
    return LOOMHIP_OK;
}

void ec_release_scratch() {
    g_ec_dev.release();
    if (g_ec_host)
        (void)hipHostFree(g_ec_host);
    g_ec_host = nullptr;
    g_ec_host_cap = 0;
    if (g_ec_tables_done)
        (void)hipEventDestroy(g_ec_tables_done);
    g_ec_tables_done = nullptr;
}

struct EcEntry {
    int expert;
    int first, n; // pairs [first, first + n) of the entry in the call's pair order
};

static int moe_cached(const loomhip_moe_layer_ec &L, loomhip_ec *c, const float *normed, size_t n,
                      float *out, uint32_t *ids_out, float *gates_out, hipStream_t st) {
    const size_t k = L.n_used, E = L.n_expert, P = n * k;
    if (!gate_supported((int)n, (int)E, (int)k))
        return fail(LOOMHIP_DECLINED, "moe_cached: %zu tokens / %zu experts / top-%zu not served", n, E, k);
    if (!dmmv_supported(L.gate_t, (int)L.dim) || !dmmv_supported(L.down_t, (int)L.ffn) || L.dim % 32 ||
        L.ffn % 32)
        return fail(LOOMHIP_DECLINED, "moe_cached: shapes dim %zu / ffn %zu not served", L.dim, L.ffn);
    const size_t gu_bytes = plane_bytes(L.gate_t, L.ffn, L.dim), dn_bytes = plane_bytes(L.down_t, L.dim, L.ffn);
    if (L.gate_off + gu_bytes > c->slot_bytes || L.up_off + gu_bytes > c->slot_bytes ||
        L.down_off + dn_bytes > c->slot_bytes)
        return fail(LOOMHIP_ERR_ARG, "moe_cached: expert tensors exceed the slot (%zu B)", c->slot_bytes);
    if (L.id_base + E > c->n_ids)
        return fail(LOOMHIP_ERR_ARG, "moe_cached: ids [%zu, %zu) exceed the cache's %zu", L.id_base,
                    L.id_base + E, c->n_ids);
    if (c->capacity == 0 && c->n_pinned == 0)
        return fail(LOOMHIP_ERR_ARG, "moe_cached: empty cache");
    const DenseFfn sh{L.shexp_gate_t, L.shexp_up_t, L.shexp_down_t, L.shexp_gate, L.shexp_up, L.shexp_down,
                      L.shexp_ffn};
    if (sh.gate)
        if (int rc = dense_ffn_check(sh, L.dim))
            return rc;
    const int nt = n == 1 ? 1 : pick_nt((int)n);

    // device workspace
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += align16(bytes);
        return o;
    };
    const size_t o_qx = take(align16(n * L.dim) + align16(n * (L.dim / 32) * 4) + align16(n * (L.dim / 16) * 4));
    const size_t o_log = take(n * E * 4), o_ids = take(P * 4), o_gates = take(P * 4);
    const size_t o_act = take(P * L.ffn * 4);
    const size_t o_qa = take(align16(P * L.ffn) + align16(P * (L.ffn / 32) * 4) + align16(P * (L.ffn / 16) * 4));
    const size_t o_y = take(P * L.dim * 4);
    // tables: pair_src[P], groups[P], first[n + 1], pair[P], gate[P] per round
    const size_t tab_bytes = align16(P * 4) + align16(P * sizeof(DmmvGroup)) + align16((n + 1) * 4) +
                             align16(P * 4) + align16(P * 4);
    // one table region per round: at most ceil(P / capacity) rounds
    const size_t n_tabs = (c->capacity ? (P + c->capacity - 1) / c->capacity : 1) + 1;
    const size_t o_tab = take(tab_bytes * n_tabs);
    if (int rc = g_ec_dev.reserve(off))
        return rc;
    char *base = (char *)g_ec_dev.ptr;
    QAct qx;
    qx.q = (int8_t *)(base + o_qx);
    qx.d = (float *)(base + o_qx + align16(n * L.dim));
    qx.s = (int32_t *)((char *)qx.d + align16(n * (L.dim / 32) * 4));
    QAct qa;
    qa.q = (int8_t *)(base + o_qa);
    qa.d = (float *)(base + o_qa + align16(P * L.ffn));
    qa.s = (int32_t *)((char *)qa.d + align16(P * (L.ffn / 32) * 4));
    uint32_t *d_ids = (uint32_t *)(base + o_ids);
    float *d_gates = (float *)(base + o_gates);
    float *act = (float *)(base + o_act), *y = (float *)(base + o_y);

    // route on the device, ids and gates to the host
    const size_t host_need = 2 * align16(P * 4) + tab_bytes * n_tabs;
    if (int rc = ec_host_reserve(host_need))
        return rc;
    if (g_ec_tables_done)
        (void)hipEventSynchronize(g_ec_tables_done); // the previous call's tables were read
    else if (hipEventCreateWithFlags(&g_ec_tables_done, hipEventDisableTiming) != hipSuccess)
        return fail(LOOMHIP_ERR_HIP, "moe_cached: event");
    uint32_t *h_ids = (uint32_t *)g_ec_host;
    float *h_gates = (float *)((char *)g_ec_host + align16(P * 4));
    char *h_tab = (char *)g_ec_host + 2 * align16(P * 4);

    GateParams gp{};
    gp.router = L.router;
    gp.router_bias = L.router_bias;
    gp.sel_bias = L.sel_bias;
    gp.x = normed;
    gp.n = (int)n;
    gp.dim = (int)L.dim;
    gp.n_expert = (int)E;
    gp.k = (int)k;
    gp.gating = L.gating;
    gp.weights_norm = L.weights_norm;
    gp.weights_scale = L.weights_scale;
    gp.logits = (float *)(base + o_log);
    gp.ids = d_ids;
    gp.gates = d_gates;
    gp.qt = L.gate_t;
    gp.qx = qx;
    gp.nt = nt;
    gp.sync = g_ctx.sync;
    gp.chain = 1; // route only: b.n_groups stays null
    launch_gate(gp, st);
    hipError_t e = hipMemcpyAsync(h_ids, d_ids, P * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(h_gates, d_gates, P * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_cached: ids readback");
    if (ids_out)
        memcpy(ids_out, h_ids, P * 4);
    if (gates_out)
        memcpy(gates_out, h_gates, P * 4);

    // the access list: n == 1, moeFFN's selection order; else distinct
    // experts ascending, each with its (token, slot) pairs in token order
    std::vector<EcEntry> list;
    std::vector<int> pair_tok, pair_slot; // pair -> token, selection slot
    if (n == 1) {
        for (size_t s = 0; s < k; s++) {
            list.push_back({(int)h_ids[s], (int)s, 1});
            pair_tok.push_back(0);
            pair_slot.push_back((int)s);
        }
    } else {
        std::vector<int> cnt(E, 0);
        for (size_t p = 0; p < P; p++)
            if (h_ids[p] < E)
                cnt[h_ids[p]]++;
        std::vector<int> at(E, 0);
        int acc = 0;
        for (size_t ex = 0; ex < E; ex++) {
            at[ex] = acc;
            if (cnt[ex])
                list.push_back({(int)ex, acc, cnt[ex]});
            acc += cnt[ex];
        }
        pair_tok.assign(acc, 0);
        pair_slot.assign(acc, 0);
        for (size_t t = 0; t < n; t++)
            for (size_t s = 0; s < k; s++) {
                const uint32_t ex = h_ids[t * k + s];
                if (ex >= E)
                    continue;
                const int p = at[ex]++;
                pair_tok[p] = (int)t;
                pair_slot[p] = (int)s;
            }
    }
    // Every exit from here on records g_ec_tables_done after the table
    // uploads already enqueued, so the next call waits for them before it
    // rewrites the pinned staging; after a failed call `out` is undefined.
    auto tables_done = [&](int rc) {
        (void)hipEventRecord(g_ec_tables_done, st);
        return rc;
    };
    const size_t cap = c->capacity ? c->capacity : list.size();
    bool first_round = true;
    size_t tab_i = 0;
    for (size_t r0 = 0; r0 < list.size() || first_round; r0 += cap, tab_i++) {
        const size_t r1 = std::min(list.size(), r0 + cap);
        // gets, in list order
        std::vector<int> plane(r1 - r0);
        for (size_t i = r0; i < r1; i++) {
            size_t s;
            if (int rc = ec_get(c, L.id_base + (size_t)list[i].expert, st, &s))
                return tables_done(rc);
            plane[i - r0] = (int)s;
        }
        // tables of this round
        const int p0 = r0 < r1 ? list[r0].first : 0;
        const int np = r0 < r1 ? list[r1 - 1].first + list[r1 - 1].n - p0 : 0;
        char *ht = h_tab + tab_i * tab_bytes;
        int *t_src = (int *)ht;
        DmmvGroup *t_groups = (DmmvGroup *)(ht + align16(P * 4));
        int *t_first = (int *)((char *)t_groups + align16(P * sizeof(DmmvGroup)));
        int *t_pair = (int *)((char *)t_first + align16((n + 1) * 4));
        float *t_gate = (float *)((char *)t_pair + align16(P * 4));
        int ng = 0;
        for (size_t i = r0; i < r1; i++)
            for (int j = 0; j < list[i].n; j += nt)
                t_groups[ng++] = DmmvGroup{plane[i - r0], list[i].first - p0 + j, std::min(nt, list[i].n - j)};
        for (int p = 0; p < np; p++)
            t_src[p] = pair_tok[p0 + p];
        // per token, its pairs of this round in list order
        std::vector<int> per(n + 1, 0);
        for (int p = 0; p < np; p++)
            per[pair_tok[p0 + p] + 1]++;
        for (size_t t = 0; t < n; t++)
            per[t + 1] += per[t];
        for (size_t t = 0; t <= n; t++)
            t_first[t] = per[t];
        for (int p = 0; p < np; p++) {
            const int t = pair_tok[p0 + p];
            const int j = per[t]++;
            t_pair[j] = p;
            t_gate[j] = h_gates[(size_t)t * k + pair_slot[p0 + p]];
        }
        char *dt = base + o_tab + tab_i * tab_bytes;
        e = hipMemcpyAsync(dt, ht, tab_bytes, hipMemcpyHostToDevice, st);
        if (e != hipSuccess)
            return tables_done(hip_fail(e, "moe_cached: tables"));
        const int *d_src = (const int *)dt;
        const DmmvGroup *d_groups = (const DmmvGroup *)(dt + align16(P * 4));
        const int *d_first = (const int *)((const char *)d_groups + align16(P * sizeof(DmmvGroup)));
        const int *d_pair = (const int *)((const char *)d_first + align16((n + 1) * 4));
        const float *d_gate = (const float *)((const char *)d_pair + align16(P * 4));
        if (np > 0) {
            DmmvParams gu{};
            gu.w = c->slab + L.gate_off;
            gu.w2 = c->slab + L.up_off;
            gu.plane_bytes = c->slot_bytes;
            gu.rows = (int)L.ffn;
            gu.cols = (int)L.dim;
            gu.xq = qx.q;
            gu.xd = qx.d;
            gu.xs = qx.s;
            gu.pair_src = d_src;
            gu.pair_dst = g_ctx.iota;
            gu.groups = d_groups;
            gu.n_groups = ng;
            gu.out = act;
            gu.out_stride = (int)L.ffn;
            gu.rpw = dmmv_pick_rpw(L.gate_t, (int)L.dim, (int)L.ffn, ng, nt, true);
            int ph = prof_begin(LOOMHIP_KT_GATE_UP, st);
            bool ok = launch_dmmv(L.gate_t, nt, true, gu, st);
            prof_end(ph, st);
            if (!ok)
                return tables_done(fail(LOOMHIP_ERR_ARG, "moe_cached: gate/up partials exceed LDS"));
            launch_quant_act(L.down_t, act, (int)L.ffn, (int)L.ffn, np, qa, st);
            DmmvParams dn{};
            dn.w = c->slab + L.down_off;
            dn.plane_bytes = c->slot_bytes;
            dn.rows = (int)L.dim;
            dn.cols = (int)L.ffn;
            dn.xq = qa.q;
            dn.xd = qa.d;
            dn.xs = qa.s;
            dn.pair_src = g_ctx.iota;
            dn.pair_dst = g_ctx.iota;
            dn.groups = d_groups;
            dn.n_groups = ng;
            dn.out = y;
            dn.out_stride = (int)L.dim;
            dn.rpw = dmmv_pick_rpw(L.down_t, (int)L.ffn, (int)L.dim, ng, nt, false);
            ph = prof_begin(LOOMHIP_KT_DOWN, st);
            ok = launch_dmmv(L.down_t, nt, false, dn, st);
            prof_end(ph, st);
            if (!ok)
                return tables_done(fail(LOOMHIP_ERR_ARG, "moe_cached: down partials exceed LDS"));
        }
        hipLaunchKernelGGL(ec_combine_kernel, dim3((L.dim + 255) / 256, n), dim3(256), 0, st, y, d_first,
                           d_pair, d_gate, (int)L.dim, first_round ? 1 : 0, out);
        note_launch();
        if (int rc = ec_release(c, st))
            return tables_done(rc);
        first_round = false;
        if (r1 >= list.size())
            break;
    }
    e = hipEventRecord(g_ec_tables_done, st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_cached: event");
    // the shared expert (resident), after the routed sum (deepseek.zig:1497-1502)
    return sh.gate ? dense_ffn_add(sh, normed, n, L.dim, out, st, true) : LOOMHIP_OK;
}

} // namespace lh

using namespace lh;

extern "C" {

void *loomhip_host_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
        fail(LOOMHIP_ERR_HIP, "hipHostMalloc of %zu bytes failed", bytes);
        return nullptr;
    }
    return p;
}

void loomhip_host_free(void *p) {
    if (p)
        (void)hipHostFree(p);
}

int loomhip_ec_create(size_t capacity, size_t pin_slots, size_t slot_bytes, size_t n_ids,
                      loomhip_ec **out) {
    if (int rc = require_ready())
        return rc;
    if (!out || slot_bytes == 0 || n_ids == 0 || capacity + pin_slots == 0)
        return fail(LOOMHIP_ERR_ARG, "ec_create: bad arguments");
    *out = nullptr;
    loomhip_ec *c = new loomhip_ec();
    c->capacity = capacity;
    c->pin_slots = pin_slots;
    c->slot_bytes = align16(slot_bytes);
    c->n_ids = n_ids;
    c->slot.resize(capacity + pin_slots);
    c->map.assign(n_ids, EC_NIL);
    c->pin_of.assign(n_ids, EC_NIL);
    c->src.assign(n_ids, nullptr);
    c->src_len.assign(n_ids, 0);
    c->access.assign(n_ids, 0);
    hipError_t e = hipMalloc((void **)&c->slab, c->slot_bytes * (capacity + pin_slots));
    for (size_t s = 0; e == hipSuccess && s < c->slot.size(); s++) {
        e = hipEventCreateWithFlags(&c->slot[s].last_use, hipEventDisableTiming);
        if (e == hipSuccess)
            e = hipEventCreateWithFlags(&c->slot[s].fill, hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        loomhip_ec_destroy(c);
        return hip_fail(e, "ec_create");
    }
    *out = c;
    return LOOMHIP_OK;
}

void loomhip_ec_destroy(loomhip_ec *c) {
    if (!c)
        return;
    (void)hipDeviceSynchronize(); // no copy or kernel may still touch the slab
    for (auto &s : c->slot) {
        if (s.last_use)
            (void)hipEventDestroy(s.last_use);
        if (s.fill)
            (void)hipEventDestroy(s.fill);
    }
    if (c->slab)
        (void)hipFree(c->slab);
    delete c;
}

int loomhip_ec_set_source(loomhip_ec *c, size_t id, const void *host, size_t len) {
    if (!c || id >= c->n_ids || !host || len == 0 || len > c->slot_bytes)
        return fail(LOOMHIP_ERR_ARG, "ec_set_source: bad arguments (id %zu, len %zu)", id, len);
    c->src[id] = host;
    c->src_len[id] = len;
    return LOOMHIP_OK;
}

int loomhip_ec_pin(loomhip_ec *c, const uint32_t *ids, size_t n) {
    if (!c || (n && !ids))
        return fail(LOOMHIP_ERR_ARG, "ec_pin: bad arguments");
    for (size_t i = 0; i < n; i++) {
        const size_t id = ids[i];
        if (id >= c->n_ids)
            return fail(LOOMHIP_ERR_ARG, "ec_pin: id %zu out of range", id);
        if (c->pin_of[id] != EC_NIL)
            continue;
        if (c->n_pinned == c->pin_slots)
            return fail(LOOMHIP_ERR_ARG, "ec_pin: all %zu pinned slots are taken", c->pin_slots);
        if (!c->src[id])
            return fail(LOOMHIP_ERR_ARG, "ec_pin: expert %zu has no backing block", id);
        const size_t s = c->capacity + c->n_pinned;
        if (int rc = fill_slot(c, s, id, false, nullptr))
            return rc;
        c->pin_of[id] = s;
        c->n_pinned++;
        c->stats.warmup_reads += 1;
        c->stats.warmup_bytes += c->src_len[id];
    }
    const hipError_t e = hipStreamSynchronize(g_ctx.copy);
    return e == hipSuccess ? LOOMHIP_OK : hip_fail(e, "ec_pin");
}

int loomhip_ec_get(loomhip_ec *c, size_t id, void *stream, void **dev_out) {
    if (!c || id >= c->n_ids || !dev_out)
        return fail(LOOMHIP_ERR_ARG, "ec_get: bad arguments (id %zu)", id);
    size_t s;
    if (int rc = ec_get(c, id, stream_of(stream), &s))
        return rc;
    *dev_out = slot_ptr(c, s);
    return LOOMHIP_OK;
}

int loomhip_ec_release(loomhip_ec *c, void *stream) {
    if (!c)
        return fail(LOOMHIP_ERR_ARG, "ec_release: null cache");
    return ec_release(c, stream_of(stream));
}

int loomhip_ec_prefetch(loomhip_ec *c, const uint32_t *ids, size_t n) {
    if (!c || (n && !ids))
        return fail(LOOMHIP_ERR_ARG, "ec_prefetch: bad arguments");
    for (size_t i = 0; i < n; i++) {
        const size_t id = ids[i];
        if (id >= c->n_ids)
            return fail(LOOMHIP_ERR_ARG, "ec_prefetch: id %zu out of range", id);
        if (c->pin_of[id] != EC_NIL || c->map[id] != EC_NIL || !c->src[id])
            continue;
        size_t evicted;
        const size_t s = lru_reserve(c, id, &evicted);
        if (s == EC_NIL)
            return fail(LOOMHIP_ERR_ARG, "ec_prefetch: no capacity");
        if (int rc = fill_slot(c, s, id, false, nullptr)) {
            lru_abort(c, id);
            return rc;
        }
        c->stats.warmup_reads += 1;
        c->stats.warmup_bytes += c->src_len[id];
    }
    return LOOMHIP_OK;
}

int loomhip_ec_get_stats(const loomhip_ec *c, loomhip_ec_stats *out) {
    if (!c || !out)
        return fail(LOOMHIP_ERR_ARG, "ec_stats: bad arguments");
    *out = c->stats;
    return LOOMHIP_OK;
}

int loomhip_ec_access_counts(const loomhip_ec *c, uint64_t *out, size_t n) {
    if (!c || !out || n > c->n_ids)
        return fail(LOOMHIP_ERR_ARG, "ec_access_counts: bad arguments");
    memcpy(out, c->access.data(), n * sizeof(uint64_t));
    return LOOMHIP_OK;
}

int loomhip_ec_clear(loomhip_ec *c) {
    if (!c)
        return fail(LOOMHIP_ERR_ARG, "ec_clear: null cache");
    for (size_t s = 0; s < c->capacity; s++) {
        if (c->slot[s].id != EC_NIL)
            c->map[c->slot[s].id] = EC_NIL;
        c->slot[s].id = EC_NIL;
    }
    c->head = c->tail = EC_NIL;
    c->free_top = 0;
    return LOOMHIP_OK;
}

int loomhip_moe_layer_cached(const loomhip_moe_layer_ec *L, loomhip_ec *ec, const float *normed,
                             size_t n_tok, float *out, uint32_t *ids_out, float *gates_out,
                             void *stream) {
    if (int rc = require_ready())
        return rc;
    if (!L || !ec || !normed || !out || !L->router || n_tok == 0)
        return fail(LOOMHIP_ERR_ARG, "moe_layer_cached: null argument");
    return moe_cached(*L, ec, normed, n_tok, out, ids_out, gates_out, stream_of(stream));
}

} // extern "C"
