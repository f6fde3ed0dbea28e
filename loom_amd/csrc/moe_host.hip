// moe_host.hip -- host orchestration of the MoE layer: route -> bucket ->
// quantize -> fused gate/up+SwiGLU -> quantize -> down -> combine, all
// stream-ordered with no host round trip (the one-submission shape of
// src/vulkan/backend.zig:455-551, generalised to n tokens with the grouped
// expert kernels).
#include "runtime.hpp"

namespace lh {

static Scratch g_moe;   // per-call workspace
static Scratch g_stage; // seam-call staging
static Scratch g_sh;    // the shared expert's workspace

// Fixed workspace of loomhip_moe_layer_dev_noalloc: a file-scope device
// array, one copy per GPU for the life of the process.  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in
// symbol): moe_noalloc_setup resolves each device's copy once, with that
// device current, and the entry point uses that address.
constexpr size_t MOE_NOALLOC_BYTES = LOOMHIP_MOE_NOALLOC_BYTES;
static __device__ __align__(256) char scratch[MOE_NOALLOC_BYTES];
constexpr int NOALLOC_MAX_DEVICES = 64;
static void *g_scratch_dev[NOALLOC_MAX_DEVICES];

int moe_noalloc_setup(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES)
        return fail(LOOMHIP_ERR_INIT, "moe noalloc: device %d out of range", device);
    if (g_scratch_dev[device])
        return LOOMHIP_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
        return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch_dev[device] = p;
    return LOOMHIP_OK;
}

void moe_release_scratch() {
    g_moe.release();
    g_stage.release();
    g_sh.release();
}

struct MoeRun {
    size_t dim, ffn, E, k;
    int gating, weights_norm;
    float weights_scale;
    const float *router, *router_bias, *sel_bias; // router null: logits given
    int gate_t, up_t, down_t;
    const void *gate, *up, *down;
    const float *norm_w = nullptr; // decode path: rmsnorm the input first (normed = residual x)
    float norm_eps = 0.0f;
    bool norm_exact = false;       // ... with the squares summed in the reference's order (one token)
    DenseFfn sh{}; // the shared expert (sh.gate null: none)
    const NextNorm *next = nullptr; // batched path: the next rmsnorm in the combine's launch
    bool *next_done = nullptr;      // ... set when it ran there
};

static size_t qbytes(size_t nvec, size_t cols) {
    return align16(nvec * cols) + align16(nvec * (cols / 32) * 4) + align16(nvec * (cols / 16) * 4);
}

static QAct qview(char *base, size_t nvec, size_t cols) {
    QAct q;
    q.q = (int8_t *)base;
    q.d = (float *)(base + align16(nvec * cols));
    q.s = (int32_t *)((char *)q.d + align16(nvec * (cols / 32) * 4));
    return q;
}

// ---- the shared expert: a dense SwiGLU FFN added after the routed sum ----------------
// out[t] = out[t] + down . swiglu(gate . x_t, up . x_t) (add; else out[t] =
// the FFN's output): the reference's
// denseFFN (llama.zig:952-958) of ffn_{gate,up,down}_shexp, then
// backend.add(acc, ffn_out) (deepseek.zig:1497-1502).  One plane each, device
// layout; the fused gate/up launch, the activations' quantization and the
// down matvec with its residual-add epilogue, all bit-identical to the CPU
// kernels.

int dense_ffn_check(const DenseFfn &f, size_t dim) {
    if (!f.gate || !f.up || !f.down || f.ffn == 0)
        return fail(LOOMHIP_ERR_ARG, "shared expert: missing tensor or width");
    if (f.gate_t != f.up_t || !dmmv_supported(f.gate_t, (int)dim) || !dmmv_supported(f.down_t, (int)f.ffn) ||
        f.ffn % 32 || (act_block(f.gate_t) == 256 && dim % 256) || (act_block(f.down_t) == 256 && f.ffn % 256))
        return fail(LOOMHIP_DECLINED, "shared expert: types %d/%d/%d at dim %zu / ffn %zu not served", f.gate_t,
                    f.up_t, f.down_t, dim, f.ffn);
    return LOOMHIP_OK;
}

int dense_ffn_add(const DenseFfn &f, const float *x, size_t n, size_t dim, float *out, hipStream_t st, bool add) {
    if (int rc = dense_ffn_check(f, dim))
        return rc;
    const size_t need = qbytes(n, dim) + align16(n * f.ffn * 4) + qbytes(n, f.ffn);
    if (int rc = g_sh.reserve(need))
        return rc;
    char *base = (char *)g_sh.ptr;
    const QAct qx = qview(base, n, dim);
    float *act = (float *)(base + qbytes(n, dim));
    const QAct qa = qview(base + qbytes(n, dim) + align16(n * f.ffn * 4), n, f.ffn);
    const int nt = pick_nt((int)n);
    int ng = 0;
    const DmmvGroup *groups = dense_groups((int)n, nt, &ng);
    if (!groups)
        return fail(LOOMHIP_ERR_HIP, "shared expert: group table");
    launch_quant_act(f.gate_t, x, (int)dim, (int)dim, (int)n, qx, st);
    DmmvParams p{};
    p.w = (const uint8_t *)f.gate;
    p.w2 = (const uint8_t *)f.up;
    p.rows = (int)f.ffn;
    p.cols = (int)dim;
    p.xq = qx.q;
    p.xd = qx.d;
    p.xs = qx.s;
    p.pair_src = g_ctx.iota;
    p.pair_dst = g_ctx.iota;
    p.groups = groups;
    p.n_groups = ng;
    p.out = act;
    p.out_stride = (int)f.ffn;
    p.rpw = dmmv_pick_rpw(f.gate_t, (int)dim, (int)f.ffn, ng, nt, true);
    if (!launch_dmmv(f.gate_t, nt, true, p, st))
        return fail(LOOMHIP_ERR_ARG, "shared expert: gate/up partials exceed LDS");
    launch_quant_act(f.down_t, act, (int)f.ffn, (int)f.ffn, (int)n, qa, st);
    DmmvParams d{};
    d.w = (const uint8_t *)f.down;
    d.rows = (int)dim;
    d.cols = (int)f.ffn;
    d.xq = qa.q;
    d.xd = qa.d;
    d.xs = qa.s;
    d.pair_src = g_ctx.iota;
    d.pair_dst = g_ctx.iota;
    d.groups = groups;
    d.n_groups = ng;
    d.out = out;
    d.out_stride = (int)dim;
    d.accumulate = add ? 1 : 0; // add: out = out + value
    d.rpw = dmmv_pick_rpw(f.down_t, (int)f.ffn, (int)dim, ng, nt, false);
    if (!launch_dmmv(f.down_t, nt, false, d, st))
        return fail(LOOMHIP_ERR_ARG, "shared expert: down partials exceed LDS");
    return LOOMHIP_OK;
}

static DenseFfn shexp_of(const loomhip_moe_layer *L) {
    return DenseFfn{L->shexp_gate_t, L->shexp_up_t, L->shexp_down_t, L->shexp_gate, L->shexp_up, L->shexp_down,
                    L->shexp_ffn};
}

static int moe_check(const MoeRun &m, size_t n) {
    if (!gate_supported((int)n, (int)m.E, (int)m.k))
        return fail(LOOMHIP_DECLINED, "moe: %zu tokens / %zu experts / top-%zu not served "
                    "(1..256 tokens, <= 256 experts, top-k <= 16)", n, m.E, m.k);
    if (m.gate_t != m.up_t)
        return fail(LOOMHIP_DECLINED, "moe: gate/up types differ (%d, %d)", m.gate_t, m.up_t);
    if (!dmmv_supported(m.gate_t, (int)m.dim) || !dmmv_supported(m.down_t, (int)m.ffn))
        return fail(LOOMHIP_DECLINED, "moe: shapes dim %zu / ffn %zu not served for types %d/%d",
                    m.dim, m.ffn, m.gate_t, m.down_t);
    if (m.dim % 32 || m.ffn % 32)
        return fail(LOOMHIP_DECLINED, "moe: dims must be multiples of 32");
    if (m.sh.gate)
        return dense_ffn_check(m.sh, m.dim);
    return LOOMHIP_OK;
}

static int moe_nt(size_t n, size_t k, size_t E) {
    if (n == 1)
        return 1;
    const size_t per = (n * k + E - 1) / E;
    return per >= 4 ? 8 : per >= 2 ? 4 : 2;
}

constexpr size_t DECODE_MAX_TOK = 4; // decode path up to this many tokens

// normed/logits/out are device pointers; logits may be null when m.router is set.
//
// Decode path (n <= DECODE_MAX_TOK), three launches, no bucketing:
//   gate     router GEMV + quantize x
//   gate/up  one work group per (token, slot, row tile): routes its token,
//            then fused gate/up + SwiGLU of the slot's expert
//   down     one work group per (token, row tile): quantizes the token's k
//            activations in LDS, down for every slot, gated combine
// Batched path, five launches, experts grouped so each weight row is read
// once per group of tokens:
//   gate     router GEMV + route + bucket + quantize x (last-arrival chain)
//   gate/up  grouped fused gate/up + SwiGLU
//   quant    int8 quantization of the activations
//   down     grouped down
//   combine  gated combine per token
// ws/ws_cap: a caller-held workspace used instead of the grow-only one (the
// no-allocation entry point); a call that needs more fails before launching.
static int moe_run(const MoeRun &m, const float *normed, const float *logits_in, size_t n,
                   int combine, float *out, uint32_t *ids_out, float *gates_out, hipStream_t st,
                   char *ws = nullptr, size_t ws_cap = 0) {
    if (int rc = moe_check(m, n))
        return rc;
    if (combine < LOOMHIP_COMBINE_SELECTION || combine > LOOMHIP_COMBINE_SELECTION_ADD)
        return fail(LOOMHIP_ERR_ARG, "moe: unknown combine mode %d", combine);
    if (m.sh.gate && (combine == LOOMHIP_COMBINE_SELECTION_ADD || m.norm_w))
        return fail(LOOMHIP_DECLINED, "moe: a shared expert is served with the SELECTION and EXPERT_ASC combines "
                    "on a normalised input");
    const size_t P = n * m.k;
    const bool decode = n <= DECODE_MAX_TOK && decode_supported(m.gate_t, m.down_t, (int)m.ffn);
    // matrix cores for the expert matmuls from MMQ_MIN_TOK tokens on, groups
    // of up to 16 tokens per expert
    const bool mq = !decode && use_mmq(m.gate_t, (int)m.dim, (int)n, 16, true) &&
                    use_mmq(m.down_t, (int)m.ffn, (int)n, 16, false);
    const int nt = mq ? 16 : moe_nt(n, m.k, m.E);
    const int maxg = moe_max_groups((int)n, (int)m.k, (int)m.E, nt);
    // workspace layout
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += align16(bytes);
        return o;
    };
    const size_t o_qx = take(qbytes(n, m.dim));
    const size_t o_log = take(n * m.E * 4);
    const size_t o_ids = take(P * 4), o_gates = take(P * 4);
    const size_t o_ptok = take(P * 4), o_pof = take(P * 4), o_iota = take(P * 4);
    const size_t o_groups = take(maxg * sizeof(DmmvGroup)), o_ng = take(16);
    const size_t o_gsrc = take(mq ? (size_t)maxg * nt * 4 : 0);
    const size_t o_act = take(P * m.ffn * 4);
    const size_t o_qa = take(qbytes(P, m.ffn));
    const size_t o_y = take(decode ? 0 : P * m.dim * 4);
    char *base;
    if (ws) {
        if (off > ws_cap)
            return fail(LOOMHIP_ERR_ARG, "moe_layer_dev_noalloc: %zu tokens need %zu B of workspace, the fixed "
                        "scratch holds %zu B", n, off, ws_cap);
        base = ws;
    } else {
        if (int rc = g_moe.reserve(off))
            return rc;
        base = (char *)g_moe.ptr;
    }
    const QAct qx = qview(base + o_qx, n, m.dim);
    uint32_t *ids = ids_out ? ids_out : (uint32_t *)(base + o_ids);
    float *gates = gates_out ? gates_out : (float *)(base + o_gates);
    float *logits = (float *)(base + o_log);
    float *act = (float *)(base + o_act);

    GateParams gp{};
    gp.router = m.router;
    gp.router_bias = m.router_bias;
    gp.sel_bias = m.sel_bias;
    gp.x = normed;
    gp.logits_in = m.router ? nullptr : logits_in;
    gp.n = (int)n;
    gp.dim = (int)m.dim;
    gp.n_expert = (int)m.E;
    gp.k = (int)m.k;
    gp.gating = m.gating;
    gp.weights_norm = m.weights_norm;
    gp.weights_scale = m.weights_scale;
    gp.logits = logits;
    gp.ids = ids;
    gp.gates = gates;
    gp.qt = m.gate_t;
    gp.qx = qx;
    gp.nt = nt;
    gp.sync = g_ctx.sync;

    if (decode) {
        DecodeParams dp{};
        dp.logits = m.router ? logits : logits_in;
        dp.sel_bias = m.sel_bias;
        dp.n_expert = (int)m.E;
        dp.k = (int)m.k;
        dp.gating = m.gating;
        dp.weights_norm = m.weights_norm;
        dp.weights_scale = m.weights_scale;
        dp.ids = ids;
        dp.gates = gates;
        dp.gate = (const uint8_t *)m.gate;
        dp.up = (const uint8_t *)m.up;
        dp.down = (const uint8_t *)m.down;
        dp.gu_plane = plane_bytes(m.gate_t, m.ffn, m.dim);
        dp.dn_plane = plane_bytes(m.down_t, m.dim, m.ffn);
        dp.dim = (int)m.dim;
        dp.ffn = (int)m.ffn;
        dp.down_t = m.down_t;
        dp.xq = qx.q;
        dp.xd = qx.d;
        dp.xs = qx.s;
        dp.act = act;
        dp.out = out;
        dp.mode = combine;
        dp.rpw_gu = dmmv_pick_rpw(m.gate_t, (int)m.dim, (int)m.ffn, (int)P, 1, true);
        // down: 4-row tiles unless the token count alone fills the chip
        int rpw = 2;
        while (rpw < 8 && ((int)m.dim / (4 * rpw)) * (int)n >= 1024)
            rpw *= 2;
        while (rpw > 1 && decode_down_lds(m.down_t, (int)m.ffn, (int)m.k, rpw) > 48 * 1024)
            rpw /= 2;
        dp.rpw_dn = rpw;
        if (decode_down_lds(m.down_t, (int)m.ffn, (int)m.k, rpw) > 64 * 1024)
            return fail(LOOMHIP_DECLINED, "moe: ffn %zu x top-%zu exceeds the decode LDS budget",
                        m.ffn, m.k);
        gp.chain = 0;
        gp.norm_w = m.norm_w;
        gp.norm_eps = m.norm_eps;
        gp.norm_exact = m.norm_w && m.norm_exact;
        if (gp.norm_exact && !router_exact_supported((int)n, (int)m.dim))
            return fail(LOOMHIP_ERR_ARG, "moe: the exact fused norm takes one token of dim <= 7936");
        launch_router_small(gp, st);
        if (!launch_moe_decode(m.gate_t, m.down_t, dp, (int)n, st, LOOMHIP_KT_GATE_UP, LOOMHIP_KT_DOWN))
            return fail(LOOMHIP_ERR_ARG, "moe: decode kernels declined the shape");
        return m.sh.gate ? dense_ffn_add(m.sh, normed, n, m.dim, out, st, true) : LOOMHIP_OK;
    }

    if (m.norm_w)
        return fail(LOOMHIP_ERR_ARG, "moe: a fused input norm is served on the decode path only");
    const QAct qa = qview(base + o_qa, P, m.ffn);
    MoeBuckets b;
    b.pair_tok = (int *)(base + o_ptok);
    b.pair_of = (int *)(base + o_pof);
    b.iota = (int *)(base + o_iota);
    b.groups = (DmmvGroup *)(base + o_groups);
    b.n_groups = (int *)(base + o_ng);
    b.group_src = mq ? (int *)(base + o_gsrc) : nullptr;
    float *y = (float *)(base + o_y);
    gp.b = b;
    gp.chain = 1;
    launch_gate(gp, st);

    const int exp_groups = (int)(P < (size_t)maxg ? P : (size_t)maxg);
    DmmvParams gu{};
    gu.w = (const uint8_t *)m.gate;
    gu.w2 = (const uint8_t *)m.up;
    gu.plane_bytes = plane_bytes(m.gate_t, m.ffn, m.dim);
    gu.rows = (int)m.ffn;
    gu.cols = (int)m.dim;
    gu.xq = qx.q;
    gu.xd = qx.d;
    gu.xs = qx.s;
    gu.pair_src = b.pair_tok;
    gu.pair_dst = b.iota;
    gu.groups = b.groups;
    gu.n_groups_dev = b.n_groups;
    gu.n_groups = maxg;
    gu.out = act;
    gu.out_stride = (int)m.ffn;
    gu.group_src = b.group_src;
    gu.group_stride = nt;
    gu.pos_ident = 1;
    gu.rpw = mq ? 0 : dmmv_pick_rpw(m.gate_t, (int)m.dim, (int)m.ffn, exp_groups, nt, true);
    int ph = prof_begin(LOOMHIP_KT_GATE_UP, st);
    bool launched = mq ? launch_mmq(m.gate_t, nt, true, gu, st) : launch_dmmv(m.gate_t, nt, true, gu, st);
    prof_end(ph, st);
    if (!launched)
        return fail(LOOMHIP_ERR_ARG, "moe: gate/up partials exceed LDS");

    launch_quant_act(m.down_t, act, (int)m.ffn, (int)m.ffn, (int)P, qa, st);

    DmmvParams dn{};
    dn.w = (const uint8_t *)m.down;
    dn.w2 = nullptr;
    dn.plane_bytes = plane_bytes(m.down_t, m.dim, m.ffn);
    dn.rows = (int)m.dim;
    dn.cols = (int)m.ffn;
    dn.xq = qa.q;
    dn.xd = qa.d;
    dn.xs = qa.s;
    dn.pair_src = b.iota;
    dn.pair_dst = b.iota;
    dn.groups = b.groups;
    dn.n_groups_dev = b.n_groups;
    dn.n_groups = maxg;
    dn.out = y;
    dn.out_stride = (int)m.dim;
    dn.rpw = mq ? 0 : dmmv_pick_rpw(m.down_t, (int)m.ffn, (int)m.dim, exp_groups, nt, false);
    ph = prof_begin(LOOMHIP_KT_DOWN, st);
    launched = mq ? launch_mmq(m.down_t, nt, false, dn, st) : launch_dmmv(m.down_t, nt, false, dn, st);
    prof_end(ph, st);
    if (!launched)
        return fail(LOOMHIP_ERR_ARG, "moe: down partials exceed LDS");

    if (m.next && combine == LOOMHIP_COMBINE_EXPERT_ASC && !m.sh.gate &&
        launch_combine_norm(y, gates, ids, b.pair_of, (int)n, (int)m.k, (int)m.dim, out, *m.next, st)) {
        if (m.next_done)
            *m.next_done = true;
        return LOOMHIP_OK;
    }
    launch_combine(y, gates, ids, b.pair_of, (int)n, (int)m.k, (int)m.dim, combine, out, st);
    return m.sh.gate ? dense_ffn_add(m.sh, normed, n, m.dim, out, st, true) : LOOMHIP_OK;
}

// Everything moe_run would decline or refuse for this layer at n tokens,
// checked before the token frame launches anything (the frame's layers are
// resolved up front, src/vulkan/backend.zig:462-489).
int moe_layer_check(const loomhip_moe_layer *L, size_t n, bool shexp_ok) {
    if (!L->router || !L->gate || !L->up || !L->down)
        return fail(LOOMHIP_ERR_ARG, "moe: layer without router or expert tensors");
    MoeRun m{L->dim, L->ffn, L->n_expert, L->n_used, L->gating, L->weights_norm, L->weights_scale,
             L->router, L->router_bias, L->sel_bias, L->gate_t, L->up_t, L->down_t, L->gate,
             L->up, L->down};
    m.sh = shexp_of(L);
    if (int rc = moe_check(m, n))
        return rc;
    if (m.sh.gate && !shexp_ok) // the frame adds its MoE output to the residual, acc = routed + shared is not formed
        return fail(LOOMHIP_DECLINED, "token_frame: a shared expert is not served inside the frame");
    if (n <= DECODE_MAX_TOK && decode_supported(m.gate_t, m.down_t, (int)m.ffn) &&
        decode_down_lds(m.down_t, (int)m.ffn, (int)m.k, 1) > 64 * 1024)
        return fail(LOOMHIP_DECLINED, "moe: ffn %zu x top-%zu exceeds the decode LDS budget", m.ffn, m.k);
    return LOOMHIP_OK;
}

int moe_frame_check(const loomhip_moe_layer *L, size_t n) { return moe_layer_check(L, n, false); }

int moe_layer_fused_norm(const loomhip_moe_layer *L, const float *x, const float *norm_w, float eps, size_t n_tok,
                         int combine, float *out, uint32_t *ids_out, bool exact, hipStream_t st) {
    MoeRun m{L->dim, L->ffn, L->n_expert, L->n_used, L->gating, L->weights_norm, L->weights_scale,
             L->router, L->router_bias, L->sel_bias, L->gate_t, L->up_t, L->down_t, L->gate,
             L->up, L->down};
    m.norm_w = norm_w;
    m.norm_eps = eps;
    m.norm_exact = exact;
    return moe_run(m, x, nullptr, n_tok, combine, out, ids_out, nullptr, st);
}

int moe_layer_next_norm(const loomhip_moe_layer *L, const float *normed, size_t n_tok, int combine, float *out,
                        uint32_t *ids_out, const NextNorm *next, bool *next_done, hipStream_t st) {
    MoeRun m{L->dim, L->ffn, L->n_expert, L->n_used, L->gating, L->weights_norm, L->weights_scale,
             L->router, L->router_bias, L->sel_bias, L->gate_t, L->up_t, L->down_t, L->gate,
             L->up, L->down};
    m.sh = shexp_of(L);
    m.next = next;
    m.next_done = next_done;
    return moe_run(m, normed, nullptr, n_tok, combine, out, ids_out, nullptr, st);
}

bool moe_decode_fusable(const loomhip_moe_layer *L, size_t n_tok, bool exact) {
    return n_tok <= DECODE_MAX_TOK && decode_supported(L->gate_t, L->down_t, (int)L->ffn) && L->router &&
           L->dim <= 8192 && L->dim % 32 == 0 && (!exact || router_exact_supported((int)n_tok, (int)L->dim));
}

} // namespace lh

using namespace lh;

extern "C" {

int loomhip_moe_layer_dev(const loomhip_moe_layer *L, const float *normed, size_t n_tok,
                          int combine, float *out, uint32_t *ids_out, float *gates_out,
                          void *stream) {
    if (int rc = require_ready())
        return rc;
    if (!L || !normed || !out || !L->router)
        return fail(LOOMHIP_ERR_ARG, "moe_layer_dev: null argument");
    MoeRun m{L->dim, L->ffn, L->n_expert, L->n_used, L->gating, L->weights_norm, L->weights_scale,
             L->router, L->router_bias, L->sel_bias, L->gate_t, L->up_t, L->down_t, L->gate,
             L->up, L->down};
    m.sh = shexp_of(L);
    return moe_run(m, normed, nullptr, n_tok, combine, out, ids_out, gates_out, stream_of(stream));
}

int loomhip_moe_layer_dev_noalloc(const loomhip_moe_layer *L, const float *normed, size_t n_tok,
                                  int combine, float *out, uint32_t *ids_out, float *gates_out,
                                  void *stream) {
    if (int rc = require_ready())
        return rc;
    if (!L || !normed || !out || !L->router)
        return fail(LOOMHIP_ERR_ARG, "moe_layer_dev_noalloc: null argument");
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES || !g_scratch_dev[dev])
        return fail(LOOMHIP_ERR_INIT, "moe_layer_dev_noalloc: no fixed scratch resolved for device %d "
                    "(loomhip_init sets it up)", dev);
    if (L->shexp_gate)
        return fail(LOOMHIP_ERR_ARG, "moe_layer_dev_noalloc: the shared expert's workspace is allocated; "
                    "use loomhip_moe_layer_dev");
    MoeRun m{L->dim, L->ffn, L->n_expert, L->n_used, L->gating, L->weights_norm, L->weights_scale,
             L->router, L->router_bias, L->sel_bias, L->gate_t, L->up_t, L->down_t, L->gate,
             L->up, L->down};
    return moe_run(m, normed, nullptr, n_tok, combine, out, ids_out, gates_out, stream_of(stream),
                   (char *)g_scratch_dev[dev], MOE_NOALLOC_BYTES);
}

int loomhip_moe_route(const float *logits, const float *bias, size_t n_expert, size_t n_used,
                      int gating, int weights_norm, float weights_scale, uint32_t *ids_out,
                      float *gates_out) {
    if (int rc = require_ready())
        return rc;
    if (!gate_supported(1, (int)n_expert, (int)n_used))
        return fail(LOOMHIP_DECLINED, "moe_route: %zu experts / top-%zu not served", n_expert, n_used);
    const size_t need = 2 * n_expert * 4 + 2 * 64;
    if (int rc = g_stage.reserve(need))
        return rc;
    char *base = (char *)g_stage.ptr;
    float *dl = (float *)base, *db = (float *)(base + n_expert * 4);
    uint32_t *di = (uint32_t *)(base + 2 * n_expert * 4);
    float *dg = (float *)(base + 2 * n_expert * 4 + 64);
    hipStream_t st = g_ctx.compute;
    hipError_t e = hipMemcpyAsync(dl, logits, n_expert * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && bias)
        e = hipMemcpyAsync(db, bias, n_expert * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_route staging");
    GateParams gp{};
    gp.sel_bias = bias ? db : nullptr;
    gp.logits_in = dl;
    gp.n = 1;
    gp.dim = 0;
    gp.n_expert = (int)n_expert;
    gp.k = (int)n_used;
    gp.gating = gating;
    gp.weights_norm = weights_norm;
    gp.weights_scale = weights_scale;
    gp.ids = di;
    gp.gates = dg;
    gp.qt = 0;
    gp.nt = 1;
    gp.sync = g_ctx.sync;
    gp.chain = 1;
    launch_gate(gp, st);
    e = hipMemcpyAsync(ids_out, di, n_used * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(gates_out, dg, n_used * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_route readback");
    return LOOMHIP_OK;
}

int loomhip_moe_ffn_routed(const float *normed, size_t n_tok, size_t dim, const float *logits,
                           const float *sel_bias, size_t n_expert, size_t n_used, int gating,
                           int weights_norm, float weights_scale, int gate_t, const void *gate_w,
                           int up_t, const void *up_w, int down_t, const void *down_w,
                           int shexp_gate_t, const void *shexp_gate_w, int shexp_up_t,
                           const void *shexp_up_w, int shexp_down_t, const void *shexp_down_w,
                           size_t ffn, size_t shexp_ffn, int combine, float *out) {
    if (int rc = require_ready())
        return rc;
    if (!normed || !logits || !gate_w || !up_w || !down_w || !out)
        return fail(LOOMHIP_ERR_ARG, "moe_ffn_routed: null argument");
    if (shexp_gate_w && (!shexp_up_w || !shexp_down_w || shexp_ffn == 0))
        return fail(LOOMHIP_ERR_ARG, "moe_ffn_routed: incomplete shared expert");
    MoeRun m{dim, ffn, n_expert, n_used, gating, weights_norm, weights_scale, nullptr, nullptr,
             nullptr, gate_t, up_t, down_t, nullptr, nullptr, nullptr};
    // the shared expert's shapes and types, checked with the rest (its
    // pointers stand in until the upload below resolves them)
    if (shexp_gate_w)
        m.sh = DenseFfn{shexp_gate_t, shexp_up_t, shexp_down_t, shexp_gate_w, shexp_up_w, shexp_down_w, shexp_ffn};
    // Decline before touching the device (src/vulkan/backend.zig:462-489).
    if (int rc = moe_check(m, n_tok))
        return rc;
    if (m.sh.gate && combine == LOOMHIP_COMBINE_SELECTION_ADD)
        return fail(LOOMHIP_DECLINED, "moe_ffn_routed: a shared expert is served with the SELECTION and "
                    "EXPERT_ASC combines");
    void *dg, *du, *dd;
    int rc;
    if ((rc = upload_weights(gate_t, gate_w, ffn, dim, n_expert, &dg)) ||
        (rc = upload_weights(up_t, up_w, ffn, dim, n_expert, &du)) ||
        (rc = upload_weights(down_t, down_w, dim, ffn, n_expert, &dd)))
        return rc;
    m.gate = dg;
    m.up = du;
    m.down = dd;
    if (m.sh.gate) {
        void *sg, *su, *sd;
        if ((rc = upload_weights(shexp_gate_t, shexp_gate_w, shexp_ffn, dim, 1, &sg)) ||
            (rc = upload_weights(shexp_up_t, shexp_up_w, shexp_ffn, dim, 1, &su)) ||
            (rc = upload_weights(shexp_down_t, shexp_down_w, dim, shexp_ffn, 1, &sd)))
            return rc;
        m.sh.gate = sg;
        m.sh.up = su;
        m.sh.down = sd;
    }
    const size_t nb = align16(n_tok * dim * 4), lb = align16(n_tok * n_expert * 4);
    if ((rc = g_stage.reserve(2 * nb + 2 * lb)))
        return rc;
    char *base = (char *)g_stage.ptr;
    float *dn = (float *)base, *dout = (float *)(base + nb), *dl = (float *)(base + 2 * nb);
    float *dsb = (float *)(base + 2 * nb + lb);
    hipStream_t st = g_ctx.compute;
    hipError_t e = hipMemcpyAsync(dn, normed, n_tok * dim * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dl, logits, n_tok * n_expert * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && sel_bias)
        e = hipMemcpyAsync(dsb, sel_bias, n_expert * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && combine != LOOMHIP_COMBINE_SELECTION)
        e = hipMemcpyAsync(dout, out, n_tok * dim * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_ffn_routed staging");
    m.sel_bias = sel_bias ? dsb : nullptr;
    if ((rc = moe_run(m, dn, dl, n_tok, combine, dout, nullptr, nullptr, st)))
        return rc;
    e = hipMemcpyAsync(out, dout, n_tok * dim * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return hip_fail(e, "moe_ffn_routed readback");
    return LOOMHIP_OK;
}

} // extern "C"
