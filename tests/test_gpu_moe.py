"""GPU parity of routing and the whole MoE layer against the CPU oracle
(llama.moeLayer/moeRun at one token, moeBatchUnion for batches).  Runs on the
MI355X box only."""
import numpy as np
import pytest

import npref

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, F32 = 12, 14, 0


@pytest.fixture(scope="module")
def be(oracle):
    import loom_amd
    from loom_amd import backend

    loom_amd.init(0)
    backend.clearWeightCache()
    yield backend
    backend.clearWeightCache()


@pytest.fixture(autouse=True)
def fresh_weight_cache(be):
    # The device weight cache is keyed by host address; numpy recycles
    # addresses between tests, so stale weights would be served (the
    # reference's tests clear their cache for the same reason,
    # src/vulkan/backend.zig:159-172).
    be.clearWeightCache()
    yield


def _maxrel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def _same_bits(got, want, what=""):
    """Bit-identical layer outputs (north_star asks for 2e-3; every matvec is
    exact and each combine runs in the reference's order, so the device
    gives the CPU path's own bits)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    print(f"{what} max-rel {_maxrel(got, want):.2e}", flush=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (what, _maxrel(got, want))


@pytest.mark.parametrize("gating,norm,scale,bias", [
    ("softmax", True, 1.0, False), ("sigmoid", True, 1.0, True), ("sigmoid", True, 1.0, False),
    ("softmax", False, 2.5, False), ("sigmoid", False, 1.0, True),
])
def test_route_matches_oracle(be, oracle, gating, norm, scale, bias):
    # src/vulkan/backend.zig:1242-1295: identical ids, gates within 1e-5
    for n_expert, n_used, seed in ((64, 6, 1), (128, 8, 2), (256, 8, 3), (8, 2, 4)):
        rng = np.random.default_rng(seed)
        logits = ((rng.random(n_expert) - 0.5) * 4).astype(np.float32)
        logits[5] = logits[7]  # a deliberate tie: lowest index must win
        b = ((rng.random(n_expert) - 0.5) * 0.5).astype(np.float32) if bias else None
        ids = np.empty(n_used, np.uint32)
        gates = np.empty(n_used, np.float32)
        assert be.moeRoute(logits, b, ids, gates, gating == "sigmoid", norm, scale)
        g = oracle.GATING_SIGMOID if gating == "sigmoid" else oracle.GATING_SOFTMAX
        wid, wg = oracle.route(logits, n_used, g, norm, scale, b)
        assert np.array_equal(ids, wid)
        assert np.all(np.abs(gates - wg) <= 1e-6)


def test_route_kats_on_device(be, oracle):
    # src/gguf/moe.zig:210-223
    ids = np.empty(2, np.uint32)
    gates = np.empty(2, np.float32)
    assert be.moeRoute(np.array([0, 1, 2, 3], np.float32), np.array([10, 0, 0, 0], np.float32),
                       ids, gates, True, False, 1.0)
    assert list(ids) == [0, 3]
    assert abs(gates[0] - 0.5) < 1e-6 and abs(gates[1] - 1 / (1 + np.exp(-3.0))) < 1e-6
    # src/gguf/moe.zig:260-267
    assert be.moeRoute(np.array([1, 2, 3, 4], np.float32), None, ids, gates, False, True, 2.5)
    assert abs(gates.sum() - 2.5) < 1e-5


def make_layer(oracle, dim, ffn, n_expert, n_used, seed, gate_t=Q4_K, down_t=Q6_K,
               router_bias=False, recipe=False):
    """recipe: the expert planes by config 3's input recipe (N(0, 0.02)
    through the oracle's GGUF quantizers); otherwise random blocks with
    pinned scales (every quant level exercised)."""
    rng = np.random.default_rng(seed)
    if recipe:
        import recipes

        gate = recipes.planes(gate_t, ffn, dim, n_expert, seed * 3 + 1)
        up = recipes.planes(gate_t, ffn, dim, n_expert, seed * 3 + 2)
        down = recipes.planes(down_t, dim, ffn, n_expert, seed * 3 + 3)
    else:
        gate = npref.pinned_scale_blocks(gate_t, ffn, dim, rng, planes=n_expert)
        up = npref.pinned_scale_blocks(gate_t, ffn, dim, rng, planes=n_expert)
        down = npref.pinned_scale_blocks(down_t, dim, ffn, rng, planes=n_expert)
    router = oracle.normal(n_expert * dim, seed + 1, 0.0, 1.0 / np.sqrt(dim)).reshape(n_expert, dim)
    rb = None
    if router_bias:  # Zipf(1.1) popularity as a logit bias (config 3)
        ranks = rng.permutation(n_expert) + 1
        rb = (np.log(1.0 / ranks ** 1.1) - np.log(1.0 / ranks ** 1.1).mean()).astype(np.float32)
    return oracle.MoeWeights(dim, ffn, n_expert, n_used, router, gate, up, down, gate_t, gate_t,
                             down_t, router_bias=rb)


@pytest.mark.parametrize("dim,ffn,E,k", [(512, 256, 16, 4), (2048, 768, 128, 8)])
def test_moe_ffn_routed_single_token(be, oracle, dim, ffn, E, k):
    from loom_amd.backend import RoutedCfg, WeightRef

    w = make_layer(oracle, dim, ffn, E, k, seed=dim + E, recipe=dim == 2048)
    normed = oracle.normal(dim, 99, 0.0, 1.0)
    logits = oracle.matvec(F32, w.router.view(np.uint8).ravel(), normed, E, dim)
    out = np.empty(dim, np.float32)
    be.takeCmdBufCount()
    ok = be.moeFfnBlockRouted(normed, logits, None, WeightRef(w.gate_t, w.gate),
                              WeightRef(w.up_t, w.up), WeightRef(w.down_t, w.down), None, ffn, 0,
                              RoutedCfg(E, k, False, True, 1.0), out)
    assert ok
    assert be.takeCmdBufCount() >= 3  # gate, gate/up, down ran on the device
    want, ids, gates = oracle.moe_layer_token(w, normed)
    _same_bits(out, want, f"dim {dim}")


def _dev_layer(be, w):
    import torch

    def dev(t, raw, rows, cols):
        return be.repack_dev(t, torch.from_numpy(raw).cuda(), rows, cols, w.n_expert)

    router = torch.from_numpy(w.router).cuda()
    rb = None if w.router_bias is None else torch.from_numpy(w.router_bias).cuda()
    return be.MoeLayer(w.dim, w.ffn, w.n_expert, w.n_used, router,
                       dev(w.gate_t, w.gate, w.ffn, w.dim), dev(w.up_t, w.up, w.ffn, w.dim),
                       dev(w.down_t, w.down, w.dim, w.ffn), w.gate_t, w.up_t, w.down_t,
                       router_bias=rb)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 32, 128])
def test_moe_layer_dev_matches_oracle(be, oracle, n):
    """Config 3 by its recipe: hidden 2048, 128 experts top-8, ffn 768, Q4_K
    gate/up and Q6_K down from N(0, 0.02) weights, f32 router with a
    Zipf(1.1) logit bias."""
    import torch

    w = make_layer(oracle, 2048, 768, 128, 8, seed=3, router_bias=True, recipe=True)
    layer = _dev_layer(be, w)
    xs = np.stack([oracle.normal(2048, 500 + i, 0.0, 1.0) for i in range(n)])
    normed = torch.from_numpy(xs).cuda()
    ids = torch.empty((n, 8), dtype=torch.int32, device="cuda")
    gates = torch.empty((n, 8), dtype=torch.float32, device="cuda")
    if n == 1:
        out = torch.empty((1, 2048), dtype=torch.float32, device="cuda")
        layer(normed, out, combine=be.COMBINE_SELECTION, ids=ids, gates=gates)
        want, wid, wg = oracle.moe_layer_token(w, xs[0])
        want = want[None]
        wid, wg = wid[None], wg[None]
    else:
        resid = np.stack([oracle.normal(2048, 900 + i, 0.0, 1.0) for i in range(n)])
        out = torch.from_numpy(resid.copy()).cuda()
        layer(normed, out, combine=be.COMBINE_EXPERT_ASC, ids=ids, gates=gates)
        want, wid, wg = oracle.moe_batch_union(w, xs, resid)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy().astype(np.uint32), wid)
    assert np.all(np.abs(gates.cpu().numpy() - wg) <= 1e-6)
    _same_bits(out.cpu().numpy(), want, f"n={n}")


@pytest.mark.parametrize("n", [1, 2, 6])
def test_moe_layer_dev_wide_hidden(be, oracle, n):
    """Hidden 7168 (28 super-blocks per row: a partial last column chunk) and
    expert ffn 2048, the DeepSeek-V3-class block's shapes, with 16 experts."""
    import torch

    w = make_layer(oracle, 7168, 2048, 16, 4, seed=11, gate_t=Q4_K, down_t=Q4_K)
    layer = _dev_layer(be, w)
    xs = np.stack([oracle.normal(7168, 700 + i, 0.0, 1.0) for i in range(n)])
    normed = torch.from_numpy(xs).cuda()
    ids = torch.empty((n, 4), dtype=torch.int32, device="cuda")
    gates = torch.empty((n, 4), dtype=torch.float32, device="cuda")
    resid = np.stack([oracle.normal(7168, 800 + i, 0.0, 1.0) for i in range(n)])
    out = torch.from_numpy(resid.copy()).cuda()
    layer(normed, out, combine=be.COMBINE_EXPERT_ASC, ids=ids, gates=gates)
    want, wid, wg = oracle.moe_batch_union(w, xs, resid)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy().astype(np.uint32), wid)
    assert np.all(np.abs(gates.cpu().numpy() - wg) <= 1e-6)
    _same_bits(out.cpu().numpy(), want, f"n={n}")


@pytest.mark.parametrize("n", [5, 7, 9, 16, 17, 31, 33, 47, 64, 65, 100, 127, 128, 129, 200, 256])
def test_moe_gate_handoff_at_many_lane_counts(be, oracle, n):
    """The batched gate kernel hands its per-chunk results from work group
    to work group inside the launch (agent-scope stores, a completion
    counter whose last arrival reads them back).  Every lane count from the
    batched path's smallest to the largest served, partial last chunks
    included, three launches each with fresh inputs: ids and outputs
    bit-identical to moeBatchUnion every time."""
    import torch

    dim, ffn, E, k = 512, 256, 32, 4
    w = make_layer(oracle, dim, ffn, E, k, seed=91, router_bias=True)
    layer = _dev_layer(be, w)
    for rep in range(3):
        xs = np.stack([oracle.normal(dim, 10_000 * rep + n * 7 + i, 0.0, 1.0) for i in range(n)])
        resid = np.zeros((n, dim), np.float32)
        out = torch.zeros((n, dim), dtype=torch.float32, device="cuda")
        ids = torch.empty((n, k), dtype=torch.int32, device="cuda")
        gates = torch.empty((n, k), dtype=torch.float32, device="cuda")
        layer(torch.from_numpy(xs).cuda(), out, combine=be.COMBINE_EXPERT_ASC, ids=ids, gates=gates)
        want, wid, wg = oracle.moe_batch_union(w, xs, resid)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy().astype(np.uint32), wid), (n, rep)
        assert np.all(np.abs(gates.cpu().numpy() - wg) <= 1e-6), (n, rep)
        _same_bits(out.cpu().numpy(), want, f"n={n} launch {rep}")


Q8_0, Q4_0 = 8, 2

# (gating, weights_norm, weights_scale, selection bias): the routing variants
# of moe.zig:106-158 (softmax, sigmoid with DeepSeek-V3's selection bias,
# softmax over the selected logits) through the whole layer
_GATINGS = [(1, True, 1.0, False), (2, True, 2.5, True), (3, False, 1.0, False),
            (1, False, 1.5, True)]


@pytest.mark.parametrize("down_t,ffn", [(Q8_0, 512), (Q4_0, 256), (Q8_0, 288), (Q6_K, 256)])
@pytest.mark.parametrize("gi", range(len(_GATINGS)))
@pytest.mark.parametrize("n", [1, 3, 8])
def test_moe_layer_dev_gatings_and_down_types(be, oracle, down_t, ffn, gi, n):
    """Every gating mode with the 32-block down types and the K-quant one,
    on the decode path (n <= 4, ffn a multiple of 256) and the batched path
    (n = 8, or an ffn that is not a multiple of 256)."""
    import torch

    gating, norm, scale, has_bias = _GATINGS[gi]
    dim, E, k = 512, 32, 4
    w = make_layer(oracle, dim, ffn, E, k, seed=40 + gi, gate_t=Q8_0 if down_t == Q6_K else Q4_K,
                   down_t=down_t)
    rng = np.random.default_rng(77 + gi)
    w.gating, w.weights_norm, w.weights_scale = gating, norm, scale
    if has_bias:
        w.sel_bias = ((rng.random(E) - 0.5) * 0.5).astype(np.float32)
    layer = _dev_layer(be, w)
    layer = be.MoeLayer(w.dim, w.ffn, E, k, *layer.keep[:4], w.gate_t, w.up_t, w.down_t,
                        sel_bias=None if w.sel_bias is None else torch.from_numpy(w.sel_bias).cuda(),
                        gating=gating, weights_norm=norm, weights_scale=scale)
    xs = np.stack([oracle.normal(dim, 300 + i, 0.0, 1.0) for i in range(n)])
    normed = torch.from_numpy(xs).cuda()
    ids = torch.empty((n, k), dtype=torch.int32, device="cuda")
    gates = torch.empty((n, k), dtype=torch.float32, device="cuda")
    resid = np.stack([oracle.normal(dim, 600 + i, 0.0, 1.0) for i in range(n)])
    out = torch.from_numpy(resid.copy()).cuda()
    layer(normed, out, combine=be.COMBINE_EXPERT_ASC, ids=ids, gates=gates)
    want, wid, wg = oracle.moe_batch_union(w, xs, resid)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy().astype(np.uint32), wid)
    assert np.all(np.abs(gates.cpu().numpy() - wg) <= 1e-5 * max(1.0, scale))
    _same_bits(out.cpu().numpy(), want, f"gating {gating} down {down_t} n={n}")


@pytest.mark.parametrize("down_t,ffn", [(Q8_0, 512), (Q4_0, 768), (Q8_0, 4096)])
@pytest.mark.parametrize("n", [16, 32])
def test_moe_layer_dev_matrix_core_32_block_downs(be, oracle, down_t, ffn, n):
    """From 16 tokens the batched path runs the expert matmuls on the int8
    matrix cores: the fused Q4_K gate/up on mmq.hip's K-quant kernels and a
    Q8_0 / Q4_0 down on mmq32_kernel in its grouped form (expert planes, the
    groups' pair sources and destinations; ffn 4096 is its widest span
    count).  8 experts top-4, so at 32 tokens the busiest experts take more
    than one group of 16.  Ids, gates and the layer's output bits against
    lo_moe_batch_union."""
    import torch

    dim, E, k = 512, 8, 4
    w = make_layer(oracle, dim, ffn, E, k, seed=90 + ffn + n, gate_t=Q4_K, down_t=down_t)
    layer = _dev_layer(be, w)
    xs = np.stack([oracle.normal(dim, 700 + i, 0.0, 1.0) for i in range(n)])
    normed = torch.from_numpy(xs).cuda()
    ids = torch.empty((n, k), dtype=torch.int32, device="cuda")
    gates = torch.empty((n, k), dtype=torch.float32, device="cuda")
    resid = np.stack([oracle.normal(dim, 900 + i, 0.0, 1.0) for i in range(n)])
    out = torch.from_numpy(resid.copy()).cuda()
    layer(normed, out, combine=be.COMBINE_EXPERT_ASC, ids=ids, gates=gates)
    want, wid, wg = oracle.moe_batch_union(w, xs, resid)
    torch.cuda.synchronize()
    got_ids = ids.cpu().numpy().astype(np.uint32)
    assert np.array_equal(got_ids, wid)
    assert np.bincount(got_ids.ravel(), minlength=E).max() > 16 or n < 32  # some expert spans two groups
    assert np.all(np.abs(gates.cpu().numpy() - wg) <= 1e-5)
    _same_bits(out.cpu().numpy(), want, f"down {down_t} ffn {ffn} n={n}")


# ---- config 5's block: the shared expert, and moeFfnBlock -------------------------


def _c5_layer(oracle, E, k, seed, dim=7168, ffn=2048, sffn=2048):
    """Config 5's routed block at its shapes (hidden 7168, expert ffn 2048,
    Q4_K, sigmoid gating with renorm) over E experts, plus the shared expert
    of width sffn."""
    rng = np.random.default_rng(seed)
    w = make_layer(oracle, dim, ffn, E, k, seed, gate_t=Q4_K, down_t=Q4_K)
    w.gating = oracle.GATING_SIGMOID
    sg = npref.pinned_scale_blocks(Q4_K, sffn, dim, rng)
    su = npref.pinned_scale_blocks(Q4_K, sffn, dim, rng)
    sd = npref.pinned_scale_blocks(Q4_K, dim, sffn, rng)
    w.shexp = (sg, su, sd, Q4_K, Q4_K, Q4_K, sffn)
    return w


def test_moe_ffn_routed_with_shared_expert(be, oracle):
    """backend.moeFfnBlockRouted with `shexp` (src/compute/cpu.zig:68;
    src/vulkan/backend.zig:527-548): the shared expert's FFN added after the
    routed sum in one submission, at config 5's shapes; against the oracle's
    moeRun + shared expert (deepseek.zig:1485-1502): bit-identical (every
    matvec is exact, the combine runs in selection order, then the shared
    expert; north_star asks for 2e-3)."""
    from loom_amd.backend import RoutedCfg, WeightRef

    w = _c5_layer(oracle, E=16, k=8, seed=51)
    sg, su, sd, _, _, _, sffn = w.shexp
    for s in range(2):
        normed = oracle.normal(w.dim, 900 + s, 0.0, 1.0)
        logits = oracle.matvec(F32, w.router.view(np.uint8).ravel(), normed, w.n_expert, w.dim)
        out = np.empty(w.dim, np.float32)
        be.takeCmdBufCount()
        ok = be.moeFfnBlockRouted(normed, logits, None, WeightRef(Q4_K, w.gate), WeightRef(Q4_K, w.up),
                                  WeightRef(Q4_K, w.down),
                                  (WeightRef(Q4_K, sg), WeightRef(Q4_K, su), WeightRef(Q4_K, sd)),
                                  w.ffn, sffn, RoutedCfg(w.n_expert, w.n_used, True, True, 1.0), out)
        assert ok
        assert be.takeCmdBufCount() >= 6  # the routed chain and the shared expert's launches
        want, _, _ = oracle.moe_layer_token(w, normed)
        print(f"routed + shared, token {s}: max-rel {_maxrel(out, want):.2e}", flush=True)
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), _maxrel(out, want)
        # the same block without the shared expert differs by that expert's output
        w2 = oracle.MoeWeights(w.dim, w.ffn, w.n_expert, w.n_used, w.router, w.gate, w.up, w.down, Q4_K, Q4_K,
                               Q4_K, gating=oracle.GATING_SIGMOID)
        routed, _, _ = oracle.moe_layer_token(w2, normed)
        assert _maxrel(out, routed) > 2e-2


@pytest.mark.parametrize("n", [1, 4, 16])
def test_moe_layer_dev_shared_expert(be, oracle, n):
    """loomhip_moe_layer_dev with the layer's shared expert: n = 1 in
    selection order (moeRun), n > 1 ascending-expert (moeBatchUnion), the
    shared expert of every token after its routed experts: bit-identical to
    the oracle."""
    import torch

    from loom_amd import COMBINE_EXPERT_ASC, COMBINE_SELECTION

    w = _c5_layer(oracle, E=16, k=8, seed=52)
    sg, su, sd, _, _, _, sffn = w.shexp

    def dev(raw, rows, cols, planes=1):
        return be.repack_dev(Q4_K, torch.from_numpy(raw).cuda(), rows, cols, planes)

    layer = be.MoeLayer(w.dim, w.ffn, w.n_expert, w.n_used, torch.from_numpy(w.router).cuda(),
                        dev(w.gate, w.ffn, w.dim, w.n_expert), dev(w.up, w.ffn, w.dim, w.n_expert),
                        dev(w.down, w.dim, w.ffn, w.n_expert), Q4_K, Q4_K, Q4_K, gating=oracle.GATING_SIGMOID,
                        shexp=(dev(sg, sffn, w.dim), dev(su, sffn, w.dim), dev(sd, w.dim, sffn), Q4_K, Q4_K, Q4_K,
                               sffn))
    xs = np.stack([oracle.normal(w.dim, 950 + i, 0.0, 1.0) for i in range(n)])
    resid = np.stack([oracle.normal(w.dim, 980 + i, 0.0, 1.0) for i in range(n)])
    out = torch.from_numpy(resid.copy()).cuda() if n > 1 else torch.zeros(1, w.dim, device="cuda")
    layer(torch.from_numpy(xs).cuda(), out, COMBINE_SELECTION if n == 1 else COMBINE_EXPERT_ASC)
    got = out.cpu().numpy()
    if n == 1:
        want, _, _ = oracle.moe_layer_token(w, xs[0])
        want = want[None]
    else:
        want, _, _ = oracle.moe_batch_union(w, xs, resid)
    print(f"n={n}: max-rel {max(_maxrel(got[i], want[i]) for i in range(n)):.2e}", flush=True)
    for i in range(n):
        assert np.array_equal(got[i].view(np.uint32), want[i].view(np.uint32)), (i, _maxrel(got[i], want[i]))


def test_moe_ffn_block_matches_oracle_and_caches(be, oracle):
    """backend.moeFfnBlock (src/compute/cpu.zig:23-30): the selected experts'
    slices with their gates plus the shared expert at weight 1, at config 5's
    shapes.  Every expert's FFN is the CPU kernels' bit for bit and the sum
    runs in list order, so the result is bit-identical to the oracle's
    moeFfnBlock.  Slices outside any registered arena are copied on every call
    -- a Source RAM-cache slot refilled in place (src/p2p/expert_fetch.zig:
    270-321) gives the new bytes' result, not a stale one; once the weights'
    arena is registered (cpu.zig:33 registerArena) a second call is served
    from the HBM tier (hits only, same bits)."""
    from loom_amd.backend import ExpertRef, WeightRef
    from oracle import row_bytes

    w = _c5_layer(oracle, E=8, k=6, seed=53)
    sg, su, sd, _, _, _, sffn = w.shexp
    gb, db = w.ffn * row_bytes(Q4_K, w.dim), w.dim * row_bytes(Q4_K, w.ffn)
    sel = [5, 1, 7, 2, 0, 6]
    gates = [0.3, 0.2, 0.15, 0.15, 0.1, 0.1]

    def refs_of(sel):
        r = [ExpertRef(WeightRef(Q4_K, w.gate[e * gb:(e + 1) * gb]), WeightRef(Q4_K, w.up[e * gb:(e + 1) * gb]),
                       WeightRef(Q4_K, w.down[e * db:(e + 1) * db]), g, w.ffn) for e, g in zip(sel, gates)]
        r.append(ExpertRef(WeightRef(Q4_K, sg), WeightRef(Q4_K, su), WeightRef(Q4_K, sd), 1.0, sffn))
        return r

    def want_of(refs):
        return oracle.moe_ffn_block(normed, [(r.gate.data, r.up.data, r.down.data, Q4_K, Q4_K, Q4_K, r.ffn,
                                              r.weight) for r in refs])

    def run(refs):
        out = np.empty(w.dim, np.float32)
        h0, m0, _ = be.moeFfnBlockStats()
        assert be.moeFfnBlock(normed, refs, out)
        h1, m1, _ = be.moeFfnBlockStats()
        return out, (h1 - h0, m1 - m0)

    be.clearWeightCache()
    try:
        refs = refs_of(sel)
        normed = oracle.normal(w.dim, 990, 0.0, 1.0)
        want = want_of(refs)
        be.takeCmdBufCount()
        out, (h, m) = run(refs)
        assert be.takeCmdBufCount() >= 3 * len(refs)
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32)) and (h, m) == (0, 3 * len(refs))
        # no arena: the same slices are copied again, and a slot refilled in place reads its new bytes
        w.gate[5 * gb:6 * gb] = w.gate[3 * gb:4 * gb]
        w.up[5 * gb:6 * gb] = w.up[3 * gb:4 * gb]
        w.down[5 * db:6 * db] = w.down[3 * db:4 * db]
        want2 = want_of(refs)
        assert not np.array_equal(want2, want)
        out, (h, m) = run(refs)
        assert np.array_equal(out.view(np.uint32), want2.view(np.uint32)) and (h, m) == (0, 3 * len(refs))
        # the weights' arena: kept across calls
        for a in (w.gate, w.up, w.down, sg, su, sd):
            assert be.registerArena(a)
        assert be.materializeArenas() >= w.gate.nbytes + w.up.nbytes + w.down.nbytes
        out, (h, m) = run(refs)
        assert np.array_equal(out.view(np.uint32), want2.view(np.uint32)) and m == 3 * len(refs)
        out, (h, m) = run(refs)
        assert np.array_equal(out.view(np.uint32), want2.view(np.uint32)) and (h, m) == (3 * len(refs), 0)
        # prefetchAsync of the next selection: its copies run on the copy stream, the call waits for them
        refs3 = refs_of([4, 3, 0, 1, 2, 7])
        be.moeFfnBlockPrefetch(w.dim, refs3)
        out, (h, m) = run(refs3)
        assert np.array_equal(out.view(np.uint32), want_of(refs3).view(np.uint32))
        assert (h, m) == (3 * len(refs3), 0)
    finally:
        be.clearWeightCache()  # the arenas end with this test's arrays


def test_moe_ffn_block_declines(be, oracle):
    """More than 16 refs, or a type the kernels do not serve, decline before
    anything is recorded (the caller then runs its own loop)."""
    import loom_amd
    from loom_amd.backend import ExpertRef, WeightRef

    dim, ffn = 512, 256
    rng = np.random.default_rng(3)
    g = npref.pinned_scale_blocks(Q4_K, ffn, dim, rng)
    d = npref.pinned_scale_blocks(Q6_K, dim, ffn, rng)
    ref = ExpertRef(WeightRef(Q4_K, g), WeightRef(Q4_K, g), WeightRef(Q6_K, d), 0.5, ffn)
    out = np.empty(dim, np.float32)
    x = oracle.normal(dim, 1, 0.0, 1.0)
    loom_amd.take_launch_count()
    assert not be.moeFfnBlock(x, [ref] * 17, out)
    bad = ExpertRef(WeightRef(F32, g), WeightRef(F32, g), WeightRef(Q6_K, d), 0.5, ffn)
    assert not be.moeFfnBlock(x, [ref, bad], out)
    assert loom_amd.take_launch_count() == 0
    assert be.moeFfnBlock(x, [ref], out)  # the served form runs
