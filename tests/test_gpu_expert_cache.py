"""GPU tests of the HBM expert cache (src/engine/expert_cache.zig on the
device tier) and the routed MoE layer that reads its experts through it.

  * the hit/miss bookkeeping equals the oracle's replay of ExpertCache.get
    (oracle/cache_ref.c, itself pinned to the reference's LRU KAT and an
    OrderedDict replay) on the same access trace, exactly;
  * every block handed out holds its backing bytes (read back from HBM);
  * the cached MoE layer's output is bit-identical to the resident layer's
    (loomhip_moe_layer_dev) on the same weights, at one token (moeFFN's
    selection order) and at batches forced through several rounds;
  * pin, prefetch, clear and a missing backing block behave as the
    reference's pin / (warm-up reads) / Lru.clear / Lru.abort.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14


@pytest.fixture(scope="module")
def ec_mod(oracle):
    import loom_amd

    loom_amd.init(0)
    from loom_amd import expert_cache

    return expert_cache


def _hip():
    """The HIP runtime torch loaded (for reading raw device addresses back)."""
    for line in open("/proc/self/maps"):
        if "libamdhip64" in line:
            L = C.CDLL(line.split()[-1])
            L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            return L
    raise RuntimeError("libamdhip64 not loaded")


def _read_dev(addr, n):
    import torch

    torch.cuda.synchronize()
    out = np.empty(n, np.uint8)
    assert _hip().hipMemcpy(out.ctypes.data, addr, n, 2) == 0  # device -> host
    return out


def _zipf_trace(rng, n_ids, n, s=1.1):
    p = 1.0 / np.arange(1, n_ids + 1) ** s
    perm = rng.permutation(n_ids)
    return perm[rng.choice(n_ids, size=n, p=p / p.sum())].astype(np.uint32)


def test_get_matches_oracle_replay_and_contents(ec_mod, oracle):
    n_ids, slot, cap = 40, 4096, 6
    rng = np.random.default_rng(3)
    host = ec_mod.HostBuffer(n_ids * slot)
    host.array[:] = rng.integers(0, 256, host.nbytes, dtype=np.uint8)
    ec = ec_mod.ExpertCache(cap, slot, n_ids, pin_slots=2)
    for i in range(n_ids):
        ec.set_source(i, host, i * slot, slot)
    ec.pin([0, 3])
    assert ec.pinnedCount() == 2
    trace = _zipf_trace(rng, n_ids, 400)
    for j, i in enumerate(trace):
        addr = ec.get(int(i))
        if j % 37 == 0:
            assert np.array_equal(_read_dev(addr, slot), host.array[i * slot:(i + 1) * slot]), j
    pinned = np.zeros(n_ids, np.uint8)
    pinned[[0, 3]] = 1
    counts, _ = oracle.cache_replay(cap, trace, pinned=pinned, n_ids=n_ids)
    st = ec.stats
    assert (st.pin_hits, st.lru_hits, st.disk_misses) == tuple(int(c) for c in counts)
    assert st.bytes_read == st.disk_misses * slot
    assert (st.warmup_reads, st.warmup_bytes) == (2, 2 * slot)
    assert abs(st.hitRate() - (counts[0] + counts[1]) / len(trace)) < 1e-12
    acc = ec.access_counts()
    assert np.array_equal(acc, np.bincount(trace, minlength=n_ids).astype(np.uint64))
    # the pinner's input: stats.hottestWithinBudget over these counts
    assert oracle.hottest_within_budget(acc, slot, 3 * slot)[0] == int(np.argmax(acc))
    ec.close()


def test_refill_waits_for_the_slot_users(ec_mod):
    """Capacity 1: every get of another id evicts the only slot; each block's
    bytes are read by a device copy enqueued right after its get, before
    the next eviction, and must be that block's bytes."""
    import torch

    n_ids, slot = 8, 1 << 20
    rng = np.random.default_rng(5)
    host = ec_mod.HostBuffer(n_ids * slot)
    host.array[:] = rng.integers(0, 256, host.nbytes, dtype=np.uint8)
    ec = ec_mod.ExpertCache(1, slot, n_ids)
    for i in range(n_ids):
        ec.set_source(i, host, i * slot, slot)
    seq = [1, 2, 1, 5, 7, 7, 0, 3]
    outs = []
    hip = _hip()
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    st = torch.cuda.current_stream()
    for i in seq:
        addr = ec.get(i)
        o = torch.empty(slot, dtype=torch.uint8, device="cuda")
        assert hip.hipMemcpyAsync(o.data_ptr(), addr, slot, 3, C.c_void_p(st.cuda_stream)) == 0
        ec.release()
        outs.append(o)
    torch.cuda.synchronize()
    for i, o in zip(seq, outs):
        assert np.array_equal(o.cpu().numpy(), host.array[i * slot:(i + 1) * slot]), i
    assert ec.stats.disk_misses == 7 and ec.stats.lru_hits == 1
    ec.close()


def test_missing_source_aborts_and_prefetch_warms(ec_mod):
    from loom_amd import LoomHipError

    n_ids, slot = 10, 256
    host = ec_mod.HostBuffer(n_ids * slot)
    host.array[:] = np.arange(host.nbytes, dtype=np.uint64).astype(np.uint8)
    ec = ec_mod.ExpertCache(3, slot, n_ids)
    for i in range(n_ids - 1):  # id 9 has no backing block
        ec.set_source(i, host, i * slot, slot)
    ec.get(0)
    with pytest.raises(LoomHipError):
        ec.get(9)
    # the failed reserve returned its slot: ids 1 and 2 still fit without evicting 0
    ec.get(1)
    ec.get(2)
    ec.get(0)
    st = ec.stats
    assert (st.lru_hits, st.disk_misses) == (1, 3)
    ec.prefetch([4, 0])  # 4 absent: warm-up read (evicts the LRU tail, 1); 0 present: untouched
    ec.get(4)
    st = ec.stats
    assert (st.lru_hits, st.disk_misses, st.warmup_reads) == (2, 3, 1)
    ec.clear()
    ec.get(0)
    assert ec.stats.disk_misses == 4
    ec.close()


def _layer(E, dim, ffn, k, seed, gating):
    import torch

    from loom_amd import backend as be

    gate = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, ffn, dim, E, seed * 10 + 1, 0.02), ffn, dim, E)
    up = be.repack_dev(Q4_K, be.synth_ggml_dev(Q4_K, ffn, dim, E, seed * 10 + 2, 0.02), ffn, dim, E)
    down = be.repack_dev(Q6_K, be.synth_ggml_dev(Q6_K, dim, ffn, E, seed * 10 + 3, 0.02), dim, ffn, E)
    g = torch.Generator(device="cuda").manual_seed(seed)
    router = (torch.randn(E, dim, generator=g, device="cuda") / np.sqrt(dim)).contiguous()
    ranks = torch.randperm(E, generator=g, device="cuda").float() + 1
    z = -1.1 * torch.log(ranks)
    bias = (z - z.mean()).contiguous()
    res = be.MoeLayer(dim, ffn, E, k, router, gate, up, down, Q4_K, Q4_K, Q6_K, router_bias=bias,
                      gating=gating)
    return res, (gate, up, down, router, bias)


def _cached_setup(ec_mod, E, dim, ffn, k, cap, tensors, gating, pin=()):
    import torch

    from loom_amd import MoeLayerEcDesc, plane_bytes

    gate, up, down, router, bias = tensors
    gb, db = plane_bytes(Q4_K, ffn, dim), plane_bytes(Q6_K, dim, ffn)
    slot = 2 * gb + db
    host = ec_mod.HostBuffer(E * slot)
    hv = torch.from_numpy(host.array)
    for e in range(E):
        o = e * slot
        hv[o:o + gb].copy_(gate[e * gb:(e + 1) * gb].cpu())
        hv[o + gb:o + 2 * gb].copy_(up[e * gb:(e + 1) * gb].cpu())
        hv[o + 2 * gb:o + slot].copy_(down[e * db:(e + 1) * db].cpu())
    ec = ec_mod.ExpertCache(cap, slot, E, pin_slots=len(pin))
    for e in range(E):
        ec.set_source(e, host, e * slot, slot)
    if pin:
        ec.pin(list(pin))
    desc = MoeLayerEcDesc(dim, ffn, E, k, gating, 1, 1.0, router.data_ptr(), bias.data_ptr(), None, Q4_K,
                          Q6_K, 0, 0, gb, 2 * gb)
    return ec, desc, host


@pytest.mark.parametrize("n_tok,cap,pin", [(1, 5, ()), (1, 3, (2,)), (6, 4, ()), (24, 7, (0, 5))])
def test_cached_layer_matches_resident(ec_mod, oracle, n_tok, cap, pin):
    import torch

    from loom_amd import COMBINE_EXPERT_ASC, COMBINE_SELECTION, GATING_SOFTMAX

    E, dim, ffn, k = 32, 512, 256, 4
    res, tensors = _layer(E, dim, ffn, k, 11, GATING_SOFTMAX)
    ec, desc, host = _cached_setup(ec_mod, E, dim, ffn, k, cap, tensors, GATING_SOFTMAX, pin)
    g = torch.Generator(device="cuda").manual_seed(n_tok)
    trace = []
    for step in range(5):
        x = torch.randn(n_tok, dim, generator=g, device="cuda")
        want = torch.zeros(n_tok, dim, device="cuda")
        ids_res = torch.zeros(n_tok, k, dtype=torch.int32, device="cuda")
        res(x, want, COMBINE_SELECTION if n_tok == 1 else COMBINE_EXPERT_ASC, ids=ids_res)
        got = torch.full((n_tok, dim), float("nan"), device="cuda")
        ids, gates = ec.moe_layer(desc, x, got, n_tok, want_ids=True)
        torch.cuda.synchronize()
        assert np.array_equal(ids.astype(np.int32), ids_res.cpu().numpy())
        assert torch.equal(got, want), (step, float((got - want).abs().max()))
        trace += list(ids[0]) if n_tok == 1 else sorted(set(ids.ravel().tolist()))
    pinned = np.zeros(E, np.uint8)
    pinned[list(pin)] = 1
    counts, _ = oracle.cache_replay(cap, np.array(trace, np.uint32), pinned=pinned, n_ids=E)
    st = ec.stats
    assert (st.pin_hits, st.lru_hits, st.disk_misses) == tuple(int(c) for c in counts)
    ec.close()


def test_hit_on_a_prefetched_slot_waits_for_its_fill(ec_mod):
    """A prefetch fills its slot on the copy stream; a get that hits that slot
    right away, from another (non-blocking) stream, must see the whole block:
    the hit makes the consumer wait for the fill still in flight.  Large
    blocks, each slot first filled with another expert's bytes, so a read
    that ran ahead of the fill would see the wrong bytes."""
    import torch

    n_ids, slot, cap = 6, 16 << 20, 2
    rng = np.random.default_rng(9)
    host = ec_mod.HostBuffer(n_ids * slot)
    host.array[:] = rng.integers(0, 256, host.nbytes, dtype=np.uint8)
    ec = ec_mod.ExpertCache(cap, slot, n_ids)
    for i in range(n_ids):
        ec.set_source(i, host, i * slot, slot)
    hip = _hip()
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    side = torch.cuda.Stream()  # non-blocking with respect to the library's copy stream
    for rnd in range(3):
        base = 2 * (rnd % 2)
        for i in (base, base + 1):  # occupy both slots with other experts' bytes
            ec.get(i)
        ec.release()
        torch.cuda.synchronize()
        want = [4, 5] if rnd != 1 else [5, 4]
        ec.prefetch(want)  # both slots refilled asynchronously
        outs = []
        for i in want:
            addr = ec.get(i, stream=side.cuda_stream)
            o = torch.empty(slot, dtype=torch.uint8, device="cuda")
            assert hip.hipMemcpyAsync(o.data_ptr(), addr, slot, 3, C.c_void_p(side.cuda_stream)) == 0
            outs.append((i, o))
        ec.release(stream=side.cuda_stream)
        side.synchronize()
        for i, o in outs:
            assert np.array_equal(o.cpu().numpy(), host.array[i * slot:(i + 1) * slot]), (rnd, i)
        ec.clear()
    st = ec.stats
    assert st.warmup_reads == 6 and st.lru_hits == 6
    ec.close()


def _c5_cached_layer(ec_mod, oracle, E, cap, seed, dim=7168, ffn=2048, sffn=2048, k=8):
    """Config 5's routed block as the benchmark builds it -- Q4_K experts of
    hidden `dim` and ffn `ffn`, sigmoid gating with renorm, the Zipf(1.1)
    popularity as a logit bias, a resident shared expert -- with its E
    experts in pinned host memory behind a `cap`-slot cache.  Returns the
    oracle's MoeWeights over the same GGML bytes, the cached layer's
    descriptor, the cache, and what must stay alive."""
    import torch

    import npref
    from loom_amd import GATING_SIGMOID, MoeLayerEcDesc, plane_bytes
    from loom_amd import backend as be

    rng = np.random.default_rng(seed)
    gate = npref.pinned_scale_blocks(Q4_K, ffn, dim, rng, planes=E)
    up = npref.pinned_scale_blocks(Q4_K, ffn, dim, rng, planes=E)
    down = npref.pinned_scale_blocks(Q4_K, dim, ffn, rng, planes=E)
    sg = npref.pinned_scale_blocks(Q4_K, sffn, dim, rng)
    su = npref.pinned_scale_blocks(Q4_K, sffn, dim, rng)
    sd = npref.pinned_scale_blocks(Q4_K, dim, sffn, rng)
    router = oracle.normal(E * dim, seed + 1, 0.0, 1.0 / np.sqrt(dim)).reshape(E, dim)
    ranks = rng.permutation(E) + 1
    zipf = np.log(1.0 / ranks ** 1.1)
    rb = (zipf - zipf.mean()).astype(np.float32)
    w = oracle.MoeWeights(dim, ffn, E, k, router, gate, up, down, Q4_K, Q4_K, Q4_K, router_bias=rb,
                          gating=oracle.GATING_SIGMOID, weights_norm=True,
                          shexp=(sg, su, sd, Q4_K, Q4_K, Q4_K, sffn))

    def dev(raw, rows, cols, planes=1):
        return be.repack_dev(Q4_K, torch.from_numpy(raw).cuda(), rows, cols, planes)

    gb, db = plane_bytes(Q4_K, ffn, dim), plane_bytes(Q4_K, dim, ffn)
    slot = 2 * gb + db
    host = ec_mod.HostBuffer(E * slot)
    hv = torch.from_numpy(host.array)
    for raw, rows, cols, off, pb in ((gate, ffn, dim, 0, gb), (up, ffn, dim, gb, gb), (down, dim, ffn, 2 * gb, db)):
        d = dev(raw, rows, cols, E).view(E, pb).cpu()
        for e in range(E):
            hv[e * slot + off:e * slot + off + pb].copy_(d[e])
        del d
    sh = (dev(sg, sffn, dim), dev(su, sffn, dim), dev(sd, dim, sffn))
    router_d, rb_d = torch.from_numpy(router).cuda(), torch.from_numpy(rb).cuda()
    desc = MoeLayerEcDesc(dim, ffn, E, k, GATING_SIGMOID, 1, 1.0, router_d.data_ptr(), rb_d.data_ptr(), None,
                          Q4_K, Q4_K, 0, 0, gb, 2 * gb, Q4_K, Q4_K, Q4_K, sh[0].data_ptr(), sh[1].data_ptr(),
                          sh[2].data_ptr(), sffn)
    ec = ec_mod.ExpertCache(cap, slot, E)
    for e in range(E):
        ec.set_source(e, host, e * slot, slot)
    return w, desc, ec, (host, sh, router_d, rb_d), slot


@pytest.mark.parametrize("n_tok,steps", [(1, 6), (64, 2)])
def test_cached_layer_config5_matches_oracle(ec_mod, oracle, n_tok, steps):
    """Config 5's routed block as the benchmark drives it: loomhip_moe_layer_
    cached at hidden 7168, expert ffn 2048, Q4_K, sigmoid gating with renorm,
    the Zipf(1.1) popularity as a logit bias, and the resident shared expert
    (its arm of the cached layer), over 32 experts streamed from pinned host
    memory through an 8-slot LRU, so misses and evictions occur and 64 tokens
    need several rounds of gets.  Against the oracle on the same GGML bytes:
    moeRun + shared expert at one token (src/gguf/deepseek.zig:1485-1502),
    moeBatchUnion + shared expert at 64 (src/gguf/llama.zig:1828-1924).  Ids
    exact, gates within 1e-6, outputs bit-identical (north_star asks for
    2e-3), and the hit and miss counts equal to the oracle's replay of the
    call's own access trace (src/engine/expert_cache.zig:230-249)."""
    import torch

    E, cap, dim = 32, 8, 7168
    w, desc, ec, keep, slot = _c5_cached_layer(ec_mod, oracle, E, cap, 77)
    trace = []
    try:
        for step in range(steps):
            xs = np.stack([oracle.normal(dim, 700 + 100 * step + i, 0.0, 1.0) for i in range(n_tok)])
            got = torch.full((n_tok, dim), float("nan"), device="cuda")
            print(f"n_tok={n_tok} step {step}", flush=True)
            ids, gates = ec.moe_layer(desc, torch.from_numpy(xs).cuda(), got, n_tok, want_ids=True)
            torch.cuda.synchronize()
            got = got.cpu().numpy()
            if n_tok == 1:
                want, wids, wgates = oracle.moe_layer_token(w, xs[0])
                want, wids, wgates = want[None], wids[None], wgates[None]
            else:
                want, wids, wgates = oracle.moe_batch_union(w, xs, np.zeros_like(xs))
            assert np.array_equal(ids, wids), step
            assert np.abs(gates - wgates).max() <= 1e-6, step
            rel = max(float(np.abs(got[i] - want[i]).max() / np.abs(want[i]).max()) for i in range(n_tok))
            print(f"  max-rel {rel:.2e}, distinct experts {len(set(ids.ravel().tolist()))}", flush=True)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (step, rel)
            trace += list(ids[0]) if n_tok == 1 else sorted(set(ids.ravel().tolist()))
        counts, _ = oracle.cache_replay(cap, np.array(trace, np.uint32))
        st = ec.stats
        assert st.disk_misses > 0 and (st.pin_hits, st.lru_hits, st.disk_misses) == tuple(int(c) for c in counts)
        assert st.bytes_read == st.disk_misses * slot
    finally:
        ec.close()
        keep[0].free()


@pytest.mark.parametrize("n", [1, 4])
def test_mla_block_with_streamed_experts_matches_the_engine_sequence(ec_mod, oracle, n):
    """Config 5 as one block (loomhip_mla_layer_cached_dev): for n sequences
    each over its own 37-position compressed cache, the MLA attention (16
    heads of nope 128 / rope 64 / v 128, kv_lora 512, Q4_K kv_b), x += wo .
    heads (Q4_K [7168][2048]), the exact FFN rmsnorm, the routed experts
    through an 8-slot cache over 32 streamed experts plus the resident shared
    expert, x += that -- against the engine's own sequence on the oracle (the
    host head loop, matvec, residual add, rmsnorm, moeRun + shared expert at
    one sequence, moeBatchUnion + shared expert for more; deepseek.zig:
    1044-1046, 1275-1440): x bit-identical over three calls, ids exact, the
    LRU counts equal to the oracle's replay."""
    import torch

    from loom_amd import backend as be
    from mla_case import make_case
    from recipes import planes

    E, cap, dim, H, nope, vd, kvr, rope, ctx, seq, eps = 32, 8, 7168, 16, 128, 128, 512, 64, 48, 37, 1e-6
    w, desc, ec, keep, slot = _c5_cached_layer(ec_mod, oracle, E, cap, 91)
    cases = [make_case(oracle, Q4_K, H, nope, vd, kvr, rope, ctx, seed=200 + i) for i in range(n)]
    kvb = cases[0].kv_b  # one layer: one kv_b for every sequence
    attn = be.MlaAttn(Q4_K, torch.from_numpy(kvb).cuda(), H, nope, vd, kvr, rope, cases[0].scale)
    wo = planes(Q4_K, dim, H * vd, 1, 93)
    wo_d = be.repack_dev(Q4_K, torch.from_numpy(wo).cuda(), dim, H * vd, 1)
    rng = np.random.default_rng(94)
    ffn_norm = (1.0 + 0.05 * rng.standard_normal(dim)).astype(np.float32)
    caches = [(torch.from_numpy(c.c_kv).cuda(), torch.from_numpy(c.k_rope).cuda()) for c in cases]
    x = rng.standard_normal((n, dim)).astype(np.float32)
    xd = torch.from_numpy(x.copy()).cuda()
    norm_d = torch.from_numpy(ffn_norm).cuda()
    trace = []
    try:
        for call in range(3):
            qn = rng.standard_normal((n, H * nope)).astype(np.float32)
            qr = rng.standard_normal((n, H * rope)).astype(np.float32)
            ids = attn.cached_block([c for c, _ in caches], [r for _, r in caches], seq, torch.from_numpy(qn).cuda(),
                                    torch.from_numpy(qr).cuda(), Q4_K, wo_d, norm_d, eps, desc, ec, xd,
                                    want_ids=True)
            torch.cuda.synchronize()
            # the engine's sequence on the oracle
            x1 = np.empty_like(x)
            for i, c in enumerate(cases):
                heads, _ = oracle.mla_attn_heads(c.c_kv, c.k_rope, seq, qn[i], qr[i], Q4_K, kvb, H, nope, vd,
                                                 c.scale)
                x1[i] = x[i] + oracle.matvec(Q4_K, wo, heads, dim, H * vd)
            normed = np.stack([oracle.rmsnorm(x1[i], ffn_norm, eps) for i in range(n)])
            if n == 1:
                acc, wids, _ = oracle.moe_layer_token(w, normed[0])
                acc, wids = acc[None], wids[None]
            else:
                acc, wids, _ = oracle.moe_batch_union(w, normed, np.zeros_like(normed))
            x = x1 + acc
            got = xd.cpu().numpy()
            print(f"n={n} call {call}: max |diff| {float(np.abs(got - x).max()):.2e}", flush=True)
            assert np.array_equal(ids, wids), call
            assert np.array_equal(got.view(np.uint32), x.view(np.uint32)), call
            trace += list(ids[0]) if n == 1 else sorted(set(ids.ravel().tolist()))
        counts, _ = oracle.cache_replay(cap, np.array(trace, np.uint32))
        st = ec.stats
        assert (st.pin_hits, st.lru_hits, st.disk_misses) == tuple(int(c) for c in counts)
    finally:
        ec.close()
        keep[0].free()
