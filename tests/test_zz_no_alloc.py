"""The no-allocation MoE entry point (loomhip_moe_layer_dev_noalloc: the
workspace in a fixed per-GPU device array) against loomhip_moe_layer_dev on
the same inputs: two calls in a row, the second with fewer tokens, each
bit-identical to the allocating entry point; an oversized call is refused
before anything launches."""
import ctypes as C

import numpy as np
import pytest

from test_gpu_moe import _dev_layer, make_layer

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14


@pytest.fixture(scope="module")
def be(oracle):
    import loom_amd
    from loom_amd import backend

    loom_amd.init(0)
    backend.clearWeightCache()
    yield backend
    backend.clearWeightCache()


def _call(fn, layer, x, out, combine, ids):
    from loom_amd import lib
    from loom_amd.backend import _ptr, _stream

    return getattr(lib(), fn)(C.byref(layer.desc), _ptr(x), x.shape[0], combine, _ptr(out), _ptr(ids), None,
                              _stream())


def test_noalloc_matches_allocating_entry_point(be, oracle):
    import torch

    import loom_amd
    from loom_amd import COMBINE_EXPERT_ASC, COMBINE_SELECTION

    w = make_layer(oracle, 2048, 768, 128, 8, seed=71, router_bias=True)  # config 3 shapes
    layer = _dev_layer(be, w)
    g = torch.Generator(device="cuda").manual_seed(5)
    # 32 tokens (grouped matrix-core path), then 3 (decode path): the second
    # call reuses the array the first one left behind
    for n, comb in ((32, COMBINE_EXPERT_ASC), (3, COMBINE_SELECTION)):
        x = torch.randn(n, 2048, generator=g, device="cuda")
        base = torch.randn(n, 2048, generator=g, device="cuda")
        out_a, out_b = base.clone(), base.clone()
        ids_a = torch.zeros(n, 8, dtype=torch.int32, device="cuda")
        ids_b = torch.full((n, 8), -1, dtype=torch.int32, device="cuda")
        assert _call("loomhip_moe_layer_dev", layer, x, out_a, comb, ids_a) == loom_amd.OK
        loom_amd.take_launch_count()
        assert _call("loomhip_moe_layer_dev_noalloc", layer, x, out_b, comb, ids_b) == loom_amd.OK, \
            loom_amd.last_error()
        assert loom_amd.take_launch_count() >= 3
        torch.cuda.synchronize()
        assert torch.equal(ids_a, ids_b), n
        assert np.array_equal(out_a.cpu().numpy().view(np.uint32), out_b.cpu().numpy().view(np.uint32)), n


def test_noalloc_refuses_a_workspace_beyond_the_array(be, oracle):
    import torch

    import loom_amd
    from loom_amd import COMBINE_EXPERT_ASC

    w = make_layer(oracle, 2048, 768, 128, 8, seed=72)
    layer = _dev_layer(be, w)
    x = torch.randn(256, 2048, device="cuda")
    out = torch.zeros(256, 2048, device="cuda")
    loom_amd.take_launch_count()
    rc = _call("loomhip_moe_layer_dev_noalloc", layer, x, out, COMBINE_EXPERT_ASC, None)
    assert rc == loom_amd.ERR_ARG
    assert "fixed scratch" in loom_amd.last_error()
    assert loom_amd.take_launch_count() == 0
