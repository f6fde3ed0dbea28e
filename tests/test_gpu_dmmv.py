"""GPU parity of the dequant and dequant-fused matvec kernels against the CPU
oracle: bit-exact (integer block dots + the reference's f32 tail and block
order).  Runs on the MI355X box only."""
import json
import os

import numpy as np
import pytest

import npref

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
Q4_0, Q8_0, Q4_K, Q6_K, F32 = 2, 8, 12, 14, 0


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


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t,rows,cols", [(Q4_0, 5, 288), (Q8_0, 5, 768), (Q4_K, 4, 512),
                                         (Q6_K, 4, 768), (Q4_K, 3, 2048), (Q6_K, 3, 2048)])
def test_dequant_row_bit_exact(be, oracle, t, rows, cols):
    rng = np.random.default_rng(1000 + t + cols)
    raw = npref.random_blocks(t, rows, cols, rng)
    for r in range(rows):
        got = np.empty(cols, np.float32)
        assert be.dequantRow(t, got, raw, r, cols)
        want = oracle.dequant_row(t, raw, r, cols)
        assert np.array_equal(_bits(got), _bits(want)), (t, r)


def test_dequant_dev_whole_tensor_bit_exact(be, oracle):
    import torch

    rng = np.random.default_rng(7)
    for t, rows, cols in ((Q4_K, 64, 2048), (Q6_K, 96, 768), (Q8_0, 40, 2048), (Q4_0, 33, 288)):
        raw = npref.random_blocks(t, rows, cols, rng)
        g = torch.from_numpy(raw).cuda()
        dev = be.repack_dev(t, g, rows, cols, 1)
        out = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
        be.dequant_dev(t, out, dev, rows, cols)
        got = out.cpu().numpy().reshape(rows, cols)
        want = oracle.dequant(t, raw, rows, cols)
        assert np.array_equal(_bits(got), _bits(want)), t


def test_handcrafted_kats_on_device(be, oracle):
    q4k = np.frombuffer(bytes.fromhex(GOLD["q4_k_handcrafted"]["block_hex"]), np.uint8).copy()
    vals = np.empty(256, np.float32)
    assert be.dequantRow(Q4_K, vals, q4k, 0, 256)
    for idx, want in GOLD["q4_k_handcrafted"]["expect_vals"].items():
        assert vals[int(idx)] == want
    out = np.empty(1, np.float32)
    assert be.matvec(Q4_K, out, q4k, np.ones(256, np.float32), 1, 256)
    assert abs(out[0] - GOLD["q4_k_handcrafted"]["expect_dot_ones"]) < 1e-2
    q6k = np.frombuffer(bytes.fromhex(GOLD["q6_k_handcrafted"]["block_hex"]), np.uint8).copy()
    assert be.dequantRow(Q6_K, vals, q6k, 0, 256)
    assert np.all(vals == GOLD["q6_k_handcrafted"]["expect_all"])


SHAPES = [
    (Q4_K, 768, 2048), (Q4_K, 2048, 2048), (Q4_K, 256, 4096), (Q4_K, 2048, 768), (Q4_K, 33, 256),
    (Q6_K, 768, 2048), (Q6_K, 2048, 768), (Q6_K, 256, 4096), (Q6_K, 97, 512),
    (Q8_0, 768, 2048), (Q8_0, 2048, 2048), (Q8_0, 300, 4096), (Q8_0, 288, 288), (Q8_0, 64, 768),
    (Q4_0, 768, 2048), (Q4_0, 288, 288), (Q4_0, 768, 288), (Q4_0, 288, 768), (Q4_0, 100, 4096),
    # rows whose block count leaves the last column chunk partial (hidden 7168 = 28 super-blocks)
    (Q4_K, 64, 2304), (Q4_K, 96, 7168), (Q6_K, 64, 7168), (Q8_0, 40, 1056), (Q4_0, 40, 2080),
]


@pytest.mark.parametrize("t,rows,cols", SHAPES)
def test_matvec_bit_exact(be, oracle, t, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols + t)
    raw = npref.pinned_scale_blocks(t, rows, cols, rng)
    x = oracle.normal(cols, rows + cols, 0.0, 1.0)
    got = np.empty(rows, np.float32)
    be.takeCmdBufCount()
    assert be.matvec(t, got, raw, x, rows, cols)
    assert be.takeCmdBufCount() >= 2  # quantize + matvec ran on the device
    want = oracle.matvec(t, raw, x, rows, cols)
    assert np.array_equal(_bits(got), _bits(want)), np.abs(got - want).max()


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_matvec_quantized_normal_weights(be, oracle, t):
    """Config-2 recipe: N(0, 0.02) weights through the GGML quantizers."""
    rows, cols = 768, 2048
    w = oracle.normal(rows * cols, 42 + t, 0.0, 0.02).reshape(rows, cols)
    raw = oracle.quantize(t, w)
    x = oracle.normal(cols, 43, 0.0, 1.0)
    got = np.empty(rows, np.float32)
    assert be.matvec(t, got, raw, x, rows, cols)
    assert np.array_equal(_bits(got), _bits(oracle.matvec(t, raw, x, rows, cols)))


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_matmul_bit_exact_to_per_vector_oracle(be, oracle, t):
    rows, cols = 300, 2048
    rng = np.random.default_rng(55 + t)
    raw = npref.pinned_scale_blocks(t, rows, cols, rng)
    for n in (2, 3, 4, 5, 8, 11, 16, 33):
        xs = np.stack([oracle.normal(cols, 1000 * n + k, 0.0, float(k + 1)) for k in range(n)])
        got = np.empty((n, rows), np.float32)
        assert be.matmul(t, got, raw, xs, n, rows, cols)
        want = np.stack([oracle.matvec(t, raw, xs[k], rows, cols) for k in range(n)])
        assert np.array_equal(_bits(got), _bits(want)), n


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0, Q4_0])
@pytest.mark.parametrize("rows,cols", [(37, 768), (300, 4096), (64, 256), (130, 2048)])
def test_matmul_matrix_cores_bit_exact(be, oracle, t, rows, cols):
    """From 16 vectors on, Q4_K / Q6_K matmuls run on the int8 matrix cores
    (mmq.hip, groups of 32), and so do Q8_0 / Q4_0 over whole 64-value spans
    (mmq32_kernel: a wave per 16-row tile walks the blocks in order, 16 vectors
    a group): bit-identical to per-vector oracle matvecs, including ragged row
    tiles and groups."""
    rng = np.random.default_rng(77 + t + rows)
    raw = npref.pinned_scale_blocks(t, rows, cols, rng)
    for n in (16, 17, 32, 45):
        xs = np.stack([oracle.normal(cols, 3000 * n + k, 0.0, float(k % 5 + 1)) for k in range(n)])
        got = np.empty((n, rows), np.float32)
        assert be.matmul(t, got, raw, xs, n, rows, cols)
        want = np.stack([oracle.matvec(t, raw, xs[k], rows, cols) for k in range(n)])
        assert np.array_equal(_bits(got), _bits(want)), n


def test_f32_matvec_bit_exact(be, oracle):
    for rows, cols in ((128, 2048), (64, 288), (30, 100), (8, 7)):
        w = oracle.normal(rows * cols, rows, 0.0, 1.0 / np.sqrt(cols)).reshape(rows, cols)
        x = oracle.normal(cols, cols, 0.0, 1.0)
        got = np.empty(rows, np.float32)
        assert be.matvec(F32, got, w.view(np.uint8).ravel(), x, rows, cols)
        want = oracle.matvec(F32, w.view(np.uint8).ravel(), x, rows, cols)
        assert np.array_equal(_bits(got), _bits(want)), (rows, cols)


def test_declines_unserved_types(be):
    raw = np.zeros(144 * 2, np.uint8)
    out = np.empty(1, np.float32)
    assert be.matvec(1, out, raw, np.zeros(4, np.float32), 1, 4) is False  # f16 declined
    assert be.matvec(Q4_K, out, raw, np.zeros(300, np.float32), 1, 300) is False  # not whole blocks


def test_nonfinite_activations_stay_finite(be, oracle):
    rows, cols = 64, 256
    raw = npref.pinned_scale_blocks(Q4_K, rows, cols, np.random.default_rng(3))
    x = oracle.normal(cols, 9, 0.0, 1.0)
    x[0], x[1], x[2] = np.nan, np.inf, -np.inf
    got = np.empty(rows, np.float32)
    assert be.matvec(Q4_K, got, raw, x, rows, cols)
    want = oracle.matvec(Q4_K, raw, x, rows, cols)
    assert np.all(np.isfinite(got))
    assert np.array_equal(_bits(got), _bits(want))
