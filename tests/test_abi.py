"""The C-ABI library loads and exports every symbol include/loomhip.h declares
(CPU only: no compute calls)."""
import ctypes
import os

import pytest

import loom_amd


def test_library_is_built():
    assert os.path.exists(loom_amd.LIB_PATH), "run python -m loom_amd.build"


def test_every_header_symbol_is_exported():
    names = loom_amd.header_symbols()
    assert len(names) >= 20
    L = ctypes.CDLL(loom_amd.LIB_PATH)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_bindings_cover_the_header():
    L = loom_amd.lib()
    for n in loom_amd.header_symbols():
        # every declared entry point has its ctypes signature set
        assert getattr(L, n).argtypes is not None, n


def test_layout_sizes_match_ggml_bytes():
    # device layout keeps GGML's byte count per plane (no padding) when the
    # plane holds a multiple of 8 blocks
    for t in (2, 8, 12, 14):
        for rows, cols in ((768, 2048), (2048, 768), (4096, 4096), (288, 288)):
            if t in (12, 14) and cols % 256:
                continue
            g = loom_amd.ggml_bytes(t, rows, cols)
            p = loom_amd.plane_bytes(t, rows, cols)
            assert p >= g and p - g < 16
            nblocks = rows * cols // (256 if t in (12, 14) else 32)
            if nblocks % 8 == 0:
                assert p == g


def test_init_without_device_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    rc = loom_amd.lib().loomhip_init(0)
    assert rc == loom_amd.ERR_INIT
    assert "device" in loom_amd.last_error()
