"""exl3_quantize_tiles_noalloc (static device scratch, no allocation) against
exl3_quantize_tiles with caller-allocated scratch, both through the C-ABI:
identical states and reconstruction on two calls in a row, the second with
fewer tiles, at several bitrates; a batch above the static scratch's limit
is rejected before anything is launched."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 512 << 20


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _max_tiles(lib, K, L=256):
    per_tile = 4 * (65536 >> K) + int(lib.exl3_scratch_edges_bytes(K, L, 1))
    return (NOALLOC_BYTES - 255) // per_tile


def _encode_reference(torch, lib, x, K):
    """exl3_quantize_tiles with torch-allocated scratch for all tiles."""
    from exl3_intel_arc_quantizer_amd._native import edges_shape
    n = x.shape[0]
    out_w = torch.empty((n, 256), dtype=torch.float32, device="cuda")
    out_i = torch.empty((n, 256), dtype=torch.int16, device="cuda")
    costs = torch.empty((n, 2, 65536 >> K), dtype=torch.float16, device="cuda")
    edges = torch.empty(edges_shape(n, K), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.exl3_quantize_tiles(x.data_ptr(), out_w.data_ptr(), out_i.data_ptr(),
                                 costs.data_ptr(), edges.data_ptr(), n, n, K, 2, 256, 0, 0, stream)
    assert rc == 0, lib.exl3_last_error()
    torch.cuda.synchronize()
    return out_w, out_i


def _encode_noalloc(torch, lib, x, K):
    n = x.shape[0]
    out_w = torch.empty((n, 256), dtype=torch.float32, device="cuda")
    out_i = torch.empty((n, 256), dtype=torch.int16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.exl3_quantize_tiles_noalloc(x.data_ptr(), out_w.data_ptr(), out_i.data_ptr(), n, K,
                                         2, 256, 0, stream)
    assert rc == 0, lib.exl3_last_error()
    torch.cuda.synchronize()
    return out_w, out_i


@pytest.mark.parametrize("K", [2, 4, 6])
def test_noalloc_matches_allocating_entry_point(torch_mod, K):
    from exl3_intel_arc_quantizer_amd._native import extension, load_library
    torch = torch_mod
    lib = load_library()
    ext = extension()
    cap = _max_tiles(lib, K)
    assert cap >= 200
    rng = np.random.default_rng(900 + K)
    for n in (min(cap, 320), 37):                  # second call smaller than the first
        print(f"noalloc K={K} n={n} (limit {cap})", flush=True)
        raw = torch.from_numpy(rng.standard_normal((n, 256)).astype(np.float32)).cuda()
        x = torch.empty_like(raw)
        ext.prepare_tiles(raw, x, True)
        want_w, want_i = _encode_reference(torch, lib, x, K)
        got_w, got_i = _encode_noalloc(torch, lib, x, K)
        assert torch.equal(got_i, want_i)
        assert torch.equal(got_w.view(torch.int32), want_w.view(torch.int32))


def test_noalloc_rejects_batches_above_the_limit(torch_mod):
    from exl3_intel_arc_quantizer_amd._native import load_library
    torch = torch_mod
    lib = load_library()
    cap = _max_tiles(lib, 2)
    n = cap + 1
    x = torch.zeros((n, 256), dtype=torch.float32, device="cuda")
    out_w = torch.full((n, 256), 7.0, dtype=torch.float32, device="cuda")
    out_i = torch.zeros((n, 256), dtype=torch.int16, device="cuda")
    rc = lib.exl3_quantize_tiles_noalloc(x.data_ptr(), out_w.data_ptr(), out_i.data_ptr(), n, 2,
                                         2, 256, 0, torch.cuda.current_stream().cuda_stream)
    assert rc != 0
    msg = lib.exl3_last_error().decode()
    assert "static scratch" in msg and f"at most {cap} tiles" in msg, msg
    torch.cuda.synchronize()
    assert bool((out_w == 7.0).all())                        # nothing was launched
    assert lib.exl3_quantize_tiles_noalloc(x.data_ptr(), out_w.data_ptr(), out_i.data_ptr(), 4,
                                           9, 2, 256, 0, None) != 0
    assert b"K must be" in lib.exl3_last_error()
    assert ctypes.c_int(lib.exl3_quantize_tiles_noalloc(None, None, None, 4, 2, 2, 256, 0,
                                                        None)).value != 0
