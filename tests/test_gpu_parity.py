"""GPU parity: the HIP encoder through the C-ABI against the reference's golden
vectors and the C oracle (bit-exact), mirroring the reference's device tests
(tests/test_xpu_quantizer.py of alpha2beta/EXL3_Intel_Arc_quantizer).

Run on an MI355X:  python -u -m pytest tests -m gpu -x -v --timeout 120
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import c_oracle
from oracle.trellis_format_ref import codebook_lut as oracle_lut
from oracle.trellis_format_ref import decode_states
from oracle.trellis_format_ref import tensor_core_perm as oracle_tc_perm

from .conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


@pytest.fixture(scope="module")
def ext():
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import build_quantize_extension
    return build_quantize_extension()


def _encoder(**kw):
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import XPUTrellisEncoder
    return XPUTrellisEncoder(**kw)


def _assert_bd_matches(bd, g, sel, K):
    np.testing.assert_array_equal(bd.output_indices, g["output_indices"][sel])
    np.testing.assert_array_equal(bd.end_states, g["end_state"][sel])
    np.testing.assert_array_equal(bd.path_costs.astype(np.float64), g["path_cost"][sel])
    np.testing.assert_array_equal(bd.distortions.astype(np.float64), g["distortion"][sel])
    if bd.packed.shape[1]:
        np.testing.assert_array_equal(bd.packed, g["packed"][sel][:, :16 * K])
    np.testing.assert_array_equal(bd.reconstructed_tiles.view(np.uint16),
                                  g["reconstructed"][sel])
    np.testing.assert_array_equal(bd.reconstructed_perm.view(np.uint16),
                                  g["reconstructed_perm"][sel])


def test_codebook_bit_exact(ext, torch_mod):
    """tests/test_xpu_quantizer.py:75-86."""
    for cb in (0, 1, 2):
        out = torch_mod.empty(65536, dtype=torch_mod.float16, device="cuda")
        ext.decode_codebook(cb, out)
        torch_mod.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16),
                                      oracle_lut(cb).view(np.uint16))


def test_fp16_fma_probe(ext, torch_mod):
    """The 11 adversarial pairs and 65536 random pairs of xpu_probe.py:153-272:
    v_fma_f16 rounds once, subnormals kept."""
    from .test_oracle_known_answers import ADV_COST, ADV_DH
    rng = np.random.default_rng(2026)
    dh = np.concatenate([np.array(ADV_DH, dtype=np.uint16).view(np.float16),
                         rng.normal(0.0, 1.0, size=65536).astype(np.float16)])
    cost = np.concatenate([np.array(ADV_COST, dtype=np.uint16).view(np.float16),
                           (rng.random(65536) * 8.0).astype(np.float16)])
    want = c_oracle.fma_f16(dh, cost).view(np.uint16)
    a = torch_mod.from_numpy(dh).cuda()
    c = torch_mod.from_numpy(cost).cuda()
    out = torch_mod.empty_like(a)
    ext.probe_hfma(a, c, out, 0)
    torch_mod.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), want)


def test_config1_golden():
    """64 tiles, K=2, mul1, kernel order: every field bit-exact."""
    g = load_golden("c1_k2_mul1")
    enc = _encoder(K=2, cb=2)
    try:
        bd = enc.encode_batch_detailed(g["tiles"], pre_permute=False)
    finally:
        enc.arena.release()
    _assert_bd_matches(bd, g, slice(None), 2)
    # Upstream's K=2 MSE ceiling (tests/test_upstream_encode_oracle.py:56-65).
    assert np.mean((g["tiles"] - bd.reconstructed_perm.astype(np.float32)) ** 2) < 0.1
    r = bd.results[5]
    assert r.end_state == g["end_state"][5] and r.path_cost == g["path_cost"][5]


@pytest.mark.parametrize("generic", [False, True])
def test_k_sweep_golden(generic):
    """K=1..8 x 3 codebooks x both tile orders (tests/test_xpu_quantizer.py:88-115)."""
    g = load_golden("k_sweep")
    for K in range(1, 9):
        for cb in (0, 1, 2):
            enc = _encoder(K=K, cb=cb, force_global_costs=generic)
            try:
                for pp in (False, True):
                    sel = (g["K"] == K) & (g["cb"] == cb) & (g["pre_permute"] == pp)
                    print(f"K={K} cb={cb} pre_permute={pp} generic={generic}", flush=True)
                    bd = enc.encode_batch_detailed(g["tiles"][sel], pre_permute=pp)
                    _assert_bd_matches(bd, g, sel, K)
            finally:
                enc.arena.release()


@pytest.mark.parametrize("name", ["heavy_tail", "edge_cases", "l160"])
def test_other_golden_sets(name):
    """Heavy tails at K=2..6, the edge cases of tests/test_xpu_quantizer.py:160-204
    (zeros, constant, outliers, alternating, overflow, +inf, subnormals) and L=160."""
    g = load_golden(name)
    n = g["tiles"].shape[0]
    Ks = np.atleast_1d(g["K"])
    pps = np.atleast_1d(g["pre_permute"])
    L = int(g["L"])
    for K in np.unique(Ks):
        for pp in np.unique(pps):
            sel = (Ks == K if Ks.size == n else np.ones(n, bool)) & \
                  (pps == pp if pps.size == n else np.ones(n, bool))
            if not sel.any():
                continue
            print(f"{name} K={K} pre_permute={pp}", flush=True)
            enc = _encoder(K=int(K), cb=int(g["cb"]), tile_len=L)
            try:
                bd = enc.encode_batch_detailed(g["tiles"][sel], pre_permute=bool(pp))
            finally:
                enc.arena.release()
            np.testing.assert_array_equal(bd.output_indices, g["output_indices"][sel])
            np.testing.assert_array_equal(bd.end_states, g["end_state"][sel])
            np.testing.assert_array_equal(bd.path_costs.astype(np.float64), g["path_cost"][sel])
            with np.errstate(invalid="ignore"):
                np.testing.assert_array_equal(bd.distortions.astype(np.float64),
                                              g["distortion"][sel])
            if L == 256:
                np.testing.assert_array_equal(bd.packed, g["packed"][sel][:, :16 * int(K)])


@pytest.mark.parametrize("K", [1, 5, 6, 7, 8])
def test_l160_against_oracle(K):
    """L = 160 at the bitrates the golden set (K = 2, 3, 4) leaves out: the
    stored-row count, the header's place (one row at every K for L = 160,
    where K = 8's 512-byte rows need two at L = 256) and the ring walk,
    against the C oracle, through both traceback kernels."""
    from exl3_intel_arc_quantizer_amd import _native
    rng = np.random.default_rng(160 + K)
    tiles = rng.normal(0.0, 1.0, size=(5, 160)).astype(np.float32)
    tiles[2] *= 3.0
    ref = c_oracle.encode_tiles(tiles, K=K, cb=2, pre_permute=False)
    prev = _native.set_traceback_policy("auto")
    try:
        for policy in ("rows", "stream"):
            _native.set_traceback_policy(policy)
            print(f"L=160 K={K} traceback={policy}", flush=True)
            enc = _encoder(K=K, cb=2, tile_len=160)
            try:
                bd = enc.encode_batch_detailed(tiles, pre_permute=False)
            finally:
                enc.arena.release()
            np.testing.assert_array_equal(bd.output_indices, ref.output_indices, err_msg=policy)
            np.testing.assert_array_equal(bd.end_states, ref.end_state, err_msg=policy)
            np.testing.assert_array_equal(bd.path_costs, ref.path_cost, err_msg=policy)
            np.testing.assert_array_equal(bd.reconstructed_perm, ref.reconstructed_perm,
                                          err_msg=policy)
    finally:
        _native.set_traceback_policy(prev)


def _check_stored_rows(block, tile16, K, roll, pre):
    """One tile's scratch block against the C oracle's forward pass: every
    stored cost row (the step after every stride-th step, at the positions
    exl3_cost_row_slot reports) and the header (pre_state, the fp16
    inputs in ring order)."""
    from exl3_intel_arc_quantizer_amd._native import load_library
    from exl3_intel_arc_quantizer_amd.scratch_estimator import row_stride, tile_rows
    E = 65536 >> K
    _, _, want_rows = c_oracle.forward_pass(tile16, K=K, cb=2, roll=roll, pre_state=pre,
                                            with_rows=True)
    lib = load_library()
    pos = np.array([lib.exl3_cost_row_slot(K, e) for e in range(E)], dtype=np.int64)
    stride = row_stride(K)
    stored = 254 // stride + 1
    assert block.shape[0] == tile_rows(K) and block.shape[1] == 2 * E
    for r in range(0, 255, stride):
        got = block[r // stride].view(np.uint16)
        np.testing.assert_array_equal(got[pos], want_rows[r], err_msg=f"K={K} row {r}")
    hdr = block[stored:].reshape(-1)
    np.testing.assert_array_equal(hdr[16:16 + 512].view(np.uint16), tile16.view(np.uint16))
    assert int(hdr[8:12].view(np.int32)[0]) == pre


@pytest.mark.parametrize("generic", [False, True])
def test_forward_pass_pins(ext, torch_mod, generic):
    """Split forward pass (quantize_xpu.cpp:169-215) against the reference's
    forward(): terminal costs bit-exact; every stored cost row (every
    stride-th step, group-major positions) against the C oracle's per-step
    costs; the header's inputs and pre_state. Then the split backward pass,
    which rebuilds the unstored steps, reaches the reference's end state."""
    from exl3_intel_arc_quantizer_amd._native import edges_shape
    g = load_golden("forward_pass")
    for i in range(4):
        K, roll, pre, best, end = (int(v) for v in g[f"case{i}_meta"])
        print(f"forward case {i}: K={K} roll={roll} pre={pre} generic={generic}", flush=True)
        tile16 = g[f"case{i}_tile"].view(np.float16)
        x = torch_mod.from_numpy(tile16.astype(np.float32)).cuda().reshape(1, 256)
        E = 65536 >> K
        costs = torch_mod.zeros((1, 2, E), dtype=torch_mod.float16, device="cuda")
        edges = torch_mod.zeros(edges_shape(1, K), dtype=torch_mod.uint8, device="cuda")
        pre_t = torch_mod.full((1,), pre, dtype=torch_mod.int32, device="cuda")
        ext.quantize_tiles_forward_pass(x, costs, edges, pre_t, K, False, True, roll, 1, 32,
                                        generic)
        ends = torch_mod.zeros((1,), dtype=torch_mod.int32, device="cuda")
        w = torch_mod.zeros((1, 256), dtype=torch_mod.float32, device="cuda")
        idx = torch_mod.zeros((1, 256), dtype=torch_mod.int16, device="cuda")
        ext.quantize_tiles_backward_pass(costs, edges, w, idx, ends, 1, K, False, True, roll, 1,
                                         False)
        torch_mod.cuda.synchronize()
        np.testing.assert_array_equal(costs[0, 1].cpu().numpy().view(np.uint16),
                                      g[f"case{i}_costs"])
        _check_stored_rows(edges[0].cpu().numpy(), tile16, K, roll, pre)
        assert int(ends.item()) == end


@pytest.mark.parametrize("generic", [False, True])
def test_cost_rows_k8(ext, torch_mod, generic):
    """K = 8 stores its cost row after every step (512 bytes) and a two-row
    header: every row, the terminal costs and the header equal the C
    oracle's forward pass (reference forward(), reference_encoder.py:130-204)
    for an unconstrained and a constrained pass, from the fast kernel and the
    reference-structured one; the split backward pass then reaches the
    oracle's end state."""
    from exl3_intel_arc_quantizer_amd._native import edges_shape
    rng = np.random.default_rng(88)
    tile16 = rng.normal(0.0, 1.1, size=256).astype(np.float16)
    x = torch_mod.from_numpy(tile16.astype(np.float32)).cuda().reshape(1, 256)
    ref = c_oracle.encode_tiles(tile16.astype(np.float32)[None], K=8, cb=2)
    for roll, pre in ((128, -1), (0, 77)):
        print(f"K=8 forward roll={roll} pre={pre} generic={generic}", flush=True)
        costs = torch_mod.zeros((1, 2, 256), dtype=torch_mod.float16, device="cuda")
        edges = torch_mod.zeros(edges_shape(1, 8), dtype=torch_mod.uint8, device="cuda")
        pre_t = torch_mod.full((1,), pre, dtype=torch_mod.int32, device="cuda")
        ext.quantize_tiles_forward_pass(x, costs, edges, pre_t, 8, False, True, roll, 0, 32,
                                        generic)
        torch_mod.cuda.synchronize()
        _, want_costs = c_oracle.forward_pass(tile16, K=8, cb=2, roll=roll, pre_state=pre)
        np.testing.assert_array_equal(costs[0, 0].cpu().numpy().view(np.uint16),
                                      want_costs.view(np.uint16))
        _check_stored_rows(edges[0].cpu().numpy(), tile16, 8, roll, pre)
        if pre < 0:
            ends = torch_mod.zeros((1,), dtype=torch_mod.int32, device="cuda")
            w = torch_mod.zeros((1, 256), dtype=torch_mod.float32, device="cuda")
            idx = torch_mod.zeros((1, 256), dtype=torch_mod.int16, device="cuda")
            ext.quantize_tiles_backward_pass(costs, edges, w, idx, ends, 1, 8, False, True, roll,
                                             0, False)
            torch_mod.cuda.synchronize()
            assert int(ends.item()) == int(ref.end_state[0])


def test_usm_host_entry_point(ext, torch_mod):
    """quantize_tiles_usm_host (quantize_xpu.cpp:261-300): CPU output tensors,
    [search_s, trace_s] timings, chunks of temp_costs' batch size; states and
    values bit-exact against the C oracle."""
    rng = np.random.default_rng(4242)
    raw = rng.normal(0.0, 1.0, size=(5, 256)).astype(np.float16).astype(np.float32)
    for K in (2, 4):
        print(f"usm_host K={K}", flush=True)
        x = torch_mod.from_numpy(raw).cuda()
        costs = torch_mod.empty((2, 2, 65536 >> K), dtype=torch_mod.float16, device="cuda")
        out_w = torch_mod.zeros((5, 256), dtype=torch_mod.float32)
        out_i = torch_mod.zeros((5, 256), dtype=torch_mod.int16)
        lut = torch_mod.zeros(65536, dtype=torch_mod.float32)
        t = ext.quantize_tiles_usm_host(x, costs, out_w, out_i, lut, K, False, True)
        assert len(t) == 2 and all(v >= 0 for v in t)
        ref = c_oracle.encode_tiles(raw, K=K, cb=2, pre_permute=False)
        np.testing.assert_array_equal(out_i.numpy().view(np.uint16), ref.output_indices)
        np.testing.assert_array_equal(out_w.numpy(), ref.reconstructed_perm.astype(np.float32))
    with pytest.raises(RuntimeError):
        ext.quantize_tiles_usm_host(x, costs, out_w.cuda(), out_i, lut, 4, False, True)


def test_tile_encoder_adapter(torch_mod):
    """make_xpu_tile_encoder (ldlq.py:344-387): (tiles_n, 256) tensor-core
    order tiles in, (reconstruction f32, int16 states) out, on the input's
    device; equal to the C oracle's encode with pre_permute=False."""
    from exl3_intel_arc_quantizer_amd.tile_encoder import make_xpu_tile_encoder
    rng = np.random.default_rng(3131)
    raw = rng.normal(0.0, 0.02, size=(6, 256)).astype(np.float32)
    raw16 = raw.astype(np.float16).astype(np.float32)
    enc = make_xpu_tile_encoder(K=4)
    try:
        assert enc.K == 4 and enc.cb == 2
        ref = c_oracle.encode_tiles(raw16, K=4, cb=2, pre_permute=False)
        # LDLQ hands over unrounded float32 tiles; the encoder rounds to fp16
        # first (xpu_quantizer.py:654-655), as the oracle's raw16 does.
        for tiles in (torch_mod.from_numpy(raw).cuda(), torch_mod.from_numpy(raw)):
            recon, idx = enc(tiles)
            assert recon.device == tiles.device and idx.dtype == torch_mod.int16
            np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint16), ref.output_indices)
            np.testing.assert_array_equal(recon.cpu().numpy(),
                                          ref.reconstructed_perm.astype(np.float32))
    finally:
        enc.encoder.arena.release()


def test_tile_encoder_nan_rejection(torch_mod):
    """NaN tiles are rejected (a documented deviation): at once by
    encode_tensor, and by the asynchronous adapter at check_finite(), which
    also resets its count; the batches queued before it stay valid."""
    from exl3_intel_arc_quantizer_amd.tile_encoder import make_xpu_tile_encoder
    rng = np.random.default_rng(77)
    good = rng.normal(0.0, 1.0, size=(3, 256)).astype(np.float32)
    bad = good.copy()
    bad[1, 17] = np.nan
    ref = c_oracle.encode_tiles(good.astype(np.float16).astype(np.float32), K=3, cb=2,
                                pre_permute=False)
    enc = make_xpu_tile_encoder(K=3)
    try:
        with pytest.raises(ValueError, match="NaN"):
            enc.encoder.encode_tensor(torch_mod.from_numpy(bad).cuda(), finalize=False)
        _, idx_good = enc(torch_mod.from_numpy(good).cuda())
        enc(torch_mod.from_numpy(bad).cuda())           # queued, not checked yet
        _, idx_after = enc(torch_mod.from_numpy(good).cuda())
        with pytest.raises(ValueError, match="1 seen"):
            enc.check_finite()
        enc.check_finite()                               # count was reset
        for idx in (idx_good, idx_after):
            np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint16), ref.output_indices)
        # A CPU input is copied back, so the adapter checks at once.
        with pytest.raises(ValueError, match="NaN"):
            enc(torch_mod.from_numpy(bad))
    finally:
        enc.encoder.arena.release()


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
def test_traceback_kernels_agree(K):
    """The two cost-row tracebacks (per-row tree loads, whole rows streamed
    through LDS) give the oracle's states in both passes, through the fused
    entry point and the split forward / backward entry points."""
    from exl3_intel_arc_quantizer_amd import _native
    rng = np.random.default_rng(600 + K)
    tiles = rng.normal(0.0, 1.0, size=(12, 256)).astype(np.float32)
    tiles[3] *= 4.0
    tiles[7, ::5] = 0.0
    ref = c_oracle.encode_tiles(tiles, K=K, cb=2, pre_permute=True)
    prev = _native.set_traceback_policy("auto")
    try:
        for policy in ("rows", "stream"):
            _native.set_traceback_policy(policy)
            for mode in ("gpu_resident", "gpu_resident_split"):
                print(f"K={K} traceback={policy} mode={mode}", flush=True)
                enc = _encoder(K=K, cb=2)
                try:
                    bd = enc.encode_batch_detailed(tiles, requested_b=12, traceback_mode=mode)
                finally:
                    enc.arena.release()
                np.testing.assert_array_equal(bd.output_indices, ref.output_indices,
                                              err_msg=f"{policy} {mode}")
                np.testing.assert_array_equal(bd.end_states, ref.end_state,
                                              err_msg=f"{policy} {mode}")
    finally:
        _native.set_traceback_policy(prev)


def test_per_call_traceback_choice_threads():
    """exl3_quantize_tiles_tb: every per-call traceback choice gives the
    oracle's states; two threads encoding at once on two streams with
    different choices both do, and neither changes the process default."""
    import threading

    import torch

    from exl3_intel_arc_quantizer_amd import _native
    from exl3_intel_arc_quantizer_amd._native import QuantizeExtension, edges_shape
    K = 4
    rng = np.random.default_rng(777)
    tiles = rng.normal(0.0, 1.0, size=(64, 256)).astype(np.float32)
    ref = c_oracle.encode_tiles(tiles, K=K, cb=2, pre_permute=False)
    x = torch.from_numpy(tiles.astype(np.float16).astype(np.float32)).cuda()
    ext = QuantizeExtension()

    def encode(policy, out, stream):
        with torch.cuda.stream(stream):
            costs = torch.empty((64, 2, 65536 >> K), dtype=torch.float16, device="cuda")
            edges = torch.empty(edges_shape(64, K), dtype=torch.uint8, device="cuda")
            w = torch.empty((64, 256), dtype=torch.float32, device="cuda")
            i = torch.empty((64, 256), dtype=torch.int16, device="cuda")
            for _ in range(4):
                ext.quantize_tiles(x, w, i, costs, edges, K, False, True,
                                   traceback_policy=policy)
            stream.synchronize()
            out[policy] = i.cpu().numpy().view(np.uint16)

    prev = _native.set_traceback_policy("auto")
    try:
        out = {}
        for policy in (None, "auto", "rows", "stream"):
            print(f"per-call traceback={policy}", flush=True)
            encode(policy, out, torch.cuda.current_stream())
            np.testing.assert_array_equal(out[policy], ref.output_indices, err_msg=str(policy))
        print("two threads: rows and stream", flush=True)
        out = {}
        threads = [threading.Thread(target=encode, args=(p, out, torch.cuda.Stream()))
                   for p in ("rows", "stream")]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        for policy in ("rows", "stream"):
            np.testing.assert_array_equal(out[policy], ref.output_indices, err_msg=policy)
        assert _native.set_traceback_policy("auto") == "auto"
    finally:
        _native.set_traceback_policy(prev)


def test_traceback_modes_and_variants_agree():
    """tests/test_xpu_quantizer.py:299-330."""
    rng = np.random.default_rng(909)
    tiles = rng.normal(0.0, 1.1, size=(4, 256)).astype(np.float32)
    ref = c_oracle.encode_tiles(tiles, K=2, cb=2, pre_permute=True)
    for mode in ("gpu_resident", "gpu_resident_split", "d2h_cpu", "usm_host"):
        enc = _encoder(K=2, cb=2)
        try:
            bd = enc.encode_batch_detailed(tiles, requested_b=4, traceback_mode=mode)
        finally:
            enc.arena.release()
        np.testing.assert_array_equal(bd.output_indices, ref.output_indices, err_msg=mode)
    for sg in (16, 32):
        for fg in (False, True):
            enc = _encoder(K=2, cb=2, sg_size=sg, force_global_costs=fg)
            try:
                bd = enc.encode_batch_detailed(tiles, requested_b=4)
            finally:
                enc.arena.release()
            np.testing.assert_array_equal(bd.output_indices, ref.output_indices)


def test_batches_partial_chunks_and_waves():
    """tests/test_xpu_quantizer.py:206-235: 19 tiles, B=6, wave cap 4."""
    rng = np.random.default_rng(555)
    tiles = rng.normal(0.0, 1.0, size=(19, 256)).astype(np.float32)
    ref = c_oracle.encode_tiles(tiles, K=3, cb=2, pre_permute=True)
    for mode in ("gpu_resident", "gpu_resident_split"):
        enc = _encoder(K=3, cb=2, wave_cap_override=4)
        try:
            bd = enc.encode_batch_detailed(tiles, requested_b=6, traceback_mode=mode)
        finally:
            enc.arena.release()
        assert bd.admitted_b == 6 and bd.num_chunks == 4 and len(bd.results) == 19
        np.testing.assert_array_equal(bd.output_indices, ref.output_indices)
        for t in range(19):
            np.testing.assert_array_equal(decode_states(bd.results[t].packed, 3),
                                          bd.output_indices[t])


def test_queue_ordering_and_async(ext, torch_mod):
    """tests/test_xpu_quantizer.py:271-297: torch ops before/after the encoder
    on the same stream, no host sync in between."""
    rng = np.random.default_rng(808)
    raw = rng.normal(0.0, 0.5, size=(4, 256)).astype(np.float16).astype(np.float32)
    from exl3_intel_arc_quantizer_amd._native import edges_shape
    in_t = torch_mod.from_numpy(raw).cuda()
    in_t.mul_(2.0)
    out_w = torch_mod.empty_like(in_t)
    out_i = torch_mod.empty((4, 256), dtype=torch_mod.int16, device="cuda")
    costs = torch_mod.empty((4, 2, 8192), dtype=torch_mod.float16, device="cuda")
    edges = torch_mod.empty(edges_shape(4, 3), dtype=torch_mod.uint8, device="cuda")
    ext.quantize_tiles(in_t, out_w, out_i, costs, edges, 3, False, True)
    out_w.add_(1.0)
    torch_mod.cuda.synchronize()
    ref = c_oracle.encode_tiles(raw * 2.0, K=3, cb=2, pre_permute=False)
    np.testing.assert_array_equal(out_i.cpu().numpy().view(np.uint16), ref.output_indices)
    np.testing.assert_allclose(out_w.cpu().numpy(),
                               ref.reconstructed_perm.astype(np.float32) + 1.0, atol=1e-5)


def test_extension_rejects_malformed_tensors(ext, torch_mod):
    """tests/test_xpu_quantizer.py:260-269."""
    from exl3_intel_arc_quantizer_amd._native import edges_shape
    in_t = torch_mod.zeros((1, 256), dtype=torch_mod.float32, device="cuda")
    out_w = torch_mod.zeros((1, 256), dtype=torch_mod.float32, device="cuda")
    out_i = torch_mod.zeros((1, 256), dtype=torch_mod.int16, device="cuda")
    costs = torch_mod.zeros((1, 2, 16384), dtype=torch_mod.float16, device="cuda")
    edges = torch_mod.zeros(edges_shape(1, 2), dtype=torch_mod.uint8, device="cuda")
    with pytest.raises(RuntimeError):
        ext.quantize_tiles(in_t, out_w, out_i, costs, edges, 2, True, True)
    with pytest.raises(RuntimeError):
        ext.quantize_tiles(in_t.cpu(), out_w, out_i, costs, edges, 2, False, True)
    with pytest.raises(RuntimeError):
        ext.quantize_tiles(in_t, out_w, out_i, costs, edges[:, :-1], 2, False, True)
    with pytest.raises(RuntimeError):
        ext.quantize_tiles(in_t, out_w, out_i.float(), costs, edges, 2, False, True)


def test_helper_wrappers_reject_short_buffers(ext, torch_mod):
    """The device-side helpers check every buffer the kernel indexes by the
    launch's sizes (shape and device) and raise before launching."""
    torch = torch_mod
    dev = "cuda"
    n, L, K = 4, 256, 3
    x = torch.zeros((n, L), dtype=torch.float32, device=dev)
    i16 = lambda *s: torch.zeros(s, dtype=torch.int16, device=dev)  # noqa: E731
    f32 = lambda *s: torch.zeros(s, dtype=torch.float32, device=dev)  # noqa: E731
    with pytest.raises(RuntimeError, match="out"):
        ext.prepare_tiles(x, f32(n - 1, L), False)
    good = dict(out_w=f32(n, L), out_idx=i16(n, L), packed=i16(n, 16 * K), path_cost=f32(n),
                distortion=f32(n), recon_orig=i16(n, L))
    for name, bad in (("path_cost", f32(n - 1)), ("distortion", f32(1)),
                      ("recon_orig", i16(n, L - 1)), ("out_w", f32(n - 1, L)),
                      ("packed", i16(n, 16 * K - 1))):
        args = dict(good, **{name: bad})
        with pytest.raises(RuntimeError, match=name):
            ext.finalize_tiles(x, x, args["out_w"], args["out_idx"], args["packed"],
                               args["path_cost"], args["distortion"], args["recon_orig"], K,
                               False)
    with pytest.raises(RuntimeError, match="raw"):
        ext.finalize_tiles(x, f32(n - 1, L), *[good[k] for k in (
            "out_w", "out_idx", "packed", "path_cost", "distortion", "recon_orig")], K, True)
    with pytest.raises(RuntimeError, match="packed"):
        ext.pack_trellis(i16(n, 256), i16(n - 1, 16 * K), K)
    with pytest.raises(RuntimeError, match="states"):
        ext.unpack_trellis(i16(n, 16 * K), i16(n, 255), K)
    h = torch.zeros(8, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="out"):
        ext.probe_hfma(h, h, h[:7], 0)
    torch.cuda.synchronize()


def test_config2_subsample_vs_c_oracle(torch_mod):
    """Config 2: a 1024x1024 N(0,1) fp16 matrix, tiles formed as ldlq.py:276-281
    (16-row blocks, tensor-core permuted), K=4; a 256-tile subsample (every
    16th tile) bit-exact against the C oracle, as configs[1] asks."""
    rng = np.random.default_rng(1)
    W = rng.standard_normal((1024, 1024), dtype=np.float32).astype(np.float16).astype(np.float32)
    tiles = W.reshape(64, 16, 64, 16).transpose(0, 2, 1, 3).reshape(4096, 256)
    enc = _encoder(K=4, cb=2)
    try:
        bd = enc.encode_batch_detailed(tiles, pre_permute=True, build_results=False)
    finally:
        enc.arena.release()
    sub = np.arange(0, 4096, 16)
    assert sub.size == 256
    ref = c_oracle.encode_tiles(tiles[sub], K=4, cb=2, pre_permute=True)
    np.testing.assert_array_equal(bd.output_indices[sub], ref.output_indices)
    np.testing.assert_array_equal(bd.packed[sub], ref.packed)
    np.testing.assert_array_equal(bd.distortions[sub], ref.distortion)
    np.testing.assert_array_equal(bd.path_costs[sub], ref.path_cost)
    np.testing.assert_array_equal(bd.reconstructed_tiles[sub].view(np.uint16),
                                  ref.reconstructed.view(np.uint16))


# Upstream's MSE ceilings for unit-variance tiles (tests/test_upstream_encode_oracle.py:56-65).
MSE_CEILING = {1: 0.3, 2: 0.1, 3: 0.1, 4: 0.1, 5: 0.1, 6: 0.07, 7: 0.05, 8: 0.04}


def _path_costs(x16, idx, lut):
    """Sequential fp16 cost along each tile's chosen path in ring order
    (xpu_quantizer.py:933-941): c = fma16(dh, dh, c), dh = fp16(lut[s] - w),
    starting from 0; one C-oracle FMA (single rounding) per step."""
    c = np.zeros(idx.shape[0], np.float16)
    for i in range(idx.shape[1]):
        dh = (lut[idx[:, i]] - x16[:, i]).astype(np.float16)
        c = c_oracle.fma_f16(dh, c)
    return c.astype(np.float32)


def _check_batch_invariants(x, bd, K, pre_permute, oracle_rows):
    """Size-independent properties of an encoded batch of unit-scale tiles
    (codebook MUL1): ring continuity and tail biting, recon == lut[idx], the
    packing round trip on a sample, every path cost recomputed along its
    path, every distortion recomputed in numpy's order, the upstream MSE
    ceiling scaled by the batch's variance; ``oracle_rows`` bit-exact
    against the C oracle."""
    n = x.shape[0]
    idx = bd.output_indices.astype(np.int64)
    mask = (65536 >> K) - 1
    np.testing.assert_array_equal(idx & mask, np.roll(idx, -1, axis=1) >> K)
    np.testing.assert_array_equal(bd.end_states, idx[:, 255] & mask)
    lut = oracle_lut(2)
    np.testing.assert_array_equal(bd.reconstructed_perm.view(np.uint16), lut[idx].view(np.uint16))
    for t in range(0, n, 1021):
        np.testing.assert_array_equal(decode_states(bd.packed[t], K), idx[t])
    assert np.all(np.isfinite(bd.path_costs)) and np.all(bd.path_costs > 0)
    # The encoder sees the tiles in kernel order: permuted when pre_permute.
    xk = x[:, oracle_tc_perm()] if pre_permute else x
    x16 = xk.astype(np.float16)
    np.testing.assert_array_equal(bd.path_costs, _path_costs(x16, idx, lut))
    # Distortion over the tile in its original order (reconstructed_tiles).
    rec = bd.reconstructed_tiles.astype(np.float32)
    np.testing.assert_array_equal(bd.distortions, np.sum((x - rec) ** 2, axis=1))
    mse = float(bd.distortions.mean()) / 256.0
    var = float(x.astype(np.float64).var())
    print(f"K={K}: {n} tiles, MSE {mse:.5f}, variance {var:.4f}, "
          f"ceiling {MSE_CEILING[K] * var:.5f}", flush=True)
    assert mse < MSE_CEILING[K] * var
    ref = c_oracle.encode_tiles(x[oracle_rows], K=K, cb=2, pre_permute=pre_permute)
    np.testing.assert_array_equal(bd.output_indices[oracle_rows], ref.output_indices)
    np.testing.assert_array_equal(bd.path_costs[oracle_rows], ref.path_cost)


@pytest.mark.parametrize("K", [2, 3, 4, 5, 6])
def test_configs2_full_matrix(K):
    """configs[2] at its full size: the 65,536 tiles of the seed-2 heavy-tailed
    4096 x 4096 matrix (tests/layer_configs.configs2_tiles, the matrix
    bench.py's sweep times) at the sweep's K = 2..6, every tile checked by
    the size-independent properties and 8 tiles bit-exact against the C
    oracle."""
    from .layer_configs import configs2_tiles
    x = configs2_tiles()
    enc = _encoder(K=K, cb=2)
    try:
        bd = enc.encode_batch_detailed(x, pre_permute=True, build_results=False)
    finally:
        enc.arena.release()
    _check_batch_invariants(x, bd, K, True, np.arange(0, 65536, 8192) + K)


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
def test_large_batch_invariants(K):
    """Config-3-style heavy-tailed tiles at scale: size-independent properties
    over 8192 tiles (ring continuity, tail biting, recon == lut[idx],
    packing round trip, every path cost recomputed along its path, every
    distortion recomputed in numpy's order, the upstream MSE ceiling scaled
    by the batch's variance), plus 16 tiles bit-exact. At K = 1 these
    launches take the in-place forward kernel (more tiles than CUs); the
    golden tests cover its ping-pong form."""
    rng = np.random.default_rng(2 + K)
    x = rng.standard_normal((8192, 256), dtype=np.float32)
    x = np.where(rng.random(x.shape) < 0.01, 4.0 * x, x).astype(np.float16).astype(np.float32)
    enc = _encoder(K=K, cb=2)
    try:
        bd = enc.encode_batch_detailed(x, pre_permute=False, build_results=False)
    finally:
        enc.arena.release()
    _check_batch_invariants(x, bd, K, False, np.arange(0, 8192, 512))
