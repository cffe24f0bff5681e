"""On-disk trellis format and the global-scale search on the GPU:
pack / unpack kernels against the oracle's pack_trellis / swap16 /
decode_states (trellis_format.py:120-213), the safetensors export and reload
(serialization.py), and the global-scale search (gss.py) against its numpy
oracle driven by the C trellis oracle."""

from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import gss_ref, ldlq_ref
from oracle.trellis_format_ref import decode_states, decode_tile_values, pack_trellis, \
    swap16_storage

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _paths(n, K, seed):
    """n valid trellis tiles: state t is the 16-bit window of a random
    symbol stream ending at bit (t + 1) K, circular."""
    rng = np.random.default_rng(seed)
    nb = 256 * K
    idx = ((np.arange(256)[:, None] + 1) * K - 16 + np.arange(16)[None, :]) % nb
    out = np.empty((n, 256), np.uint16)
    for i in range(n):
        sym = rng.integers(0, 1 << K, 256)
        bits = ((sym[:, None] >> np.arange(K - 1, -1, -1)) & 1).reshape(-1)
        out[i] = (bits[idx] << np.arange(15, -1, -1)).sum(axis=1)
    return out


@pytest.mark.parametrize("K", range(1, 9))
def test_pack_unpack_module_trellis(torch_mod, K):
    from exl3_intel_arc_quantizer_amd.serialization import pack_module_trellis, \
        unpack_module_trellis
    torch = torch_mod
    states = _paths(15, K, 40 + K)
    enc = torch.from_numpy(states.view(np.int16).reshape(3, 5, 256)).cuda()
    packed = pack_module_trellis(enc, K)
    assert packed.shape == (3, 5, 16 * K) and packed.dtype == torch.int16
    want = np.stack([swap16_storage(pack_trellis(s, K)) for s in states])
    np.testing.assert_array_equal(packed.cpu().numpy().view(np.uint16).reshape(15, -1), want)
    back = unpack_module_trellis(packed, K)
    np.testing.assert_array_equal(back.cpu().numpy().view(np.uint16).reshape(15, 256), states)
    # Arbitrary words (not a trellis path) decode as the reference reads them.
    words = np.random.default_rng(K).integers(0, 65536, (6, 16 * K)).astype(np.uint16)
    got = unpack_module_trellis(torch.from_numpy(words.view(np.int16).reshape(2, 3, -1)).cuda(), K)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16).reshape(6, 256),
                                  np.stack([decode_states(w, K) for w in words]).astype(np.uint16))
    # Host tensors go through the same kernels and come back on the host.
    assert pack_module_trellis(enc.cpu(), K).device.type == "cpu"


def test_export_and_reload_layer(torch_mod, tmp_path):
    from exl3_intel_arc_quantizer_amd.layer_quant import hessian_from_activations, \
        quantize_linear_module
    from exl3_intel_arc_quantizer_amd.serialization import decode_weight_from_storage, \
        export_layer_safetensors, load_and_verify_layer_safetensors
    torch = torch_mod
    rng = np.random.default_rng(8)
    W = torch.from_numpy((rng.standard_normal((384, 256)) * 0.02).astype(np.float32)).cuda()
    X = torch.from_numpy(rng.standard_normal((1024, 256)).astype(np.float32)).cuda()
    H, _ = hessian_from_activations(X)
    res = quantize_linear_module("mlp.up_proj", W, H, K=3)
    st, qc = export_layer_safetensors({"mlp.up_proj": res}, tmp_path, layer_idx=2)
    from safetensors import safe_open
    with safe_open(str(st), framework="pt") as f:
        keys = set(f.keys())
        trellis = f.get_tensor("model.layers.2.mlp.up_proj.trellis")
        suh = f.get_tensor("model.layers.2.mlp.up_proj.suh")
        svh = f.get_tensor("model.layers.2.mlp.up_proj.svh")
        meta = f.metadata()
    assert keys == {f"model.layers.2.mlp.up_proj.{s}" for s in ("trellis", "suh", "svh", "mul1")}
    assert trellis.shape == (16, 24, 48) and trellis.dtype == torch.int16
    assert suh.dtype == torch.float16 and suh.shape == (256,) and svh.shape == (384,)
    assert meta["quant_format"] == "exl3" and meta["bits"] == "3"
    cfg = json.loads(qc.read_text())
    assert cfg["tensor_storage"]["model.layers.2.mlp.up_proj"]["bits_per_weight"] == 3
    index = json.loads((tmp_path / "model.safetensors.index.json").read_text())
    assert set(index["weight_map"]) == keys
    # Reload: decoded weights equal w_hat up to the fp16 rounding of the scales.
    dec = load_and_verify_layer_safetensors(st, {"mlp.up_proj": res}, atol=5e-3)
    w_dec = dec["model.layers.2.mlp.up_proj"]
    # And equal the oracle's decode of the same stored tensors.
    t = trellis.numpy().view(np.uint16).reshape(16 * 24, 48)
    tiles = np.stack([decode_tile_values(x, 3).astype(np.float32) for x in t])
    w_hat = tiles.reshape(16, 24, 16, 16).transpose(0, 2, 1, 3).reshape(256, 384)
    want = ldlq_ref.weight_from_quantized(w_hat, suh.float().numpy()[:, None],
                                          svh.float().numpy()[None, :])
    np.testing.assert_allclose(w_dec.numpy(), want, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(
        decode_weight_from_storage(trellis.cuda(), suh.cuda(), svh.cuda(), 3).cpu().numpy(),
        w_dec.numpy(), rtol=0, atol=0)


def test_linear_module_codebook_choice(torch_mod, tmp_path):
    """cb reaches the encoder: an MCG module's stored tensors carry the mcg
    marker and decode with the MCG table to w_hat; an encoder of another
    codebook is refused (its states would be labelled wrongly)."""
    from exl3_intel_arc_quantizer_amd.layer_quant import hessian_from_activations, \
        quantize_linear_module
    from exl3_intel_arc_quantizer_amd.serialization import export_layer_safetensors, \
        load_and_verify_layer_safetensors
    from exl3_intel_arc_quantizer_amd.tile_encoder import make_xpu_tile_encoder
    from exl3_intel_arc_quantizer_amd.trellis_format import CB_MCG, CB_MUL1
    torch = torch_mod
    rng = np.random.default_rng(12)
    W = torch.from_numpy((rng.standard_normal((256, 128)) * 0.02).astype(np.float32)).cuda()
    X = torch.from_numpy(rng.standard_normal((512, 128)).astype(np.float32)).cuda()
    H, _ = hessian_from_activations(X)
    res = quantize_linear_module("mlp.gate_proj", W, H, K=2, cb=CB_MCG)
    assert res.cb == CB_MCG
    st, _ = export_layer_safetensors({"mlp.gate_proj": res}, tmp_path, layer_idx=0)
    from safetensors import safe_open
    with safe_open(str(st), framework="pt") as f:
        assert "model.layers.0.mlp.gate_proj.mcg" in set(f.keys())
        assert f.metadata()["codebook"] == "mcg"
    load_and_verify_layer_safetensors(st, {"mlp.gate_proj": res}, atol=5e-3)
    enc = make_xpu_tile_encoder(K=2)
    try:
        with pytest.raises(ValueError, match="cb"):
            quantize_linear_module("q", W, H, K=2, cb=CB_MCG, tile_encoder=enc)
        assert enc.cb == CB_MUL1
    finally:
        enc.encoder.arena.release()


def _hip_encoder(K):
    from exl3_intel_arc_quantizer_amd.tile_encoder import make_xpu_tile_encoder
    return make_xpu_tile_encoder(K=K)


def test_gss_matches_oracle_with_c_encoder(torch_mod):
    """gss.py on the HIP encoder against the numpy search on the C oracle:
    the encoders agree bit for bit, so scale and MSE agree to float
    rounding of the MSE sums."""
    from exl3_intel_arc_quantizer_amd.gss import g_scale_gss
    w = (np.random.default_rng(9).standard_normal((128, 128)) * 0.7).astype(np.float32)
    enc = _hip_encoder(2)
    try:
        scale, mse = g_scale_gss(torch_mod.from_numpy(w).cuda(), enc, width=1)
    finally:
        enc.encoder.arena.release()
    print("gss oracle search (C encoder, ~200 tiles)", flush=True)
    (ws, wm), = gss_ref.g_scale_search([gss_ref.sample_scale_tiles(w, 1)],
                                       ldlq_ref.c_oracle_encoder(2))
    assert scale == pytest.approx(ws, abs=1e-6)
    assert mse == pytest.approx(wm, rel=1e-5)


def test_gss_search_properties(torch_mod):
    """tests/test_gss.py:263-332 of the reference on the HIP encoder."""
    from exl3_intel_arc_quantizer_amd.gss import COARSE_POINTS, COARSE_START, COARSE_STEP, \
        FINE_STEP, g_scale_gss, g_scale_search_batch, sample_scale_tiles
    torch = torch_mod
    rng = np.random.default_rng(10)
    weight = torch.from_numpy(rng.standard_normal((256, 256)).astype(np.float32)).cuda()
    enc = _hip_encoder(2)

    def mse_at(tiles, s):
        recon, _ = enc(tiles * s)
        return float((recon / s - tiles).square().mean())

    try:
        tiles = sample_scale_tiles(weight)
        coarse = [COARSE_START + COARSE_STEP * i for i in range(COARSE_POINTS)]
        curve = [mse_at(tiles[::3], s) for s in coarse]
        centre = coarse[int(np.argmin(curve))]
        fine = [centre + FINE_STEP * (i - 2) for i in range(5)]
        fine_curve = [mse_at(tiles, s) for s in fine]
        best = int(np.argmin(fine_curve))
        scale, mse = g_scale_gss(weight, enc)
        assert mse == pytest.approx(fine_curve[best], abs=1e-6)
        assert max(0.01, fine[best] - FINE_STEP / 2) <= scale <= fine[best] + FINE_STEP / 2 + 1e-9
        assert mse < mse_at(tiles, 1.0)
        assert g_scale_gss(weight, enc) == (scale, mse)
        other = sample_scale_tiles(weight[:128] * 3.0)
        both = g_scale_search_batch([tiles, other], enc)
        assert both == g_scale_search_batch([tiles, other], enc, max_tiles=300)
        assert both[0] == g_scale_search_batch([tiles], enc)[0]
        huge, _ = g_scale_gss(weight * 50.0, enc)
        assert huge < 0.1
        enc.check_finite()
    finally:
        enc.encoder.arena.release()


def test_linear_module_with_global_scale(torch_mod):
    """quantize_linear_module(skip_g_scale=False): the scale applied is the
    search's result on the regularised weight, su carries 1/g, and the
    encoded layer decodes back to w_hat."""
    from exl3_intel_arc_quantizer_amd.gss import g_scale_gss
    from exl3_intel_arc_quantizer_amd.layer_quant import hessian_from_activations, \
        quantize_linear_module
    from exl3_intel_arc_quantizer_amd.regularize import regularize
    from exl3_intel_arc_quantizer_amd.tile_encoder import make_xpu_tile_encoder
    torch = torch_mod
    rng = np.random.default_rng(11)
    W = torch.from_numpy((rng.standard_normal((256, 256)) * 0.02).astype(np.float32)).cuda()
    X = torch.from_numpy(rng.standard_normal((1024, 256)).astype(np.float32)).cuda()
    H, _ = hessian_from_activations(X)
    enc = make_xpu_tile_encoder(K=3)
    try:
        res = quantize_linear_module("q", W, H, K=3, tile_encoder=enc, skip_g_scale=False)
        plain = regularize(W.T.contiguous(), torch.ones((256, 1), device="cuda"),
                           torch.ones((1, 256), device="cuda"), H_diag=H.diagonal())
        g, _ = g_scale_gss(plain.weight, enc)
    finally:
        enc.encoder.arena.release()
    assert res.metrics.g_scale == g and g != 1.0
    torch.testing.assert_close(res.su, plain.su / g)
    assert np.isfinite(res.metrics.proxy_loss) and res.metrics.normalized_proxy_loss < 0.5
