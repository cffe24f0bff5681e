"""The reference's format API and its tie-aware quality check on the GPU:

* trellis_format.pack_trellis (pre-swap words) and swap16_storage, whose
  composition is what a ``.trellis`` tensor stores; decode_states and
  decode_tile_values over the unpacking kernel (trellis_format.py:120-227),
  against the oracle's restatement and the reference's golden packed words;
* verify_tile_encoding_quality (xpu_quantizer.py:108-169) as the reference's
  device test uses it (tests/test_xpu_quantizer.py:160-204): the edge-case
  tiles encoded on the GPU pass against the reference encoder's golden
  results with identical indices, and a ring broken at index 10 is
  rejected with the broken step reported.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import trellis_format_ref as ref

from .conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _golden_result(g, i):
    """The reference encoder's EncodingResult for golden row i."""
    from exl3_intel_arc_quantizer_amd.reference_encoder import EncodingResult
    K = int(g["K"][i])
    return EncodingResult(
        output_indices=g["output_indices"][i].copy(),
        reconstructed=g["reconstructed"][i].view(np.float16).copy(),
        reconstructed_perm=g["reconstructed_perm"][i].view(np.float16).copy(),
        packed=g["packed"][i][:16 * K].copy(),
        end_state=int(g["end_state"][i]), distortion=float(g["distortion"][i]),
        mse=float(g["mse"][i]), path_cost=float(g["path_cost"][i]), K=K, cb=int(g["cb"]))


@pytest.mark.parametrize("K", range(1, 9))
def test_pack_trellis_pre_swap_and_storage(K):
    """pack_trellis returns the reference's pre-swap words; swap16_storage of
    them equals the golden stored words of the reference encoder."""
    from exl3_intel_arc_quantizer_amd import trellis_format as tf
    g = load_golden("k_sweep")
    sel = np.flatnonzero(g["K"] == K)[:6]
    print(f"pack_trellis K={K} tiles {sel.tolist()}", flush=True)
    for i in sel:
        states = g["output_indices"][i]
        pre = tf.pack_trellis(states, K)
        assert pre.dtype == np.uint16 and pre.shape == (16 * K,)
        np.testing.assert_array_equal(pre, ref.pack_trellis(states, K))
        np.testing.assert_array_equal(tf.swap16_storage(pre), g["packed"][i][:16 * K])
    batch = tf.pack_trellis_batch(g["output_indices"][sel], K)
    np.testing.assert_array_equal(batch, g["packed"][sel][:, :16 * K])


@pytest.mark.parametrize("K", range(1, 9))
def test_decode_states_and_tile_values(torch_mod, K):
    """decode_states / decode_tile_values on the GPU equal the oracle's on
    golden stored words (one tile and a batch) and on arbitrary words; the
    device-tensor form returns int16 states on the device."""
    from exl3_intel_arc_quantizer_amd import trellis_format as tf
    g = load_golden("k_sweep")
    sel = np.flatnonzero(g["K"] == K)[:6]
    words = g["packed"][sel][:, :16 * K]
    print(f"decode_states K={K}", flush=True)
    one = tf.decode_states(words[0], K)
    assert one.dtype == np.int64 and one.shape == (256,)
    np.testing.assert_array_equal(one, ref.decode_states(words[0], K))
    np.testing.assert_array_equal(one.astype(np.uint16), g["output_indices"][sel[0]])
    batch = tf.decode_states(words, K)
    np.testing.assert_array_equal(batch.astype(np.uint16), g["output_indices"][sel])
    rnd = np.random.default_rng(60 + K).integers(0, 65536, (5, 16 * K)).astype(np.uint16)
    np.testing.assert_array_equal(tf.decode_states(rnd, K),
                                  np.stack([ref.decode_states(w, K) for w in rnd]))
    dev = tf.decode_states(torch_mod.from_numpy(rnd.view(np.int16)).cuda(), K)
    assert dev.is_cuda and dev.dtype == torch_mod.int16
    np.testing.assert_array_equal(dev.cpu().numpy().view(np.uint16),
                                  tf.decode_states(rnd, K).astype(np.uint16))
    for cb in (0, 1, 2):
        vals = tf.decode_tile_values(words[0], K, cb)
        assert vals.dtype == np.float16
        np.testing.assert_array_equal(vals.view(np.uint16),
                                      ref.decode_tile_values(words[0], K, cb).view(np.uint16))
    # A pre-permuted MUL1 golden tile: the values in original order are the
    # reference encoder's ``reconstructed``.
    j = int(np.flatnonzero((g["K"] == K) & (g["cb"] == 2) & g["pre_permute"])[0])
    np.testing.assert_array_equal(
        tf.decode_tile_values(g["packed"][j][:16 * K], K).view(np.uint16), g["reconstructed"][j])


def test_verify_tile_encoding_quality_edge_cases():
    """tests/test_xpu_quantizer.py:160-204: zeros, constant 0.5, outliers
    25.0 at every 17th position, alternating +-1.5 (and subnormal, ramp) at
    K = 2, 4, 6 in both tile orders: the GPU encoding passes the tie-aware
    check against the reference encoder's result with identical indices."""
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import (XPUTrellisEncoder,
                                                            verify_tile_encoding_quality)
    g = load_golden("edge_cases")
    finite = ("zeros", "constant", "outliers", "alternating", "subnormal", "ramp")
    checked = 0
    for K in (2, 4, 6):
        enc = XPUTrellisEncoder(K=K, cb=2)
        try:
            for i in np.flatnonzero(g["K"] == K):
                name = str(g["name"][i])
                if name not in finite:
                    continue
                pp = bool(g["pre_permute"][i])
                print(f"verify K={K} {name} pre_permute={pp}", flush=True)
                got = enc.encode_tile(g["tiles"][i], pre_permute=pp)
                check = verify_tile_encoding_quality(got, _golden_result(g, i), cost_atol=0.0)
                assert check["passed"], (name, K, pp, check)
                assert check["indices_identical"], (name, K, pp)
                assert check["ring_valid"] and check["broken_step"] == -1
                assert check["cost_diff"] == 0.0 and check["distortion_rel_diff"] == 0.0
                checked += 1
        finally:
            enc.arena.release()
    assert checked == 3 * 2 * len(finite)


def test_verify_tile_encoding_quality_rejects_broken_results():
    """A ring broken at index 10 fails with ring_valid False and broken_step
    10 (tests/test_xpu_quantizer.py:187-202); a reconstruction that is not
    the codebook value of its state, a wrong end state and a different path
    cost each fail the check too."""
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import (XPUTrellisEncoder,
                                                            verify_tile_encoding_quality)
    from exl3_intel_arc_quantizer_amd.reference_encoder import EncodingResult
    g = load_golden("edge_cases")
    i = int(np.flatnonzero((g["K"] == 2) & (g["name"] == "alternating") & g["pre_permute"])[0])
    ref_res = _golden_result(g, i)
    enc = XPUTrellisEncoder(K=2, cb=2)
    try:
        got = enc.encode_tile(g["tiles"][i])
        lut = enc.lut
    finally:
        enc.arena.release()

    def copy(r, **kw):
        fields = dict(output_indices=r.output_indices.copy(), reconstructed=r.reconstructed.copy(),
                      reconstructed_perm=r.reconstructed_perm.copy(), packed=r.packed.copy(),
                      end_state=r.end_state, distortion=r.distortion, mse=r.mse,
                      path_cost=r.path_cost, K=r.K, cb=r.cb)
        fields.update(kw)
        return EncodingResult(**fields)

    broken = copy(got)
    broken.output_indices[10] ^= 1
    broken.reconstructed_perm[10] = lut[broken.output_indices[10]]
    bad = verify_tile_encoding_quality(broken, ref_res)
    assert not bad["passed"] and not bad["ring_valid"] and bad["broken_step"] == 10
    assert bad["rec_exact"] and not bad["indices_identical"]

    wrong_rec = copy(got)
    wrong_rec.reconstructed_perm[3] = np.float16(float(wrong_rec.reconstructed_perm[3]) + 0.5)
    chk = verify_tile_encoding_quality(wrong_rec, ref_res)
    assert not chk["passed"] and not chk["rec_exact"] and chk["ring_valid"]

    wrong_end = copy(got, end_state=(got.end_state + 1) % (65536 >> 2))
    chk = verify_tile_encoding_quality(wrong_end, ref_res)
    assert not chk["passed"] and not chk["end_state_valid"]

    wrong_cost = copy(got, path_cost=float(got.path_cost) + 0.25)
    chk = verify_tile_encoding_quality(wrong_cost, ref_res)
    assert not chk["passed"] and chk["cost_diff"] == pytest.approx(0.25)
    assert verify_tile_encoding_quality(wrong_cost, ref_res, cost_atol=0.5)["passed"]
