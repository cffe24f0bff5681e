"""The product's format helpers that run on the host (trellis_format.py:162-202
of the reference: swap16_storage, words_from_storage, stream_from_words,
state_index) against known answers and the oracle's restatement; the
argument checks of the GPU-backed helpers, which fire before any device
call."""

from __future__ import annotations

import numpy as np
import pytest

from exl3_intel_arc_quantizer_amd import trellis_format as tf
from oracle import trellis_format_ref as ref


def test_reference_names_are_exported():
    """Every public name of the reference's trellis_format module
    (trellis_format.py:28-227) imports from the product module."""
    for name in ("CB_3INST", "CB_MCG", "CB_MUL1", "MUL1_MULT", "MCG_MULT", "THREEINST_MULT",
                 "THREEINST_ADD", "codebook_lut", "tensor_core_perm", "tensor_core_perm_inv",
                 "pack_trellis", "swap16_storage", "words_from_storage", "stream_from_words",
                 "state_index", "decode_states", "decode_tile_values"):
        assert hasattr(tf, name), name


def test_swap16_known_answer_and_involution():
    """tests/test_trellis_format.py:163-167 of the reference; applying the
    swap twice is the identity; 2-D batches swap row by row."""
    s = np.array([0x1111, 0x2222, 0x3333, 0x4444], dtype=np.uint16)
    assert tf.swap16_storage(s).tolist() == [0x2222, 0x1111, 0x4444, 0x3333]
    rng = np.random.default_rng(3)
    w = rng.integers(0, 65536, (5, 48)).astype(np.uint16)
    np.testing.assert_array_equal(tf.swap16_storage(tf.swap16_storage(w)), w)
    for row in range(5):
        np.testing.assert_array_equal(tf.swap16_storage(w)[row], ref.swap16_storage(w[row]))
    assert tf.swap16_storage(w.view(np.int16)).dtype == np.uint16
    with pytest.raises(ValueError):
        tf.swap16_storage(np.zeros(3, np.uint16))


def test_swap16_torch_tensor():
    import torch
    w = np.random.default_rng(4).integers(0, 65536, (3, 32)).astype(np.uint16)
    t = torch.from_numpy(w.view(np.int16))
    got = tf.swap16_storage(t)
    assert isinstance(got, torch.Tensor) and got.dtype == torch.int16
    np.testing.assert_array_equal(got.numpy().view(np.uint16), tf.swap16_storage(w))


def test_words_and_stream_known_answers():
    """Word j is t16[2j] | t16[2j+1] << 16, bits most significant first."""
    t16 = np.array([0x0001, 0x8000, 0xFFFF, 0x0000], dtype=np.uint16)
    words = tf.words_from_storage(t16)
    assert words.dtype == np.uint64 and words.tolist() == [0x80000001, 0x0000FFFF]
    bits = tf.stream_from_words(words)
    assert bits.shape == (64,)
    assert bits[0] == 1 and bits[1:31].sum() == 0 and bits[31] == 1
    assert bits[32:48].sum() == 0 and bits[48:].sum() == 16
    rng = np.random.default_rng(5)
    t = rng.integers(0, 65536, 64).astype(np.uint16)
    np.testing.assert_array_equal(tf.words_from_storage(t), ref.words_from_storage(t))
    np.testing.assert_array_equal(tf.stream_from_words(tf.words_from_storage(t)),
                                  ref.stream_from_words(ref.words_from_storage(t)))


@pytest.mark.parametrize("K", range(1, 9))
def test_state_index_windows(K):
    """State t is the 16-bit window ending at bit (t + 1) K, circular
    (tests/test_trellis_format.py:169-179 of the reference)."""
    idx = tf.state_index(K)
    nbits = 256 * K
    assert idx.shape == (256, 16)
    for t in (0, 1, 17, 255):
        np.testing.assert_array_equal(idx[t], np.arange((t + 1) * K - 16, (t + 1) * K) % nbits)
    np.testing.assert_array_equal(idx, ref.state_index(K))


def test_gpu_helpers_validate_before_device_calls():
    with pytest.raises(ValueError):
        tf.pack_trellis(np.zeros(256, np.uint16), 0)
    with pytest.raises(ValueError):
        tf.pack_trellis(np.zeros(255, np.uint16), 2)
    with pytest.raises(ValueError):
        tf.decode_states(np.zeros(31, np.uint16), 2)
    with pytest.raises(ValueError):
        tf.decode_states(np.zeros(32, np.uint16), 9)
