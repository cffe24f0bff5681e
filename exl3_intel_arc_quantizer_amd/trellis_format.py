"""EXL3 format constants and format helpers (reference: exl3_quant/trellis_format.py).

Every public name of the reference module is here with the reference's
meaning, so code written against it imports this module unchanged:

* ``codebook_lut``: the fp16 value of every 16-bit state, decoded by the
  HIP kernel of ``libexl3_hip.so``;
* ``tensor_core_perm`` / ``tensor_core_perm_inv``: the fixed tile order;
* ``pack_trellis``: one tile's packed words BEFORE the half-word swap
  (trellis_format.py:120-159), and ``swap16_storage`` the swap itself
  (:162-178), so ``swap16_storage(pack_trellis(s, K))`` is what a
  ``.trellis`` tensor stores;
* ``words_from_storage``, ``stream_from_words``, ``state_index``,
  ``decode_states``, ``decode_tile_values``: the read-back side (:181-227).

The bit layouts are fixed by the EXL3 format (upstream exllamav3
codebook.cuh, pack.cu) and are restated here. Packing and decoding run on
the GPU: ``pack_trellis_batch`` and ``decode_states`` over many tiles are
one launch of ``exl3_pack_trellis`` / ``exl3_unpack_trellis`` each, and the
single-tile forms go through the same kernels. The half-word swap, the
word and bit-stream views and the window index table are data movement or
index formulas and are built on the host.
"""

from __future__ import annotations

from typing import Optional

import numpy as np

# Codebook selectors (trellis_format.py:28-33) and the hash constants of the
# procedural codebooks (codebook.cuh:56-123).
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
MUL1_MULT = 0x83DCD12D
MCG_MULT = 0xCBAC1FED
THREEINST_MULT = 89226354
THREEINST_ADD = 64248484

TILE_STATES = 256
_LUT_CACHE: dict = {}


def _check_k(K: int) -> None:
    if not 1 <= int(K) <= 8:
        raise ValueError(f"K must be in 1..8, got {K}")


def tensor_core_perm() -> np.ndarray:
    """Index table of the EXL3 tensor-core tile order (trellis_format.py:88-108).

    Encoded element ``8t + s`` (t < 32, s < 8) is original position
    ``row*16 + col`` with ``row = 2(t%4) + (s%2) + 8*((s//2)%2)`` and
    ``col = t//4 + 8*(s//4)``.
    """
    i = np.arange(256)
    t, s = i // 8, i % 8
    row = 2 * (t % 4) + (s % 2) + 8 * ((s // 2) % 2)
    col = t // 4 + 8 * (s // 4)
    return (row * 16 + col).astype(np.int64)


def tensor_core_perm_inv() -> np.ndarray:
    """Inverse table (trellis_format.py:111-113)."""
    inv = np.empty(256, dtype=np.int64)
    inv[tensor_core_perm()] = np.arange(256)
    return inv


def codebook_lut(cb: int, device_index: Optional[int] = None) -> np.ndarray:
    """fp16 value of every 16-bit state, decoded on the GPU
    (trellis_format.py:41-81; decode_codebook, quantize_kernels.sycl:594-601)."""
    if cb not in (CB_3INST, CB_MCG, CB_MUL1):
        raise ValueError(f"Unknown codebook {cb}")
    import torch

    from ._native import extension

    dev = torch.cuda.current_device() if device_index is None else int(device_index)
    key = (cb, dev)
    if key not in _LUT_CACHE:
        out = torch.empty(65536, dtype=torch.float16, device=f"cuda:{dev}")
        extension().decode_codebook(cb, out)
        _LUT_CACHE[key] = out.cpu().numpy()
    return _LUT_CACHE[key].copy()


# --------------------------------------------------------------- packing

def pack_trellis_batch(states, K: int):
    """``swap16_storage(pack_trellis(s, K))`` for every row of a batch, in
    one launch of the packing kernel: the words a ``.trellis`` tensor
    stores. ``states``: (n, 256) uint16/int16 numpy array or device tensor.
    Returns (n, 16K) words (uint16 numpy for numpy input, an int16 device
    tensor for tensor input)."""
    import torch

    from ._native import extension

    _check_k(K)
    if isinstance(states, torch.Tensor):
        s = states.to(torch.int16).contiguous()
        out = torch.empty((s.shape[0], 16 * K), dtype=torch.int16, device=s.device)
        extension().pack_trellis(s, out, K)
        return out
    arr = np.ascontiguousarray(np.asarray(states, dtype=np.uint16).reshape(-1, TILE_STATES))
    s = torch.from_numpy(arr.view(np.int16)).cuda()
    out = torch.empty((s.shape[0], 16 * K), dtype=torch.int16, device=s.device)
    extension().pack_trellis(s, out, K)
    return out.cpu().numpy().view(np.uint16)


def pack_trellis(states: np.ndarray, K: int) -> np.ndarray:
    """One tile's 256 states packed into ``256 K / 16`` uint16 words BEFORE
    the half-word swap (trellis_format.py:120-159, pack.cu:9-54): 16 spans of
    16 states, each state's low K bits appended most-significant bit first,
    a word emitted whenever 16 bits are buffered. Apply ``swap16_storage``
    to get the stored words."""
    _check_k(K)
    s = np.asarray(states, dtype=np.uint16)
    if s.size != TILE_STATES:
        raise ValueError(f"Expected 256 states per tile, got {s.size}")
    return swap16_storage(pack_trellis_batch(s.reshape(1, TILE_STATES), K)[0])


def swap16_storage(s_packed):
    """Exchange the two 16-bit halves of every 32-bit word (pack.cu:55-56;
    trellis_format.py:162-178): element 2j takes element 2j + 1 and the
    reverse. The operation is its own inverse. Accepts a numpy array (any
    16-bit dtype, returned as uint16) or a torch tensor (returned as a tensor
    of the same dtype and device)."""
    try:
        import torch
        is_tensor = isinstance(s_packed, torch.Tensor)
    except ImportError:  # pragma: no cover
        is_tensor = False
    if is_tensor:
        if s_packed.shape[-1] % 2:
            raise ValueError("swap16_storage needs an even number of 16-bit words")
        return s_packed.reshape(*s_packed.shape[:-1], -1, 2).flip(-1).reshape(s_packed.shape)
    a = np.asarray(s_packed, dtype=np.uint16)
    if a.shape[-1] % 2:
        raise ValueError("swap16_storage needs an even number of 16-bit words")
    return np.ascontiguousarray(a.reshape(*a.shape[:-1], -1, 2)[..., ::-1]).reshape(a.shape)


# -------------------------------------------------------------- read-back

def words_from_storage(t16: np.ndarray) -> np.ndarray:
    """Stored 16-bit words -> the 32-bit words a decoder reads: word j is
    ``t16[2j] | t16[2j+1] << 16`` (trellis_format.py:181-184), as uint64."""
    a = np.asarray(t16, dtype=np.uint16).reshape(-1, 2).astype(np.uint64)
    return a[:, 0] | (a[:, 1] << np.uint64(16))


def stream_from_words(words: np.ndarray) -> np.ndarray:
    """32-bit words -> their bits, most significant first, word after word
    (trellis_format.py:187-190), as uint64 zeros and ones."""
    w = np.asarray(words, dtype=np.uint64).reshape(-1, 1)
    return ((w >> np.arange(31, -1, -1, dtype=np.uint64)) & np.uint64(1)).reshape(-1)


def state_index(K: int) -> np.ndarray:
    """(256, 16) bit positions of each state's window (trellis_format.py:193-202):
    state t is the 16 bits ending at bit (t + 1) K of the tile's 256 K-bit
    stream, wrapping around its start."""
    nbits = TILE_STATES * K
    start = (np.arange(1, TILE_STATES + 1) * K - 16) % nbits
    return (start[:, None] + np.arange(16)[None, :]) % nbits


def decode_states(t16, K: int):
    """Stored words -> 16-bit states (trellis_format.py:205-213), on the GPU.

    ``t16``: one tile's (16K,) stored words, or an (n, 16K) batch, as a numpy
    array (returns int64 (256,) / (n, 256)) or an int16 device tensor
    (returns int16 (n, 256) on the same device). One launch of the unpacking
    kernel for the whole batch."""
    import torch

    from ._native import extension

    _check_k(K)
    if isinstance(t16, torch.Tensor):
        w = t16.to(torch.int16).reshape(-1, 16 * K).contiguous()
        out = torch.empty((w.shape[0], TILE_STATES), dtype=torch.int16, device=w.device)
        extension().unpack_trellis(w, out, K)
        return out
    a = np.asarray(t16, dtype=np.uint16)
    single = a.ndim == 1
    if a.shape[-1] != 16 * K:
        raise ValueError(f"expected {16 * K} stored words per tile at K={K}, got {a.shape[-1]}")
    w = torch.from_numpy(np.ascontiguousarray(a.reshape(-1, 16 * K)).view(np.int16)).cuda()
    out = torch.empty((w.shape[0], TILE_STATES), dtype=torch.int16, device=w.device)
    extension().unpack_trellis(w, out, K)
    states = out.cpu().numpy().view(np.uint16).astype(np.int64)
    return states[0] if single else states


def decode_tile_values(t16, K: int, cb: int = CB_MUL1) -> np.ndarray:
    """Stored words -> the tile's 256 codebook values in original (row-major
    16 x 16) order, fp16 (trellis_format.py:216-227): the states' values
    scattered back through the tensor-core order. Batched like
    ``decode_states`` for numpy input ((n, 16K) -> (n, 256))."""
    states = decode_states(np.asarray(t16), K)
    vals = codebook_lut(cb)[states]
    tile = np.empty(vals.shape, dtype=np.float16)
    tile[..., tensor_core_perm()] = vals
    return tile


__all__ = ["CB_3INST", "CB_MCG", "CB_MUL1", "MUL1_MULT", "MCG_MULT", "THREEINST_MULT",
           "THREEINST_ADD", "codebook_lut", "tensor_core_perm", "tensor_core_perm_inv",
           "pack_trellis", "pack_trellis_batch", "swap16_storage", "words_from_storage",
           "stream_from_words", "state_index", "decode_states", "decode_tile_values"]
