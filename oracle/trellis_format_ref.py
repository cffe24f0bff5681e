"""numpy restatement of the EXL3 format primitives — TEST INFRASTRUCTURE ONLY.

Restates exl3_quant/trellis_format.py of the reference (itself a transcription
of exllamav3 codebook.cuh / pack.cu / quantize.py and the exl3xpu decode
oracle). Used by the tests as the checker for the HIP kernels and for the
product's format helpers; never imported by the product package.
"""

from __future__ import annotations

import numpy as np

# Codebook selectors and hash constants (trellis_format.py:28-33).
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
MUL1_MULT = 0x83DCD12D
MCG_MULT = 0xCBAC1FED
THREEINST_MULT = 89226354
THREEINST_ADD = 64248484

# fp16 bit patterns used by the mul1 decoder: 0x1EEE (~1/128.6) and 0xC931.
_MUL1_SCALE_BITS = 0x1EEE
_MUL1_BIAS_BITS = 0xC931
# 0x6400 is the fp16 pattern of 1024.0; the lop3 mask/xor of the 3inst/mcg
# decoders (codebook.cuh immLut 0x6a == (a & b) ^ c).
_LOP3_AND = 0x8FFF8FFF
_LOP3_XOR = 0x3B603B60


def _as_f16(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


def codebook_lut(cb: int) -> np.ndarray:
    """fp16 value of every 16-bit state (trellis_format.py:41-81).

    The only fp16 operation of each decoder (mul1: one fused multiply-add;
    3inst/mcg: one add) is evaluated exactly in float64 and rounded once.
    """
    if cb not in (CB_3INST, CB_MCG, CB_MUL1):
        raise ValueError(f"Unknown codebook {cb}")
    state = np.arange(1 << 16, dtype=np.uint64)
    if cb == CB_MUL1:
        x = (state * np.uint64(MUL1_MULT)) & np.uint64(0xFFFFFFFF)
        byte_sum = sum((x >> np.uint64(s)) & np.uint64(0xFF) for s in (0, 8, 16, 24))
        # 0x6400 + byte_sum is the fp16 encoding of the integer 1024 + byte_sum.
        h = (np.uint64(0x6400) + byte_sum).astype(np.uint16).view(np.float16).astype(np.float64)
        scale = float(_as_f16([_MUL1_SCALE_BITS])[0])
        bias = float(_as_f16([_MUL1_BIAS_BITS])[0])
        return (h * scale + bias).astype(np.float16)
    if cb == CB_3INST:
        x = (state * np.uint64(THREEINST_MULT) + np.uint64(THREEINST_ADD)) & np.uint64(0xFFFFFFFF)
    else:
        x = (state * np.uint64(MCG_MULT)) & np.uint64(0xFFFFFFFF)
    x = (x & np.uint64(_LOP3_AND)) ^ np.uint64(_LOP3_XOR)
    lo = _as_f16((x & np.uint64(0xFFFF)).astype(np.uint16)).astype(np.float64)
    hi = _as_f16((x >> np.uint64(16)).astype(np.uint16)).astype(np.float64)
    return (lo + hi).astype(np.float16)


def tensor_core_perm() -> np.ndarray:
    """Tile permutation of the EXL3 tensor-core layout (trellis_format.py:88-108).

    Encoded element ``8*t + s`` is original position ``row*16 + col`` with
    rows {2(t%4), 2(t%4)+1, 2(t%4)+8, 2(t%4)+9} and columns {t//4, t//4+8}.
    """
    t = np.arange(32)
    r0 = (t % 4) * 2
    c0 = t // 4
    rows = np.stack([r0, r0 + 1, r0 + 8, r0 + 9] * 2, axis=1)
    cols = np.concatenate([np.repeat(c0[:, None], 4, 1), np.repeat(c0[:, None] + 8, 4, 1)], 1)
    return (rows * 16 + cols).reshape(-1).astype(np.int64)


def tensor_core_perm_inv() -> np.ndarray:
    """Inverse permutation (trellis_format.py:111-113)."""
    inv = np.empty(256, dtype=np.int64)
    inv[tensor_core_perm()] = np.arange(256)
    return inv


def pack_trellis(states: np.ndarray, K: int) -> np.ndarray:
    """Bit-pack one tile's states (trellis_format.py:120-159, pack.cu:9-57).

    Restated as a bit stream: within each of the 16 spans of 16 states, the
    low ``K`` bits of every state are concatenated MSB-first into a
    ``16*K``-bit string, which is cut into ``K`` big-endian uint16 words.
    """
    if not 1 <= K <= 8:
        raise ValueError(f"K must be in 1..8, got {K}")
    s = np.asarray(states, dtype=np.uint16).reshape(-1)
    if s.size != 256:
        raise ValueError(f"Expected 256 states per tile, got {s.size}")
    sym = (s & ((1 << K) - 1)).astype(np.int64).reshape(16, 16)
    bit = (sym[:, :, None] >> np.arange(K - 1, -1, -1)) & 1          # (span, elem, K) MSB first
    words = bit.reshape(16, K, 16)                                    # K words of 16 bits per span
    return (words << np.arange(15, -1, -1)).sum(-1).astype(np.uint16).reshape(-1)


def swap16_storage(s_packed: np.ndarray) -> np.ndarray:
    """Half-word swap of each uint16 pair (trellis_format.py:162-174, pack.cu:55-56)."""
    s = np.asarray(s_packed, dtype=np.uint16).reshape(-1, 2)
    return s[:, ::-1].reshape(-1).copy()


def words_from_storage(t16: np.ndarray) -> np.ndarray:
    """uint16 storage -> uint32 words, low half first (trellis_format.py:181-184)."""
    t = np.asarray(t16, dtype=np.uint16).reshape(-1, 2).astype(np.uint64)
    return t[:, 0] | (t[:, 1] << np.uint64(16))


def stream_from_words(words: np.ndarray) -> np.ndarray:
    """uint32 words -> MSB-first bit stream (trellis_format.py:187-190)."""
    w = np.asarray(words, dtype=np.uint64)
    return ((w[:, None] >> np.arange(31, -1, -1, dtype=np.uint64)) & np.uint64(1)).reshape(-1)


def state_index(K: int) -> np.ndarray:
    """Bit positions of element t's 16-bit window, ending at bit (t+1)K, circular
    (trellis_format.py:193-202)."""
    nbits = 256 * K
    end = (np.arange(256) + 1) * K
    return (end[:, None] - 16 + np.arange(16)[None, :]) % nbits


def decode_states(t16: np.ndarray, K: int) -> np.ndarray:
    """Packed tile -> 256 states (trellis_format.py:205-213)."""
    bits = stream_from_words(words_from_storage(t16)).astype(np.int64)
    win = bits[state_index(K)]
    return (win << np.arange(15, -1, -1)).sum(-1).astype(np.int64)


def decode_tile_values(t16: np.ndarray, K: int, cb: int = CB_MUL1) -> np.ndarray:
    """Packed tile -> 256 codebook values scattered to original order
    (trellis_format.py:216-227)."""
    vals = codebook_lut(cb)[decode_states(t16, K)]
    tile = np.empty(256, dtype=np.float16)
    tile[tensor_core_perm()] = vals
    return tile
