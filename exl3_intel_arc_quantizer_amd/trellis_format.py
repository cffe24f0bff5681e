"""EXL3 format constants and the device-side format helpers.

Counterpart of the reference's exl3_quant/trellis_format.py. The bit layouts
are fixed by the EXL3 format (upstream exllamav3 codebook.cuh, pack.cu,
quantize.py) and are restated here; the arithmetic runs on the GPU:
``codebook_lut`` launches the decode kernel and ``pack_trellis_batch`` the
packing kernel of ``libexl3_hip.so``. The tensor-core permutation is a fixed
index table and is built on the host.
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

_LUT_CACHE: dict = {}


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


def pack_trellis_batch(states, K: int):
    """pack_trellis + swap16_storage (trellis_format.py:120-174) of a batch of
    states on the GPU. ``states``: (n, 256) uint16/int16 array or device tensor.
    Returns the (n, 16K) uint16 storage words (numpy for numpy input, an int16
    device tensor for tensor input)."""
    import torch

    from ._native import extension

    if not 1 <= K <= 8:
        raise ValueError(f"K must be in 1..8, got {K}")
    if isinstance(states, torch.Tensor):
        s = states.to(torch.int16).contiguous()
        out = torch.empty((s.shape[0], 16 * K), dtype=torch.int16, device=s.device)
        extension().pack_trellis(s, out, K)
        return out
    arr = np.ascontiguousarray(np.asarray(states, dtype=np.uint16).reshape(-1, 256))
    s = torch.from_numpy(arr.view(np.int16)).cuda()
    out = torch.empty((s.shape[0], 16 * K), dtype=torch.int16, device=s.device)
    extension().pack_trellis(s, out, K)
    return out.cpu().numpy().view(np.uint16)


def pack_trellis(states: np.ndarray, K: int) -> np.ndarray:
    """Single-tile packing in stored (SWAP16) order."""
    return pack_trellis_batch(np.asarray(states).reshape(1, 256), K)[0]
