"""Blockwise Sylvester Hadamard transforms (reference: exl3_quant/hadamard.py).

EXL3 rotates weights and Hessians with the orthonormal Sylvester matrix of
order 128 applied blockwise: ``preapply_had_l`` multiplies each 128-row block
from the left (``H @ x``), ``preapply_had_r`` each 128-column block from the
right (``x @ H``). The matrix is symmetric and its own inverse, so decoding
applies the same transforms in reverse order (``weight_from_quantized``).

On the GPU the transforms are one launch of a fast Walsh-Hadamard kernel
(``exl3_hadamard128``, HIP): 7 butterfly levels of fp32 additions and one
scale per element instead of a 128-term product, bound by one HBM read and
write of the matrix. The results equal the matrix products up to fp32
rounding of the summation order.
"""

from __future__ import annotations

import functools
import math
from typing import Optional

import torch

HAD_DIM = 128


def sylvester_hadamard(n: int) -> torch.Tensor:
    """Unnormalised Sylvester matrix of order n (+-1, float64; hadamard.py:
    34-54), from its closed form: entry (i, j) is (-1)^popcount(i & j), the
    parity of the bits row and column share. n must be a power of two."""
    if n < 1 or (n & (n - 1)) != 0:
        raise ValueError(f"Sylvester construction requires a power-of-two size, got {n}")
    idx = torch.arange(n, dtype=torch.int64)
    shared = idx[:, None] & idx[None, :]
    parity = torch.zeros_like(shared)
    for bit in range(n.bit_length() - 1):
        parity ^= (shared >> bit) & 1
    return (1 - 2 * parity).to(torch.float64)


@functools.lru_cache(maxsize=None)
def _scaled_hadamard(n: int, dtype: torch.dtype, scale: float, device: str) -> torch.Tensor:
    return (sylvester_hadamard(n) * scale).to(dtype=dtype, device=device)


def hadamard(n: int = HAD_DIM, dtype: torch.dtype = torch.float32,
             scale: Optional[float] = None,
             device: Optional[torch.device] = None) -> torch.Tensor:
    """Sylvester matrix times ``scale`` (default 1/sqrt(n): orthonormal), in
    ``dtype`` on ``device`` (hadamard.py:57-70). One tensor per argument set
    is built and then shared, so callers must not modify it."""
    factor = 1.0 / math.sqrt(n) if scale is None else float(scale)
    return _scaled_hadamard(n, dtype, factor, "cpu" if device is None else str(device))


def _had128(x: torch.Tensor, side: int, had_dim: int, out: Optional[torch.Tensor]) -> torch.Tensor:
    """The blockwise transform through the HIP fast Walsh-Hadamard kernel
    (``exl3_hadamard128``); GPU tensors only."""
    if had_dim != HAD_DIM:
        raise ValueError(f"only had_dim={HAD_DIM} is supported, got {had_dim}")
    if x.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(x.shape)}")
    k, n = x.shape
    if side == 0 and k % had_dim != 0:
        raise ValueError(f"rows ({k}) must be divisible by had_dim ({had_dim})")
    if side == 1 and n % had_dim != 0:
        raise ValueError(f"columns ({n}) must be divisible by had_dim ({had_dim})")
    if x.device.type != "cuda":
        raise ValueError("the Hadamard transforms run on the GPU; move the tensor to a cuda device")
    from ._native import hadamard128
    work = x if (x.dtype == torch.float32 and x.is_contiguous()) else \
        x.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(work)
    hadamard128(work, out, side)
    return out


def preapply_had_l(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """H @ x on each 128-row block (hadamard.py:73-83), as a new tensor of
    x's dtype."""
    return _had128(x, 0, had_dim, None).to(x.dtype)


def preapply_had_r(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """x @ H on each 128-column block (hadamard.py:86-96), as a new tensor of
    x's dtype."""
    return _had128(x, 1, had_dim, None).to(x.dtype)


def _in_place(x: torch.Tensor, side: int, had_dim: int) -> torch.Tensor:
    if x.dtype != torch.float32:
        raise ValueError(f"in-place Hadamard requires float32, got {x.dtype}")
    if x.is_contiguous():
        _had128(x, side, had_dim, x)
    else:
        x.copy_(_had128(x, side, had_dim, None))
    return x


def blockwise_preapply_had_l_(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """In-place H @ x on 128-row blocks of a float32 matrix (hadamard.py:99-111)."""
    return _in_place(x, 0, had_dim)


def blockwise_preapply_had_r_(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """In-place x @ H on 128-column blocks of a float32 matrix (hadamard.py:114-126)."""
    return _in_place(x, 1, had_dim)


def weight_from_quantized(w_hat: torch.Tensor, su: torch.Tensor,
                          sv: torch.Tensor) -> torch.Tensor:
    """Original-basis weight from the transformed reconstruction: H_l, x su,
    H_r, x sv (hadamard.py:129-140)."""
    k, n = w_hat.shape
    if su.numel() != k or sv.numel() != n:
        raise ValueError(f"su must have {k} elements and sv {n}, got {su.numel()} / {sv.numel()}")
    work = _had128(w_hat, 0, HAD_DIM, None)          # a new tensor: w_hat is not modified
    work.mul_(su.to(device=work.device, dtype=torch.float32).reshape(k, 1))
    _had128(work, 1, HAD_DIM, work)
    return work.mul_(sv.to(device=work.device, dtype=torch.float32).reshape(1, n))
