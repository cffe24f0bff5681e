"""Blockwise Sylvester Hadamard transforms (reference: exl3_quant/hadamard.py).

EXL3 rotates weights and Hessians with the orthonormal Sylvester matrix of
order 128 applied blockwise: ``preapply_had_l`` multiplies each 128-row block
from the left (``H @ x``), ``preapply_had_r`` each 128-column block from the
right (``x @ H``). The matrix is symmetric and its own inverse, so decoding
applies the same transforms in reverse order (``weight_from_quantized``).

On the GPU every block product of a call is one batched fp32 GEMM
(hipBLASLt through torch) instead of a Python loop over blocks.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

HAD_DIM = 128
_HAD_CACHE: dict = {}


def sylvester_hadamard(n: int) -> torch.Tensor:
    """Unnormalised Sylvester matrix of order n (+-1, float64), built by the
    recursion [[h, h], [h, -h]] (hadamard.py:34-54). n must be a power of two."""
    if n < 1 or (n & (n - 1)) != 0:
        raise ValueError(f"Sylvester construction requires a power-of-two size, got {n}")
    h = torch.ones((1, 1), dtype=torch.float64)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], dim=1), torch.cat([h, -h], dim=1)], dim=0)
    return h


def hadamard(n: int = HAD_DIM, dtype: torch.dtype = torch.float32,
             scale: Optional[float] = None,
             device: Optional[torch.device] = None) -> torch.Tensor:
    """Orthonormal Sylvester matrix, scale 1/sqrt(n) by default (hadamard.py:57-70)."""
    if scale is None:
        scale = 1.0 / math.sqrt(n)
    key = (n, dtype, float(scale), str(device) if device is not None else "cpu")
    cached = _HAD_CACHE.get(key)
    if cached is None:
        cached = (sylvester_hadamard(n) * scale).to(dtype=dtype, device=device)
        _HAD_CACHE[key] = cached
    return cached


def preapply_had_l(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """H @ x on each 128-row block (hadamard.py:73-83)."""
    k, n = x.shape
    if k % had_dim != 0:
        raise ValueError(f"rows ({k}) must be divisible by had_dim ({had_dim})")
    work = x.to(torch.float32).contiguous()
    had = hadamard(had_dim, torch.float32, device=x.device)
    return torch.matmul(had, work.view(-1, had_dim, n)).view(k, n).to(x.dtype)


def preapply_had_r(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """x @ H on each 128-column block (hadamard.py:86-96)."""
    k, n = x.shape
    if n % had_dim != 0:
        raise ValueError(f"columns ({n}) must be divisible by had_dim ({had_dim})")
    work = x.to(torch.float32).contiguous()
    had = hadamard(had_dim, torch.float32, device=x.device)
    return torch.matmul(work.view(k, -1, had_dim), had).view(k, n).to(x.dtype)


def blockwise_preapply_had_l_(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """In-place H @ x on 128-row blocks of a float32 matrix (hadamard.py:99-111)."""
    if x.dtype != torch.float32:
        raise ValueError(f"in-place Hadamard requires float32, got {x.dtype}")
    x.copy_(preapply_had_l(x, had_dim))
    return x


def blockwise_preapply_had_r_(x: torch.Tensor, had_dim: int = HAD_DIM) -> torch.Tensor:
    """In-place x @ H on 128-column blocks of a float32 matrix (hadamard.py:114-126)."""
    if x.dtype != torch.float32:
        raise ValueError(f"in-place Hadamard requires float32, got {x.dtype}")
    x.copy_(preapply_had_r(x, had_dim))
    return x


def weight_from_quantized(w_hat: torch.Tensor, su: torch.Tensor,
                          sv: torch.Tensor) -> torch.Tensor:
    """Original-basis weight from the transformed reconstruction: H_l, x su,
    H_r, x sv (hadamard.py:129-140)."""
    k, n = w_hat.shape
    if su.numel() != k or sv.numel() != n:
        raise ValueError(f"su must have {k} elements and sv {n}, got {su.numel()} / {sv.numel()}")
    work = preapply_had_l(w_hat.to(torch.float32), HAD_DIM)
    work = work * su.to(torch.float32).reshape(k, 1)
    work = preapply_had_r(work, HAD_DIM)
    return work * sv.to(torch.float32).reshape(1, n)
