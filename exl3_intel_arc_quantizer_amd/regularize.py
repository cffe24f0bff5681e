"""EXL3 weight regularisation before encoding (reference: exl3_quant/regularize.py).

Per linear layer, before the Hessian factorisation: optional output-channel
normalisation (decided by the Hessian-diagonal skew heuristic), folding of
the su / sv scale vectors, the right and left blockwise Hadamard transforms
and an optional global scale. The order is fixed: divide by sv, H_r, divide
by su, H_l; ``hadamard.weight_from_quantized`` undoes it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional

import torch

from .hadamard import HAD_DIM, blockwise_preapply_had_l_, blockwise_preapply_had_r_

CODEBOOK_SCALE = 1.24371088     # regularize.py:33
OUT_SCALE_SKEW_CUTOFF = 0.15
SKEW_FRACTION = 50              # top 2 % of the diagonal
ZERO_FLOOR = 0.1
EPS = 1e-10


def block_rms(x: torch.Tensor, dim: int, keepdim: bool = False,
              blocksize: int = 32) -> torch.Tensor:
    """sqrt(mean of squares) along ``dim`` of a 2-D GPU tensor, the squares
    summed in ``blocksize`` slices whose sums are accumulated in slice order
    (regularize.py:41-56); the slice order fixes the rounding. One launch of
    the HIP kernel ``exl3_block_rms``."""
    if x.dim() != 2:
        raise ValueError(f"block_rms expects a 2-D tensor, got shape {tuple(x.shape)}")
    if x.device.type != "cuda":
        raise ValueError("block_rms runs on the GPU; move the tensor to a cuda device")
    from ._native import block_rms as _block_rms
    d = dim % 2
    rows, cols = x.shape
    work = x if (x.dtype == torch.float32 and x.is_contiguous()) else \
        x.to(torch.float32).contiguous()
    if keepdim:
        shape = (1, cols) if d == 0 else (rows, 1)
    else:
        shape = (cols,) if d == 0 else (rows,)
    out = torch.empty(shape, dtype=torch.float32, device=x.device)
    _block_rms(work, out, d, int(blocksize))
    return out


@dataclass
class RegularizeResult:
    """Outputs of :func:`regularize` (regularize.py:59-71)."""

    apply_out_scales: bool
    weight: torch.Tensor
    g_scale: float
    su: torch.Tensor
    sv: torch.Tensor
    out_channel_scales: torch.Tensor
    in_channel_scales: torch.Tensor
    zeros: bool
    skew_factor: Optional[float]


def regularize(weight: torch.Tensor, su: torch.Tensor, sv: torch.Tensor,
               quant_args: Optional[dict] = None, H_diag: Optional[torch.Tensor] = None,
               skip_g_scale: bool = True, q_fallback: bool = False,
               g_scale_fn: Optional[Callable[[torch.Tensor], float]] = None,
               had_dim: int = HAD_DIM) -> RegularizeResult:
    """Transform a (k, n) float32 layer weight into the encoder's basis
    (regularize.py:74-211). ``weight`` is not modified."""
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D, got shape {tuple(weight.shape)}")
    if weight.dtype != torch.float32:
        raise ValueError(f"weight must be float32, got {weight.dtype}")
    k, n = weight.shape
    if su.numel() != k or sv.numel() != n:
        raise ValueError(f"su must have {k} elements and sv {n}, got {su.numel()} / {sv.numel()}")
    if k % had_dim != 0 or n % had_dim != 0:
        raise ValueError(f"both dimensions must be divisible by {had_dim}, got {(k, n)}")
    args = {} if quant_args is None else quant_args
    force_out_scales = args.get("apply_out_scales")

    # Output-scale decision from the skew of the Hessian diagonal.
    skew_factor: Optional[float] = None
    if not q_fallback and H_diag is not None:
        diag, _ = torch.sort(H_diag.sqrt(), descending=True)
        cutoff = diag.shape[0] // SKEW_FRACTION
        skew_factor = float(diag[:cutoff].sum() / diag.sum())
        apply_out_scales = (skew_factor < OUT_SCALE_SKEW_CUTOFF if force_out_scales is None
                            else bool(force_out_scales))
    else:
        apply_out_scales = True if force_out_scales is None else bool(force_out_scales)
    if q_fallback:
        apply_out_scales = bool(force_out_scales)

    # Output channel scales.
    work = weight.clone()
    out_channel_scales = block_rms(work, dim=0, keepdim=True)
    mean = out_channel_scales.mean().item()
    if mean > 1e-30:
        out_channel_scales /= mean
        zeros = False
    else:
        zeros = True
        if force_out_scales is not None:
            apply_out_scales = True
    zero_out_scales = out_channel_scales.abs() < 1e-30
    su = su.to(torch.float32).clone()
    sv = sv.to(torch.float32).clone()
    if apply_out_scales:
        out_channel_scales[zero_out_scales] = ZERO_FLOOR
        sv = (sv * out_channel_scales + EPS).float()

    # Fold sv, right Hadamard.
    work /= sv
    sv[zero_out_scales] = 0.0
    blockwise_preapply_had_r_(work, had_dim)

    # Input channel scales, su, left Hadamard.
    in_channel_scales = block_rms(work, dim=1, keepdim=True)
    in_channel_scales[in_channel_scales.abs() < 1e-30] = ZERO_FLOOR
    su = (su * in_channel_scales / (-CODEBOOK_SCALE) + EPS).float()
    work /= su
    blockwise_preapply_had_l_(work, had_dim)

    # Global scale.
    if skip_g_scale:
        g_scale = 1.0
    else:
        if g_scale_fn is None:
            raise ValueError("skip_g_scale=False requires g_scale_fn")
        g_scale = float(g_scale_fn(work))
        if not g_scale > 0.0:
            raise ValueError(f"g_scale_fn returned a non-positive scale: {g_scale}")
    work *= g_scale
    su /= g_scale
    if "zeros" in args or quant_args is not None:
        args["zeros"] = zeros
    return RegularizeResult(apply_out_scales=bool(apply_out_scales), weight=work, g_scale=g_scale,
                            su=su, sv=sv, out_channel_scales=out_channel_scales,
                            in_channel_scales=in_channel_scales, zeros=zeros,
                            skew_factor=skew_factor)
