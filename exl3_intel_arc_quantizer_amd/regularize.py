"""Weight regularisation before LDLQ, as a three-pass GPU pipeline
(reference: exl3_quant/regularize.py:41-211; public names and signatures kept).

What the transform is (fixed by the EXL3 format, because decoding undoes it
in reverse with ``hadamard.weight_from_quantized``): a (k, n) weight W
becomes ``H_l((H_r(W / sv)) / su) * g``, where

* sv (1, n) carries the output-channel scales: the RMS of each column of W
  divided by the mean column RMS, plus 1e-10, when the Hessian diagonal is
  not too skewed (the top 2 % of sqrt(diag H) hold less than 15 % of its
  sum), else the caller's sv unchanged; columns whose RMS is zero keep a
  0.1 scale for the division and are stored as sv = 0;
* su (k, 1) carries the input-channel scales: the RMS of each row of
  H_r(W / sv), divided by -1.24371088 (the codebook's scale), plus 1e-10;
  zero rows use 0.1;
* g is the global scale (1 unless a search function is given).

How it runs here. The reference spends about a dozen full passes over the
matrix (clone, RMS, division, transform, RMS, division, transform). This
module makes three, on HIP kernels of ``libexl3_hip.so``:

1. ``exl3_block_rms`` along the columns of W (two launches);
2. ``exl3_hadamard128_scaled`` side 1: W / sv and the right transform into a
   new matrix in one read and one write, with the sums of squares of every
   32-element row slice as a by-product; ``exl3_block_rms_from_slices``
   turns those into the row RMS (a reduction over k x n/32 floats);
3. ``exl3_hadamard128_scaled`` side 0: division by su and the left
   transform, in place.

The scale vectors (n and k floats) are handled by torch between the passes;
one host read of the mean column RMS decides the all-zero case, as in the
reference.

Rounding. Divisions are correctly rounded fp32, like torch's; the transform
is the fast Walsh-Hadamard transform of ``exl3_hadamard128``. The RMS splits
each row or column into 32-element slices and adds the slice sums in slice
order, as the reference's ``block_rms`` does; within a slice the order is
this build's (sequential for the column RMS, a butterfly over lanes for the
row RMS), just as torch's own reduction order is an implementation detail.
Results therefore agree with the reference's to float32 rounding.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Tuple

import torch

from .hadamard import HAD_DIM

CODEBOOK_SCALE = 1.24371088     # the codebook's RMS, regularize.py:33
OUT_SCALE_SKEW_CUTOFF = 0.15    # output scales only below this skew
SKEW_FRACTION = 50              # the skew looks at the top 1/50 of the diagonal
ZERO_FLOOR = 0.1                # scale used for an all-zero row or column
EPS = 1e-10                     # added to every scale
RMS_SLICE = 32                  # block_rms slice length
_TINY = 1e-30                   # below this an RMS counts as zero


def block_rms(x: torch.Tensor, dim: int, keepdim: bool = False,
              blocksize: int = RMS_SLICE) -> torch.Tensor:
    """Root mean square along ``dim`` of a 2-D GPU tensor (regularize.py:41-56):
    squares summed in ``blocksize`` slices, slice sums added in slice order,
    one launch pair of ``exl3_block_rms``."""
    if x.dim() != 2:
        raise ValueError(f"block_rms expects a 2-D tensor, got shape {tuple(x.shape)}")
    if x.device.type != "cuda":
        raise ValueError("block_rms runs on the GPU; move the tensor to a cuda device")
    from ._native import block_rms as _block_rms
    axis = dim % 2
    rows, cols = x.shape
    src = x if (x.dtype == torch.float32 and x.is_contiguous()) else \
        x.to(torch.float32).contiguous()
    n_out = cols if axis == 0 else rows
    out = torch.empty(n_out, dtype=torch.float32, device=x.device)
    _block_rms(src, out, axis, int(blocksize))
    if keepdim:
        return out.reshape(1, cols) if axis == 0 else out.reshape(rows, 1)
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


def _skew_tensor(H_diag: torch.Tensor) -> torch.Tensor:
    root = torch.sort(H_diag.sqrt(), descending=True).values
    top = root.shape[0] // SKEW_FRACTION
    return root[:top].sum() / root.sum()


def hessian_skew(H_diag: torch.Tensor) -> float:
    """Share of sum(sqrt(diag H)) held by its largest len/50 entries."""
    return float(_skew_tensor(H_diag))


def _out_scale_decision(H_diag: Optional[torch.Tensor], forced: Optional[bool],
                        q_fallback: bool) -> Tuple[Optional[bool], Optional[torch.Tensor]]:
    """(apply the output-channel scales?, skew as a device scalar or None).
    A forced value wins; without one the skew decides, and without a
    Hessian diagonal the scales apply. In fallback mode only a forced True
    applies them. The decision is None when the skew makes it: the caller
    then selects on the device and reads it back once, at the end."""
    if q_fallback:
        return bool(forced), None
    if H_diag is None:
        return (True if forced is None else bool(forced)), None
    return (None if forced is None else bool(forced)), _skew_tensor(H_diag)


def _check_inputs(weight: torch.Tensor, su: torch.Tensor, sv: torch.Tensor, had_dim: int) -> None:
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D, got shape {tuple(weight.shape)}")
    if weight.dtype != torch.float32:
        raise ValueError(f"weight must be float32, got {weight.dtype}")
    k, n = weight.shape
    if su.numel() != k or sv.numel() != n:
        raise ValueError(f"su must have {k} elements and sv {n}, got {su.numel()} / {sv.numel()}")
    if k % had_dim != 0 or n % had_dim != 0:
        raise ValueError(f"both dimensions must be divisible by {had_dim}, got {(k, n)}")
    if had_dim != HAD_DIM:
        raise ValueError(f"only had_dim={HAD_DIM} is supported, got {had_dim}")
    if weight.device.type != "cuda":
        raise ValueError("regularize runs on the GPU; move the weight to a cuda device")


def regularize(weight: torch.Tensor, su: torch.Tensor, sv: torch.Tensor,
               quant_args: Optional[dict] = None, H_diag: Optional[torch.Tensor] = None,
               skip_g_scale: bool = True, q_fallback: bool = False,
               g_scale_fn: Optional[Callable[[torch.Tensor], float]] = None,
               had_dim: int = HAD_DIM) -> RegularizeResult:
    """Transform a (k, n) float32 GPU weight into the encoder's basis
    (regularize.py:83-211). ``weight`` is not modified. ``quant_args`` may
    force ``apply_out_scales``; when given, its ``zeros`` entry is set to
    whether W had no energy at all."""
    from ._native import block_rms_from_slices, hadamard128_scaled

    _check_inputs(weight, su, sv, had_dim)
    k, n = weight.shape
    dev = weight.device
    forced = None if quant_args is None else quant_args.get("apply_out_scales")
    apply_out, skew_t = _out_scale_decision(H_diag, forced, q_fallback)
    w = weight.contiguous()

    # Pass 1: output-channel scales from the column RMS, normalised by
    # their mean unless W has no energy (the scales then stay as they are).
    # Nothing is read back here: the decisions select on the device and
    # come back together after the last pass.
    out_scales = block_rms(w, dim=0, keepdim=True)
    mean = out_scales.mean()
    live = mean > _TINY
    out_scales /= torch.where(live, mean, torch.ones_like(mean))
    if forced is not None and not bool(live):
        apply_out = True          # a forced decision on an all-zero W applies the scales
    dead_cols = out_scales.abs() < _TINY
    sv = sv.to(device=dev, dtype=torch.float32).reshape(1, n).clone()
    if apply_out is None:
        apply_t = skew_t < OUT_SCALE_SKEW_CUTOFF
        out_scales.copy_(torch.where(dead_cols & apply_t, ZERO_FLOOR, out_scales))
        sv = torch.where(apply_t, (sv * out_scales + EPS).float(), sv)
    elif apply_out:
        out_scales[dead_cols] = ZERO_FLOOR
        sv = (sv * out_scales + EPS).float()

    # Pass 2: W / sv and the right transform, with the row slice sums of
    # squares for the input-channel scales.
    work = torch.empty_like(w)
    slice_sq = torch.empty((k, n // RMS_SLICE), dtype=torch.float32, device=dev)
    hadamard128_scaled(w, work, 1, divisor=sv.reshape(n).contiguous(), slice_sumsq=slice_sq)
    sv[dead_cols] = 0.0
    in_scales = torch.empty((k, 1), dtype=torch.float32, device=dev)
    block_rms_from_slices(slice_sq, in_scales, n)
    del slice_sq
    in_scales[in_scales.abs() < _TINY] = ZERO_FLOOR
    su = su.to(device=dev, dtype=torch.float32).reshape(k, 1)
    su = (su * in_scales / (-CODEBOOK_SCALE) + EPS).float()

    # Pass 3: divide by su and the left transform, in place.
    hadamard128_scaled(work, work, 0, divisor=su.reshape(k).contiguous())

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
    flags = [live.to(torch.float64)]
    if skew_t is not None:
        flags += [skew_t.to(torch.float64), (skew_t < OUT_SCALE_SKEW_CUTOFF).to(torch.float64)]
    flags = torch.stack(flags).tolist()          # the one read-back of the pipeline
    zeros = not flags[0]
    skew = flags[1] if skew_t is not None else None
    if apply_out is None:
        apply_out = bool(flags[2])
    if quant_args is not None:
        quant_args["zeros"] = zeros
    return RegularizeResult(apply_out_scales=bool(apply_out), weight=work, g_scale=g_scale,
                            su=su, sv=sv, out_channel_scales=out_scales,
                            in_channel_scales=in_scales, zeros=zeros, skew_factor=skew)

