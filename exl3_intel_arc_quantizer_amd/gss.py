"""Global-scale search over the HIP tile encoder (reference: exl3_quant/gss.py).

Before LDLQ, ``regularize`` may multiply the transformed weight by one
global scale g (and divide su by it) so the weight sits where the trellis
codebook reconstructs it best. The search measures, for candidate scales s,
the tile MSE of encode(s * tiles) / s - tiles on a sample of the weight's
tiles:

* sample (gss.py:65-97): a wrapped diagonal of width ``width`` over the
  tile grid (every tile row and column at least once) plus the
  highest- and lowest-RMS tiles;
* coarse grid 0.1, 0.3, ..., 1.9 on every third sampled tile, then five
  points 0.075 apart around the coarse minimum on the whole sample, then a
  parabolic step from the three points around the fine minimum, clamped to
  half a grid step, floored at 0.01 (gss.py:100-184).

Here every candidate's tiles go to the encoder in as few calls as the
``max_tiles`` bound allows, the calls are queued without waiting (the HIP
adapter is asynchronous) and each stage reads its MSEs back once. A
candidate's MSE is computed from its own slice, so batching and chunking do
not change any value.
"""

from __future__ import annotations

from typing import Callable, List, Sequence, Tuple

import torch

from .trellis_format import tensor_core_perm

COARSE_START = 0.1
COARSE_STEP = 0.2
COARSE_POINTS = 10
FINE_POINTS = 5
FINE_STEP = 0.075
MIN_SCALE = 0.01
MAX_TILES_PER_CALL = 65536

TileEncoder = Callable[[torch.Tensor], Tuple[torch.Tensor, torch.Tensor]]

__all__ = ["COARSE_START", "COARSE_STEP", "COARSE_POINTS", "FINE_POINTS", "FINE_STEP",
           "MIN_SCALE", "MAX_TILES_PER_CALL", "sample_scale_tiles", "select_refined_scale",
           "g_scale_search_batch", "g_scale_gss", "g_scale_fn_from_encoder"]


def sample_scale_tiles(weight_r: torch.Tensor, width: int = 3) -> torch.Tensor:
    """(T, 256) float32 tensor-core-order sample of a (k, n) weight's 16x16
    tiles (gss.py:65-97): tile (d mod tiles_k, (d + w) mod tiles_n) for
    d < max(tiles_k, tiles_n), w < width; then the num_x highest- and the
    num_x lowest-mean-square tiles, num_x = max(8, diagonal size / 16)
    capped at half the tile count (rounded up)."""
    if weight_r.dim() != 2 or weight_r.shape[0] % 16 or weight_r.shape[1] % 16:
        raise ValueError(f"weight must be (k, n) with both multiples of 16, got "
                         f"{tuple(weight_r.shape)}")
    device = weight_r.device
    tk, tn = weight_r.shape[0] // 16, weight_r.shape[1] // 16
    grid = weight_r.reshape(tk, 16, tn, 16).permute(0, 2, 1, 3)          # (tk, tn, 16, 16)
    span = max(tk, tn)
    d = torch.arange(span, device=device).repeat_interleave(width)
    w = torch.arange(width, device=device).repeat(span)
    rows, cols = d % tk, (d + w) % tn
    ms = grid.square().mean(dim=(2, 3)).flatten()
    num_x = min(max(8, (span * width) // 16), (ms.numel() + 1) // 2)
    extreme = torch.cat((torch.topk(ms, num_x).indices,
                         torch.topk(ms, num_x, largest=False).indices))
    rows = torch.cat((rows, extreme // tn))
    cols = torch.cat((cols, extreme % tn))
    tiles = grid[rows, cols].reshape(-1, 256)
    perm = torch.as_tensor(tensor_core_perm(), dtype=torch.long, device=device)
    return tiles[:, perm].contiguous()


def select_refined_scale(fine_scales: Sequence[float], fine_mses: Sequence[float]) -> float:
    """Fine-grid minimum (first on ties) moved by the vertex of the parabola
    through it and its neighbours when it is interior and the parabola opens
    upward, by at most half a step; floored at MIN_SCALE (gss.py:100-115)."""
    best = min(range(len(fine_mses)), key=lambda i: fine_mses[i])
    shift = 0.0
    if 0 < best < len(fine_scales) - 1:
        left, mid, right = fine_mses[best - 1], fine_mses[best], fine_mses[best + 1]
        curvature = left - 2.0 * mid + right
        if curvature > 0:
            shift = min(0.5, max(-0.5, 0.5 * (left - right) / curvature))
    return max(fine_scales[best] + shift * FINE_STEP, MIN_SCALE)


def _candidate_mses(cands: List[Tuple[int, float]], tile_sets: Sequence[torch.Tensor],
                    encode_tiles: TileEncoder, max_tiles: int) -> torch.Tensor:
    """MSE of every (tensor, scale) candidate: consecutive candidates share an
    encoder call while their tiles fit in ``max_tiles`` (at least one per
    call); results stay on the device."""
    device = tile_sets[0].device
    out = torch.empty(len(cands), dtype=torch.float32, device=device)
    start = 0
    while start < len(cands):
        stop, tiles = start, 0
        while stop < len(cands) and tiles + tile_sets[cands[stop][0]].shape[0] <= max_tiles:
            tiles += tile_sets[cands[stop][0]].shape[0]
            stop += 1
        stop = max(stop, start + 1)
        batch = torch.cat([tile_sets[t] * s for t, s in cands[start:stop]])
        recon, _ = encode_tiles(batch)
        recon = recon.to(device=device, dtype=torch.float32)
        off = 0
        for c, (t, s) in enumerate(cands[start:stop], start=start):
            cnt = tile_sets[t].shape[0]
            out[c] = (recon[off:off + cnt] / s - tile_sets[t]).square().mean()
            off += cnt
        start = stop
    return out


def g_scale_search_batch(samples: Sequence[torch.Tensor], encode_tiles: TileEncoder,
                         max_tiles: int = MAX_TILES_PER_CALL) -> List[Tuple[float, float]]:
    """(best scale, its fine-grid MSE) for each (T, 256) tensor-core-order
    sample (gss.py:118-184)."""
    if len(samples) == 0:
        return []
    for t, s in enumerate(samples):
        if s.dim() != 2 or s.shape[1] != 256 or s.shape[0] < 1:
            raise ValueError(f"samples[{t}] must be (T, 256) tensor-core-order tiles, "
                             f"got {tuple(s.shape)}")
    n_t = len(samples)
    coarse = [COARSE_START + COARSE_STEP * i for i in range(COARSE_POINTS)]
    thinned = [s[::3] for s in samples]
    stage1 = _candidate_mses([(t, s) for t in range(n_t) for s in coarse], thinned,
                             encode_tiles, max_tiles)
    centres = [coarse[i] for i in stage1.view(n_t, COARSE_POINTS).argmin(dim=1).tolist()]
    fine = [[c + FINE_STEP * (i - FINE_POINTS // 2) for i in range(FINE_POINTS)] for c in centres]
    stage2 = _candidate_mses([(t, s) for t in range(n_t) for s in fine[t]], samples,
                             encode_tiles, max_tiles).view(n_t, FINE_POINTS).tolist()
    return [(select_refined_scale(fine[t], stage2[t]), min(stage2[t])) for t in range(n_t)]


def g_scale_gss(weight_r: torch.Tensor, encode_tiles: TileEncoder,
                width: int = 3) -> Tuple[float, float]:
    """Global scale of one transformed weight (gss.py:187-197)."""
    return g_scale_search_batch([sample_scale_tiles(weight_r, width)], encode_tiles)[0]


def g_scale_fn_from_encoder(encode_tiles: TileEncoder,
                            width: int = 3) -> Callable[[torch.Tensor], float]:
    """The ``g_scale_fn`` hook of ``regularize`` (gss.py:200-207)."""
    def g_scale_fn(weight_r: torch.Tensor) -> float:
        return g_scale_gss(weight_r, encode_tiles, width)[0]
    return g_scale_fn
