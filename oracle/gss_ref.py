"""CPU oracle for the global-scale search — TEST INFRASTRUCTURE ONLY.

numpy restatement of exl3_quant/gss.py: the tile sample (gss.py:65-97),
the refined-scale selection (gss.py:100-115) and the two-stage grid search
(gss.py:118-184) over any tile encoder given as a numpy callback
(tiles (n, 256) float32 -> (reconstruction, states)). Only tests/ may use it.

Pinned by tests/test_gss_host.py: the sample covers every tile row and
column and contains the extreme-RMS tiles found by brute force; the
refinement returns the exact vertex of a sampled parabola, walks ties to the
left edge and floors at 0.01; with a clipped-grid quantiser whose MSE curve
is known in closed form, the search lands within a fine step of the
brute-force minimum.
"""

from __future__ import annotations

import numpy as np

from oracle.trellis_format_ref import tensor_core_perm

COARSE = [0.1 + 0.2 * i for i in range(10)]
FINE_STEP = 0.075
MIN_SCALE = 0.01


def sample_scale_tiles(w: np.ndarray, width: int = 3) -> np.ndarray:
    tk, tn = w.shape[0] // 16, w.shape[1] // 16
    grid = w.reshape(tk, 16, tn, 16).transpose(0, 2, 1, 3).astype(np.float32)
    span = max(tk, tn)
    picks = [(d % tk, (d + j) % tn) for d in range(span) for j in range(width)]
    ms = (grid.astype(np.float64) ** 2).mean(axis=(2, 3)).reshape(-1)
    num_x = min(max(8, span * width // 16), (ms.size + 1) // 2)
    order = np.argsort(-ms, kind="stable")
    hi = order[:num_x]
    lo = np.argsort(ms, kind="stable")[:num_x]
    picks += [(int(i) // tn, int(i) % tn) for i in np.concatenate((hi, lo))]
    tiles = np.stack([grid[r, c].reshape(256) for r, c in picks])
    return np.ascontiguousarray(tiles[:, tensor_core_perm()])


def select_refined_scale(scales, mses) -> float:
    best = int(np.argmin(np.asarray(mses)))
    off = 0.0
    if 0 < best < len(scales) - 1:
        y0, y1, y2 = mses[best - 1], mses[best], mses[best + 1]
        den = y0 - 2.0 * y1 + y2
        if den > 0:
            off = float(np.clip(0.5 * (y0 - y2) / den, -0.5, 0.5))
    return max(scales[best] + off * FINE_STEP, MIN_SCALE)


def _mse(tiles: np.ndarray, s: float, encode) -> float:
    recon, _ = encode((tiles * np.float32(s)).astype(np.float32))
    return float(((recon.astype(np.float32) / np.float32(s) - tiles) ** 2).mean(dtype=np.float64))


def g_scale_search(samples, encode):
    out = []
    for tiles in samples:
        coarse = [_mse(tiles[::3], s, encode) for s in COARSE]
        c = COARSE[int(np.argmin(coarse))]
        fine_s = [c + FINE_STEP * (i - 2) for i in range(5)]
        fine = [_mse(tiles, s, encode) for s in fine_s]
        out.append((select_refined_scale(fine_s, fine), min(fine)))
    return out
