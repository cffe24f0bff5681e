"""Global-scale search host logic (exl3_intel_arc_quantizer_amd/gss.py) on
the CPU: the oracle (oracle/gss_ref.py) pinned by brute force and closed
forms, and the torch implementation against it with a clipped-grid
quantiser standing in for the trellis encoder (tests/test_gss.py of the
reference covers the same properties)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gss_ref
from oracle.trellis_format_ref import tensor_core_perm_inv


def _grid_np(tiles):
    return np.clip(np.round(tiles * 4.0) / 4.0, -1.5, 1.5).astype(np.float32), None


def _grid_torch(tiles):
    return torch.clamp(torch.round(tiles * 4.0) / 4.0, -1.5, 1.5), None


def _weight(k, n, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n)) * scale).astype(np.float32)
    w[:, rng.integers(0, n)] *= 6.0        # one loud column
    return w


@pytest.mark.parametrize("shape,width", [((128, 256), 3), ((256, 128), 2), ((64, 64), 1)])
def test_oracle_sample_covers_grid_and_extremes(shape, width):
    w = _weight(*shape, seed=1)
    tiles = gss_ref.sample_scale_tiles(w, width)
    tk, tn = shape[0] // 16, shape[1] // 16
    span = max(tk, tn)
    grid = w.reshape(tk, 16, tn, 16).transpose(0, 2, 1, 3).reshape(tk * tn, 256)
    orig = tiles[:, tensor_core_perm_inv()]
    pos = [int(np.flatnonzero((grid == t).all(axis=1))[0]) for t in orig]
    diag = pos[:span * width]
    assert {p // tn for p in diag} == set(range(tk))
    assert {p % tn for p in diag} == set(range(tn))
    ms = (grid.astype(np.float64) ** 2).mean(axis=1)
    num_x = min(max(8, span * width // 16), (tk * tn + 1) // 2)
    extra = pos[span * width:]
    assert sorted(extra[:num_x]) == sorted(np.argsort(-ms)[:num_x].tolist())
    assert sorted(extra[num_x:]) == sorted(np.argsort(ms)[:num_x].tolist())


def test_torch_sample_matches_oracle():
    from exl3_intel_arc_quantizer_amd.gss import sample_scale_tiles
    for shape, width in (((128, 256), 3), ((256, 128), 2), ((96, 32), 1)):
        w = _weight(*shape, seed=2)
        got = sample_scale_tiles(torch.from_numpy(w), width).numpy()
        np.testing.assert_array_equal(got, gss_ref.sample_scale_tiles(w, width))


def test_refinement_closed_forms():
    from exl3_intel_arc_quantizer_amd.gss import FINE_STEP, MIN_SCALE, select_refined_scale
    fine = [0.5 + FINE_STEP * (i - 2) for i in range(5)]
    # A sampled parabola: the step lands on its vertex.
    for vertex in (0.47, 0.5, 0.52):
        ms = [(s - vertex) ** 2 + 0.3 for s in fine]
        assert select_refined_scale(fine, ms) == pytest.approx(vertex, abs=1e-12)
        assert gss_ref.select_refined_scale(fine, ms) == pytest.approx(vertex, abs=1e-12)
    # Ties walk to the first (left) point; the floor applies below 0.01.
    low = [-0.14 + FINE_STEP * i for i in range(5)]
    assert select_refined_scale(low, [0.0] * 5) == MIN_SCALE
    assert select_refined_scale(fine, [1.0] * 5) == fine[0]
    # A minimum at the edge is not refined. An interior minimum tied with its
    # right neighbour gives the largest shift, exactly half a step.
    assert select_refined_scale(fine, [5, 4, 3, 2, 1]) == fine[4]
    assert select_refined_scale(fine, [9, 1.0, 1.0, 9, 9]) == pytest.approx(
        fine[1] + 0.5 * FINE_STEP, abs=1e-12)
    rng = np.random.default_rng(3)
    for _ in range(200):
        ms = rng.random(5).tolist()
        assert select_refined_scale(fine, ms) == gss_ref.select_refined_scale(fine, ms)


def test_oracle_search_finds_brute_force_minimum():
    w = _weight(128, 128, seed=4, scale=0.6)
    tiles = gss_ref.sample_scale_tiles(w, 3)
    (scale, mse), = gss_ref.g_scale_search([tiles], _grid_np)
    dense = np.arange(0.05, 2.0, 0.005)
    curve = [gss_ref._mse(tiles, s, _grid_np) for s in dense]
    assert abs(scale - dense[int(np.argmin(curve))]) <= gss_ref.FINE_STEP
    assert mse <= gss_ref._mse(tiles, 1.0, _grid_np)


def test_torch_search_matches_oracle_and_ignores_batching():
    from exl3_intel_arc_quantizer_amd.gss import g_scale_gss, g_scale_search_batch, \
        sample_scale_tiles
    ws = [_weight(128, 128, seed=5, scale=0.6), _weight(64, 256, seed=6, scale=2.5),
          _weight(256, 64, seed=7, scale=0.1)]
    samples = [sample_scale_tiles(torch.from_numpy(w)) for w in ws]
    want = gss_ref.g_scale_search([s.numpy() for s in samples], _grid_np)
    got = g_scale_search_batch(samples, _grid_torch)
    for (gs, gm), (ws_, wm) in zip(got, want):
        assert gs == pytest.approx(ws_, abs=1e-6)
        assert gm == pytest.approx(wm, rel=1e-5)
    assert g_scale_search_batch(samples, _grid_torch, max_tiles=40) == got
    assert [g_scale_search_batch([s], _grid_torch)[0] for s in samples] == got
    assert g_scale_gss(torch.from_numpy(ws[0]), _grid_torch) == got[0]
    assert g_scale_search_batch([], _grid_torch) == []
    with pytest.raises(ValueError):
        g_scale_search_batch([torch.zeros(4, 128)], _grid_torch)
