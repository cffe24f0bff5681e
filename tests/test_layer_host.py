"""Host-side pieces of the layer driver (exl3_intel_arc_quantizer_amd/
layer_quant.py) on CPU tensors."""

from __future__ import annotations

import pytest
import torch


@pytest.mark.parametrize("n,block", [(64, 16), (300, 128), (1100, 256), (1100, 4096)])
def test_factorization_residual_matches_full_product(n, block):
    """The row-blocked residual (layer_quant.py:95-101) over a lower
    triangular factor equals ||H - L L^T||_F / ||H||_F computed with the
    full product, for a factor perturbed well above rounding level."""
    from exl3_intel_arc_quantizer_amd.layer_quant import compute_factorization_residual
    g = torch.Generator().manual_seed(n)
    X = torch.randn(n + 10, n, generator=g, dtype=torch.float64)
    H = (X.T @ X) / n + 0.1 * torch.eye(n, dtype=torch.float64)
    L = torch.linalg.cholesky(H)
    L += torch.tril(torch.randn(n, n, generator=g, dtype=torch.float64)) * 1e-4
    H32, L32 = H.float(), L.float()
    got = compute_factorization_residual(H32, L32, block_rows=block)
    want = float(torch.linalg.norm(H - L @ L.T) / torch.linalg.norm(H))
    assert got == pytest.approx(want, rel=1e-4)
