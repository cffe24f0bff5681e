"""Synthetic inputs of the configs[2] sweep matrix and of the two layer
workloads, built the same way by the fixture script
(tests/golden/make_layer_fixture.py, on the CPU), the full-size GPU tests and
bench.py.

a 4096 x 4096 N(0, 1) matrix, numpy seed 2, with a seeded 1 % of
the entries scaled x4, rounded to fp16, cut into 65,536 tensor-core-order
tiles (16-row blocks, ldlq.py:276-281).

W ~ N(0, 0.02^2) of shape (4096 out, 4096 in), numpy seed 3;
activations X [8192, 4096] N(0, 1), numpy seed 4, with a seeded 5 % of the
channels (205) scaled x10, rounded to bf16; H = X^T X / 8192 evaluated in
float64 from the bf16 values and rounded once to float32, then the diagonal
damped by 1 % of its mean (calibration.py:370-377). Products of two bf16
values are exact in float64, so the CPU and the GPU evaluation of H differ
only in the float64 summation order, far below one float32 rounding step.
"""

from __future__ import annotations

import numpy as np

C3_K = 4
C3_OUT = 4096
C3_IN = 4096
C3_TOKENS = 8192
C3_W_SEED = 3
C3_X_SEED = 4
OUTLIER_FRACTION = 0.05
DAMPING = 0.01


def configs2_tiles() -> np.ndarray:
    """The 65,536 (256-value) tiles of the configs[2] matrix."""
    rng = np.random.default_rng(2)
    W = rng.standard_normal((4096, 4096), dtype=np.float32)
    W = np.where(rng.random(W.shape) < 0.01, 4.0 * W, W)
    W = W.astype(np.float16).astype(np.float32)
    return W.reshape(256, 16, 256, 16).transpose(0, 2, 1, 3).reshape(65536, 256)


def synthetic_activations(rng: np.random.Generator, tokens: int, width: int,
                          outlier_frac: float = OUTLIER_FRACTION) -> np.ndarray:
    """float32 N(0, 1) activations with round(outlier_frac * width) seeded
    channels scaled x10 (the same draw order as bench.py)."""
    X = rng.standard_normal((tokens, width), dtype=np.float32)
    chans = rng.choice(width, size=int(round(outlier_frac * width)), replace=False)
    X[:, chans] *= 10.0
    return X


def configs3_weight() -> np.ndarray:
    """(out, in) float32 weight of configs[3]."""
    rng = np.random.default_rng(C3_W_SEED)
    return rng.standard_normal((C3_OUT, C3_IN), dtype=np.float32) * np.float32(0.02)


def configs3_activations_bf16():
    """configs[3]'s activations as a CPU bf16 torch tensor [8192, 4096]."""
    import torch
    X = synthetic_activations(np.random.default_rng(C3_X_SEED), C3_TOKENS, C3_IN)
    return torch.from_numpy(X).to(torch.bfloat16)


def damp_hessian(H32):
    """H += max(1e-8, 0.01 * mean(diag H)) on the diagonal, in float32, in
    place (numpy array or torch tensor); returns the damping value."""
    if isinstance(H32, np.ndarray):
        d = np.diagonal(H32)
        damp = max(1e-8, DAMPING * float(d.mean(dtype=np.float64)))
        H32[np.diag_indices(H32.shape[0])] += np.float32(damp)
        return damp
    d = H32.diagonal()
    damp = max(1e-8, DAMPING * float(d.double().mean().item()))
    d.add_(float(np.float32(damp)))
    return damp


def configs3_hessian_cpu() -> tuple:
    """(H float32 numpy, damping) evaluated on the CPU."""
    import torch
    Xb = configs3_activations_bf16().to(torch.float64).numpy()
    H = (Xb.T @ Xb / float(C3_TOKENS)).astype(np.float32)
    damp = damp_hessian(H)
    return H, damp


def configs3_hessian_gpu(device: str = "cuda") -> tuple:
    """(H float32 torch tensor on ``device``, damping), the same evaluation
    as configs3_hessian_cpu with the float64 product on the GPU."""
    import torch
    Xb = configs3_activations_bf16().to(device).to(torch.float64)
    H = (Xb.T @ Xb / float(C3_TOKENS)).to(torch.float32)
    del Xb
    damp = damp_hessian(H)
    return H, damp
