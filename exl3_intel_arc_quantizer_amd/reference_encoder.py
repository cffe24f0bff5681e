"""Result record and constants shared with the reference's encoder module.

Counterpart of exl3_quant/reference_encoder.py:44-59 (``H_INF``,
``EncodingResult``). The reference's CPU golden encoder
(``ReferenceTrellisEncoder``) is deliberately not part of this package: it is
the parity oracle and lives under ``oracle/`` with the tests, so that no
product path can fall back to it.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .trellis_format import CB_3INST, CB_MCG, CB_MUL1  # noqa: F401  (re-export)

H_INF = np.uint16(0x7C00).view(np.float16)


@dataclass
class EncodingResult:
    """Per-tile encoder output, field for field as reference_encoder.py:47-59."""

    output_indices: np.ndarray        # (L,) uint16 16-bit states, kernel (tensor-core) order
    reconstructed: np.ndarray         # (L,) float16 reconstruction, original tile order
    reconstructed_perm: np.ndarray    # (L,) float16 reconstruction, kernel order
    packed: np.ndarray                # (16K,) uint16 storage words after SWAP16 (L = 256)
    end_state: int                    # tail-biting wrap edge
    distortion: float                 # sum((w - w_hat)^2), float32
    mse: float                        # distortion / L
    path_cost: float                  # fp16 path cost of the chosen trajectory
    K: int
    cb: int
