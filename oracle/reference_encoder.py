"""numpy restatement of ``ReferenceTrellisEncoder`` — TEST INFRASTRUCTURE ONLY.

Follows exl3_quant/reference_encoder.py of the reference op for op where the
fp16 semantics matter; same class, method and field names so the parity tests
read like the reference's own tests. Never imported by the product package.

fp16 semantics restated (reference_encoder.py:152-202):

* ``dh = fp16(val - w)``: numpy's fp16 subtraction (computed in float32 and
  rounded once; exact by the 2p+2 rule);
* step 0: ``err = fp16(dh*dh)``, masked to +inf where ``pred != pre_state``
  when a wrap constraint is given;
* steps 1..L-1: ``err = fp16(dh*dh + cost_prev[pred])`` evaluated exactly in
  float64 and rounded once (a fused multiply-add);
* per edge, branch ``k = 0`` initialises unconditionally and a later branch
  replaces the running minimum only when strictly smaller (so ties keep the
  lowest ``k`` and a NaN at ``k = 0`` sticks);
* terminal argmin: lowest index of the minimum, 0 when no cost is finite or
  every cost is +inf (reference_encoder.py:206-214).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .trellis_format_ref import (
    CB_3INST,
    CB_MCG,
    CB_MUL1,
    codebook_lut,
    pack_trellis,
    swap16_storage,
    tensor_core_perm,
    tensor_core_perm_inv,
)

H_INF = np.uint16(0x7C00).view(np.float16)


@dataclass
class EncodingResult:
    """Field-for-field restatement of reference_encoder.py:47-59."""

    output_indices: np.ndarray
    reconstructed: np.ndarray
    reconstructed_perm: np.ndarray
    packed: np.ndarray
    end_state: int
    distortion: float
    mse: float
    path_cost: float
    K: int
    cb: int


class ReferenceTrellisEncoder:
    """CPU golden encoder (reference_encoder.py:62-350)."""

    def __init__(self, K: int = 2, cb: int = CB_MUL1, tile_len: int = 256):
        if not 1 <= K <= 8:
            raise ValueError(f"K must be between 1 and 8, got {K}")
        if cb not in (CB_3INST, CB_MCG, CB_MUL1):
            raise ValueError(f"Unknown codebook {cb}")
        if tile_len <= 0 or tile_len % 2:
            raise ValueError(f"tile_len must be positive even integer, got {tile_len}")
        self.K, self.cb, self.L = K, cb, tile_len
        self.Kr = 16 - K
        self.max_q = 1 << K
        self.edges = 65536 >> K
        self.lut = codebook_lut(cb)
        # Candidate tables (reference_encoder.py:99-113): branch k of edge e is
        # the state sigma = (k << Kr) | e, whose predecessor edge is sigma >> K.
        k = np.arange(self.max_q, dtype=np.uint32)[:, None]
        e = np.arange(self.edges, dtype=np.uint32)[None, :]
        sigma = (k << np.uint32(self.Kr)) | e
        self.k_states = sigma.astype(np.uint16)
        self.k_preds = (sigma >> np.uint32(K)).astype(np.uint16)
        self.k_vals = self.lut[self.k_states]
        if tile_len == 256:
            self.perm, self.inv_perm = tensor_core_perm(), tensor_core_perm_inv()
        else:
            self.perm = self.inv_perm = None

    @staticmethod
    def ring(i: int, roll: int, L: int = 256) -> int:
        """Ring index (reference_encoder.py:122-128)."""
        return i + roll - L if i + roll >= L else i + roll

    def forward(self, input_tile, roll: int, pre_state: int, temp_edges) -> np.ndarray:
        """Add-compare-select over the ring (reference_encoder.py:130-204)."""
        prev_cost = None
        for i in range(self.L):
            ri = self.ring(i, roll, self.L)
            w = input_tile[ri]
            best_cost = best_pred = None
            for k in range(self.max_q):
                pred = self.k_preds[k]
                dh = (self.k_vals[k] - w).astype(np.float64)          # fp16 subtract
                if prev_cost is None:
                    err = (dh * dh).astype(np.float16)
                    if pre_state >= 0:
                        err = np.where(pred != pre_state, H_INF, err)
                else:
                    err = (dh * dh + prev_cost[pred].astype(np.float64)).astype(np.float16)
                if best_cost is None:
                    best_cost, best_pred = err.copy(), pred.copy()
                else:
                    better = err < best_cost
                    best_cost[better] = err[better]
                    best_pred[better] = pred[better]
            temp_edges[ri] = best_pred
            prev_cost = best_cost
        return prev_cost

    def argmin_cost(self, costs: np.ndarray) -> int:
        """Terminal edge (reference_encoder.py:206-214)."""
        if not np.isfinite(costs).any() or (costs == H_INF).all():
            return 0
        return int(np.argmin(costs))

    def backward(self, temp_edges, roll: int, write: bool, edge: int):
        """Traceback (reference_encoder.py:216-251)."""
        idx = np.zeros(self.L, dtype=np.uint16)
        tile = np.zeros(self.L, dtype=np.float16)
        for i in range(self.L - 1, -1, -1):
            ri = self.ring(i, roll, self.L)
            prev = int(temp_edges[ri, edge])
            state = (prev << self.K) | edge
            edge = prev
            if write:
                idx[ri] = state
                tile[ri] = self.lut[state]
            elif ri == 0:
                break
        return edge, idx, tile

    def encode_tile(self, tile, pre_permute: bool = True) -> EncodingResult:
        """Two-pass tail-biting encode (reference_encoder.py:253-324)."""
        raw = np.asarray(tile, dtype=np.float32).reshape(-1)
        if raw.size != self.L:
            raise ValueError(f"Tile must have {self.L} elements, got {raw.size}")
        if pre_permute:
            if self.perm is None:
                raise ValueError("tensor_core_perm is defined only for tile_len=256")
            x16 = raw[self.perm].astype(np.float16)
        else:
            x16 = raw.astype(np.float16)

        edges = np.zeros((self.L, self.edges), dtype=np.uint16)
        c1 = self.forward(x16, roll=self.L // 2, pre_state=-1, temp_edges=edges)
        end_state, _, _ = self.backward(edges, self.L // 2, False, self.argmin_cost(c1))
        c2 = self.forward(x16, roll=0, pre_state=end_state, temp_edges=edges)
        _, idx, rec_perm = self.backward(edges, 0, True, end_state)

        packed = (swap16_storage(pack_trellis(idx, self.K)) if self.L == 256
                  else np.array([], dtype=np.uint16))
        if pre_permute:
            rec, orig = rec_perm[self.inv_perm], raw
        else:
            rec, orig = rec_perm, x16.astype(np.float32)
        distortion = float(np.sum((orig - rec.astype(np.float32)) ** 2))
        return EncodingResult(
            output_indices=idx, reconstructed=rec, reconstructed_perm=rec_perm,
            packed=packed, end_state=end_state, distortion=distortion,
            mse=distortion / float(self.L), path_cost=float(c2[end_state]),
            K=self.K, cb=self.cb)

    def encode_batch(self, tiles, pre_permute: bool = True):
        """Per-tile loop (reference_encoder.py:326-350)."""
        arr = np.asarray(tiles, dtype=np.float32)
        if arr.ndim not in (2, 3):
            raise ValueError(f"Expected 2D or 3D array of tiles, got shape {arr.shape}")
        flat = arr.reshape(arr.shape[0], -1)
        return [self.encode_tile(t, pre_permute=pre_permute) for t in flat]
