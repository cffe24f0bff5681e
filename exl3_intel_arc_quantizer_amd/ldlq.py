"""Block LDL factorisation and the LDLQ error-feedback traversal on the GPU
(reference: exl3_quant/ldlq.py).

``block_ldl`` factors the (Hadamard-rotated, damped) Hessian H = L L^T with
rocSOLVER (``torch.linalg.cholesky``), inverts every 16x16 diagonal block in
one batched call and folds the inverses into their block columns with one
batched GEMM; the diagonal blocks become identities.

``ldlq`` quantises a (k, n) weight bottom-up: spans of ``buf_size_k`` rows
from the last, 16-row blocks inside a span from the last. Each block's rows
get the compensation of the rows already quantised below it in the span
(``addmm`` against the strictly lower slice of L) plus the span-level
feedback ``prod_cache``; the 16 x n rows become n / 16 tiles in tensor-core
order, go through the tile encoder (the HIP encoder, tiles staying in HBM),
and the reconstruction is un-permuted into ``weight_q`` while the states stay
in tensor-core order. After a span its residual is propagated into
``prod_cache`` for the spans above. All of it runs on the weight's device.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable

import torch

from .tile_encoder import TileEncoder, make_gpu_tile_encoder, make_xpu_tile_encoder
from .trellis_format import tensor_core_perm, tensor_core_perm_inv

DEFAULT_BLOCK_SIZE = 16
DEFAULT_SIGMA_REG = 0.025
DEFAULT_MAX_RETRIES = 10
DEFAULT_BUF_SIZE_K = 128

__all__ = ["DEFAULT_BLOCK_SIZE", "DEFAULT_SIGMA_REG", "DEFAULT_MAX_RETRIES", "DEFAULT_BUF_SIZE_K",
           "BlockLDLResult", "block_ldl", "LDLQResult", "ldlq", "TileEncoder",
           "make_xpu_tile_encoder", "make_gpu_tile_encoder"]


@dataclass(frozen=True)
class BlockLDLResult:
    """Folded factor and intermediates (ldlq.py:45-56)."""

    transformed: torch.Tensor
    cholesky: torch.Tensor
    block_inverses: torch.Tensor
    retries: int
    damping_applied: bool
    n: int
    block_size: int


def block_ldl(H: torch.Tensor, block_size: int = DEFAULT_BLOCK_SIZE,
              sigma_reg: float = DEFAULT_SIGMA_REG,
              max_retries: int = DEFAULT_MAX_RETRIES) -> BlockLDLResult:
    """Block-folded Cholesky factor consumed by :func:`ldlq` (ldlq.py:76-142).
    ``H`` is not modified; after a failed factorisation an internal copy is
    damped by 2 sigma_reg mean(diag) and factored again, up to
    ``max_retries`` times."""
    if H.dim() != 2 or H.shape[0] != H.shape[1]:
        raise ValueError(f"H must be a square 2-D tensor, got shape {tuple(H.shape)}")
    if H.dtype != torch.float32:
        raise ValueError(f"block_ldl requires float32, got {H.dtype}")
    if block_size <= 0 or block_size > H.shape[0] or H.shape[0] % block_size:
        raise ValueError(f"block_size {block_size} must be positive and divide {H.shape[0]}")
    if max_retries < 0:
        raise ValueError(f"max_retries must be non-negative, got {max_retries}")
    n = H.shape[0]
    work = H.clone()
    chol = None
    retries = 0
    for attempt in range(max_retries + 1):
        chol, info = torch.linalg.cholesky_ex(work)
        if int(info.item()) == 0:
            retries = attempt
            break
        if attempt == max_retries:
            raise torch.linalg.LinAlgError(
                f"block_ldl: Cholesky failed after {max_retries} damping steps")
        work.diagonal().add_(2.0 * sigma_reg * work.diagonal().mean())
    m = n // block_size
    # (m, bs, bs) diagonal blocks, inverted in one batched call.
    diag_blocks = torch.stack([chol[b * block_size:(b + 1) * block_size,
                                    b * block_size:(b + 1) * block_size] for b in range(m)])
    inverses = torch.linalg.inv(diag_blocks.contiguous())
    # Column block b of the factor times its inverse: one batched GEMM.
    cols = chol.view(n, m, block_size).permute(1, 0, 2).contiguous()      # (m, n, bs)
    folded = torch.matmul(cols, inverses.contiguous())                      # (m, n, bs)
    transformed = folded.permute(1, 0, 2).reshape(n, n).contiguous()
    eye = torch.eye(block_size, dtype=H.dtype, device=H.device)
    for b in range(m):
        transformed[b * block_size:(b + 1) * block_size,
                    b * block_size:(b + 1) * block_size] = eye
    return BlockLDLResult(transformed=transformed, cholesky=chol, block_inverses=inverses,
                          retries=retries, damping_applied=retries > 0, n=n,
                          block_size=block_size)


@dataclass
class LDLQResult:
    """Quantised layer and its trellis states (ldlq.py:150-158)."""

    weight_q: torch.Tensor
    encoded: torch.Tensor
    tiles_k: int
    tiles_n: int
    buf_size_k: int
    encoder_seconds: float = 0.0
    encoder_calls: int = 0
    timings: dict = field(default_factory=dict)


def _as_int16_states(indices: torch.Tensor) -> torch.Tensor:
    """16-bit states in a signed int16 container, bit pattern kept (ldlq.py:147-160)."""
    if indices.dtype == torch.int16:
        return indices
    values = indices.to(torch.int64) & 0xFFFF
    return torch.where(values >= 0x8000, values - 0x10000, values).to(torch.int16)


def ldlq(weight: torch.Tensor, L: torch.Tensor, encode_tiles: TileEncoder,
         buf_size_k: int = DEFAULT_BUF_SIZE_K,
         synchronize: Callable[[], None] = None) -> LDLQResult:
    """Bottom-up one-sided LDLQ (ldlq.py:163-309). ``weight`` (k, n) float32
    in the transformed basis and ``L`` (k, k) from :func:`block_ldl` are not
    modified. ``encode_tiles`` maps (tiles_n, 256) tensor-core-order tiles to
    (reconstruction, int16 states).

    ``encoder_seconds`` is the encoder's share: on a CUDA weight, the sum of
    HIP-event intervals around each call on the current stream, read once
    after the traversal, so nothing in the loop waits for the device; with
    ``synchronize`` given, host wall time between two ``synchronize()``
    calls around each call instead. An encoder exposing ``check_finite``
    (the HIP adapter) is asked once at the end to raise on NaN inputs."""
    if weight.dim() != 2 or weight.dtype != torch.float32:
        raise ValueError(f"weight must be a 2-D float32 tensor, got {weight.dtype} "
                         f"{tuple(weight.shape)}")
    k, n = weight.shape
    if k % 16 != 0:
        raise ValueError(f"rows ({k}) must be a multiple of 16")
    if n % 128 != 0:
        raise ValueError(f"columns ({n}) must be a multiple of 128")
    if L.dim() != 2 or tuple(L.shape) != (k, k) or L.dtype != torch.float32:
        raise ValueError(f"L must be a float32 ({k}, {k}) tensor, got {L.dtype} {tuple(L.shape)}")
    if L.device != weight.device:
        raise ValueError(f"L and weight must be on the same device, got {L.device} / {weight.device}")
    buf_size_k = int(buf_size_k)
    if buf_size_k < 16 or buf_size_k % 16 != 0:
        raise ValueError(f"buf_size_k must be a positive multiple of 16, got {buf_size_k}")
    if n % buf_size_k != 0 or k % buf_size_k != 0:
        raise ValueError(f"rows ({k}) and columns ({n}) must be divisible by buf_size_k "
                         f"({buf_size_k})")

    device = weight.device
    tiles_k, tiles_n = k // 16, n // 16
    perm = torch.as_tensor(tensor_core_perm(), dtype=torch.long, device=device)
    inv_perm = torch.as_tensor(tensor_core_perm_inv(), dtype=torch.long, device=device)
    prod_cache = torch.zeros((k, n), dtype=torch.float32, device=device)
    weight_q = torch.zeros((k, n), dtype=torch.float32, device=device)
    encoded = torch.zeros((tiles_k, tiles_n, 256), dtype=torch.int16, device=device)
    enc_s = 0.0
    calls = 0
    use_events = synchronize is None and device.type == "cuda"
    events = []

    for j in range(k, 0, -buf_size_k):
        i = j - buf_size_k
        for bj in range(buf_size_k, 0, -16):
            bi = bj - 16
            r0, r1 = i + bi, i + bj           # the 16 rows being quantised
            comp = prod_cache[r0:r1]
            if r1 < j:
                # Rows already quantised below, within this span.
                err = weight[r1:j] - weight_q[r1:j]
                comp.addmm_(L[r1:j, r0:r1].T, err, alpha=1.0, beta=1.0)
            rows = weight[r0:r1] + comp
            tiles = rows.reshape(16, tiles_n, 16).permute(1, 0, 2).reshape(tiles_n, 256)
            tiles = tiles[:, perm].contiguous()
            if use_events:
                ev0 = torch.cuda.Event(enable_timing=True)
                ev0.record()
            elif synchronize is not None:
                synchronize()
            t0 = time.perf_counter()
            quant_w, quant_i = encode_tiles(tiles)
            if use_events:
                ev1 = torch.cuda.Event(enable_timing=True)
                ev1.record()
                events.append((ev0, ev1))
            else:
                if synchronize is not None:
                    synchronize()
                enc_s += time.perf_counter() - t0
            calls += 1
            if tuple(quant_w.shape) != (tiles_n, 256) or tuple(quant_i.shape) != (tiles_n, 256):
                raise ValueError("encode_tiles must return two (tiles_n, 256) tensors, got "
                                 f"{tuple(quant_w.shape)} / {tuple(quant_i.shape)}")
            quant_w = quant_w.to(device=device, dtype=torch.float32)[:, inv_perm]
            weight_q[r0:r1] = quant_w.reshape(tiles_n, 16, 16).permute(1, 0, 2).reshape(16, n)
            encoded[r0 // 16] = _as_int16_states(quant_i.to(device=device))
        # Span residual into the feedback of the spans above.
        prod_cache.addmm_(L[i:j].T, weight[i:j] - weight_q[i:j], alpha=1.0, beta=1.0)

    if events:
        events[-1][1].synchronize()
        enc_s = sum(a.elapsed_time(b) for a, b in events) / 1e3
    check_finite = getattr(encode_tiles, "check_finite", None)
    if check_finite is not None:
        check_finite()
    return LDLQResult(weight_q=weight_q, encoded=encoded, tiles_k=tiles_k, tiles_n=tiles_n,
                      buf_size_k=buf_size_k, encoder_seconds=enc_s, encoder_calls=calls)
