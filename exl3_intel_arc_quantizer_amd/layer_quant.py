"""Linear-layer and decoder-layer quantisation driver on the GPU
(reference: exl3_quant/layer_quant.py, calibration.py:242-407).

``quantize_linear_module`` runs one projection through the EXL3 pipeline:
regularise the weight (scales, blockwise Hadamard), rotate the Hessian with
the same transforms, factor it (``block_ldl``), quantise with LDLQ error
feedback through the HIP tile encoder, map the reconstruction back to the
original basis and report the distortion and Hessian proxy metrics.
``quantize_decoder_layer`` does every bias-free ``nn.Linear`` of a layer
with one shared encoder and scratch arena. Everything stays on the GPU; the
encoder is the only consumer of the trellis kernels and there is no CPU
fallback.

``hessian_from_activations`` and ``hessian_groups`` restate the reference's
calibration: H = X^T X / tokens in float32, plus lambda * mean(diag H) on
the diagonal and a floor on inactive channels; projections that read the
same input share one Hessian.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from .hadamard import HAD_DIM, blockwise_preapply_had_l_, blockwise_preapply_had_r_, \
    weight_from_quantized
from .ldlq import (DEFAULT_BLOCK_SIZE, DEFAULT_BUF_SIZE_K, BlockLDLResult, LDLQResult,
                   block_ldl, ldlq, ldlq_lockstep)
from .gss import g_scale_fn_from_encoder
from .regularize import RegularizeResult, regularize
from .tile_encoder import TileEncoder, make_xpu_tile_encoder
from .trellis_format import CB_MUL1

DEFAULT_DAMPING_LAMBDA = 0.01        # calibration.py:43
DEFAULT_ZERO_CHANNEL_FLOOR = 1e-7    # calibration.py:44


# ------------------------------------------------------------------ Hessians

def hessian_from_activations(x: torch.Tensor, damping_lambda: float = DEFAULT_DAMPING_LAMBDA,
                             zero_floor: float = DEFAULT_ZERO_CHANNEL_FLOOR,
                             chunk_tokens: int = 8192) -> Tuple[torch.Tensor, float]:
    """Hessian of one projection input: sum over token chunks of X^T X in
    float32 (calibration.py:337-352), divided by the token count, diagonal
    damped by lambda * mean(diag) and floored at ``zero_floor``
    (calibration.py:359-385). Returns (H, applied damping).

    bf16 / fp16 activations on the GPU go straight into a half-precision
    GEMM with float32 output (``torch.mm(..., out_dtype=float32)``, MFMA
    with fp32 accumulation): their products are exact in float32, so the
    result is the float32 GEMM of the converted values up to summation
    order, without the conversion pass and at the half-precision MFMA
    rate."""
    d = x.shape[-1]
    flat = x.reshape(-1, d)
    H = torch.zeros((d, d), dtype=torch.float32, device=x.device)
    half = flat.device.type == "cuda" and flat.dtype in (torch.bfloat16, torch.float16)
    for s in range(0, flat.shape[0], chunk_tokens):
        if half:
            xc = flat[s:s + chunk_tokens]
            H += torch.mm(xc.T, xc, out_dtype=torch.float32)
        else:
            xf = flat[s:s + chunk_tokens].to(torch.float32)
            H += xf.T @ xf
    H /= max(1, flat.shape[0])
    diag = H.diagonal()
    damp = max(1e-8, damping_lambda * diag.mean().item())
    diag.add_(damp)
    floor = torch.as_tensor(zero_floor, dtype=diag.dtype, device=diag.device)
    diag.copy_(torch.where(diag.abs() < zero_floor, floor, diag))
    return H, damp


def hessian_groups(module_names: List[str]) -> Dict[str, List[str]]:
    """Projections that read the same input share one Hessian
    (calibration.py:242-289): q/k/v, the GatedDeltaNet input projections,
    gate/up; every other projection is its own group."""
    groups: Dict[str, List[str]] = {}
    for key, members in (("self_attn.input", ("self_attn.q_proj", "self_attn.k_proj",
                                              "self_attn.v_proj")),
                         ("self_attn.o_proj", ("self_attn.o_proj",)),
                         ("linear_attn.input", ("linear_attn.in_proj_qkv",
                                                "linear_attn.in_proj_z",
                                                "linear_attn.in_proj_b",
                                                "linear_attn.in_proj_a")),
                         ("linear_attn.out_proj", ("linear_attn.out_proj",)),
                         ("mlp.input", ("mlp.gate_proj", "mlp.up_proj")),
                         ("mlp.down_proj", ("mlp.down_proj",))):
        present = [m for m in members if m in module_names]
        if present:
            groups[key] = present
    assigned = {m for ms in groups.values() for m in ms}
    for name in module_names:
        if name not in assigned:
            groups[name] = [name]
    return groups


# ------------------------------------------------------------------- results

@dataclass
class ModuleMetrics:
    """Distortion and proxy metrics of one quantised projection (layer_quant.py:49-60)."""

    mse: float
    relative_frobenius_error: float
    tile_distortion: float
    proxy_loss: float
    normalized_proxy_loss: float
    factorization_residual: float
    retries: int
    g_scale: float
    elapsed_seconds: float
    encoder_seconds: float = 0.0
    encoder_calls: int = 0


@dataclass
class QuantizedModuleResult:
    """Outputs of a quantised projection (layer_quant.py:63-77)."""

    name: str
    K: int
    cb: int
    original_shape: Tuple[int, int]
    weight_orig: torch.Tensor
    w_hat: torch.Tensor
    encoded: torch.Tensor
    su: torch.Tensor
    sv: torch.Tensor
    metrics: ModuleMetrics
    regularize_result: RegularizeResult
    ldl_result: BlockLDLResult


@dataclass
class LayerQuantizationReport:
    """Report of a decoder-layer conversion (layer_quant.py:80-92)."""

    K: int
    codebook: str
    total_elapsed_seconds: float
    module_results: Dict[str, QuantizedModuleResult]
    total_proxy_loss: float
    mean_mse: float
    peak_device_memory_bytes: int
    scratch_arena_reused: bool
    device_index: int
    tiles: int = 0
    encoder_seconds: float = 0.0
    extra: dict = field(default_factory=dict)


def _factorization_residual_parts(H: torch.Tensor, chol: torch.Tensor,
                                  block_rows: int = 1024) -> Tuple[torch.Tensor, torch.Tensor]:
    """(||H - L L^T||_F, ||H||_F) as device scalars, nothing read back."""
    n = H.shape[0]
    sq = torch.zeros((), dtype=torch.float64, device=H.device)
    for i0 in range(0, n, block_rows):
        i1 = min(n, i0 + block_rows)
        diff = H[i0:i1] - chol[i0:i1, :i1] @ chol[:, :i1].T
        sq += diff.square().sum(dtype=torch.float64)
    return sq.sqrt(), torch.linalg.norm(H)


def compute_factorization_residual(H: torch.Tensor, chol: torch.Tensor,
                                   block_rows: int = 1024) -> float:
    """||H - L L^T||_F / ||H||_F (layer_quant.py:95-101) for a lower
    triangular L. Row block [i0, i1) of L L^T is L[i0:i1, :i1] @ L[:, :i1]^T
    (the rows' entries past column i1 are zero), so the blocks together
    take about half the flops of the full product; each block's squared
    residual is summed in float64."""
    res, norm = _factorization_residual_parts(H, chol, block_rows)
    return float(res.item() / max(1e-12, norm.item()))


def _proxy_parts(W: torch.Tensor, W_hat: torch.Tensor,
                 H: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(tr(E^T H E), tr(W^T H W)) as float32 device scalars, E = W - W_hat."""
    E = (W - W_hat).to(dtype=torch.float32, device=H.device)
    H32 = H.to(torch.float32)
    W32 = W.to(dtype=torch.float32, device=H.device)
    return ((H32 @ E) * E).sum(), ((H32 @ W32) * W32).sum()


def compute_proxy_loss(W: torch.Tensor, W_hat: torch.Tensor,
                       H: torch.Tensor) -> Tuple[float, float]:
    """tr(E^T H E) as sum((H E) * E), E = W - W_hat, and its ratio to
    tr(W^T H W) (layer_quant.py:104-127)."""
    proxy_t, energy_t = _proxy_parts(W, W_hat, H)
    proxy, energy = torch.stack([proxy_t, energy_t]).tolist()
    return proxy, proxy / max(1e-12, energy)


# -------------------------------------------------------------------- driver

@dataclass
class _PreparedModule:
    """A projection between regularisation and LDLQ."""

    name: str
    W: torch.Tensor            # (k, n) float32, original basis
    H: torch.Tensor
    reg: RegularizeResult
    ldl: BlockLDLResult
    fact_parts: Tuple[torch.Tensor, torch.Tensor]  # read back with the module's metrics
    prep_seconds: float


def _prepare_module(name: str, weight: torch.Tensor, H: torch.Tensor, K: int, cb: int,
                    tile_encoder: TileEncoder, skip_g_scale: bool, block_size: int,
                    ldl_cache: Optional[dict] = None) -> _PreparedModule:
    """Shape checks, regularisation (with the global-scale search unless
    ``skip_g_scale``), Hessian rotation and block LDL (layer_quant.py:130-214).
    The rotation and factor depend on H alone: with ``ldl_cache``,
    projections given the same Hessian tensor share one factorisation."""
    t0 = time.time()
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2D, got shape {tuple(weight.shape)}")
    device = H.device
    if device.type != "cuda":
        raise ValueError("quantize_linear_module runs on the GPU; move H to a cuda device")
    k_dim = H.shape[0]
    if weight.shape[1] == k_dim:
        W = weight.T.to(device=device, dtype=torch.float32).contiguous()
    elif weight.shape[0] == k_dim:
        W = weight.to(device=device, dtype=torch.float32).clone()
    else:
        raise ValueError(f"Weight shape {tuple(weight.shape)} does not match Hessian dim {k_dim}")
    k, n = W.shape
    enc_k = getattr(tile_encoder, "K", None)
    if enc_k is not None and enc_k != K:
        raise ValueError(f"Tile encoder K={enc_k} does not match the requested K={K}.")
    # The result (and its exported codebook marker) carries cb, so an encoder
    # of another codebook would label its states wrongly.
    enc_cb = getattr(tile_encoder, "cb", None)
    if enc_cb is not None and enc_cb != cb:
        raise ValueError(f"Tile encoder cb={enc_cb} does not match the requested cb={cb}.")
    # Global scale from the same encoder (layer_quant.py:197-203).
    g_scale_fn = None if skip_g_scale else g_scale_fn_from_encoder(tile_encoder)

    su = torch.ones((k, 1), dtype=torch.float32, device=device)
    sv = torch.ones((1, n), dtype=torch.float32, device=device)
    reg = regularize(weight=W, su=su, sv=sv, H_diag=H.diagonal(), skip_g_scale=skip_g_scale,
                     g_scale_fn=g_scale_fn, had_dim=HAD_DIM)

    key = (id(H), block_size)
    cached = ldl_cache.get(key) if ldl_cache is not None else None
    if cached is not None and cached[0] is H:
        ldl, fact_parts = cached[1], cached[2]
    else:
        H_work = H.to(torch.float32).clone()
        blockwise_preapply_had_l_(H_work, HAD_DIM)
        blockwise_preapply_had_r_(H_work, HAD_DIM)
        ldl = block_ldl(H_work, block_size=block_size)
        fact_parts = _factorization_residual_parts(H_work, ldl.cholesky)
        if ldl_cache is not None:
            ldl_cache[key] = (H, ldl, fact_parts)   # keeps H alive: id stays unique
    return _PreparedModule(name=name, W=W, H=H, reg=reg, ldl=ldl, fact_parts=fact_parts,
                           prep_seconds=time.time() - t0)


def _apply_global_scales(prepared: List[_PreparedModule], tile_encoder: TileEncoder) -> None:
    """Global-scale search (gss.py:187-207) for several regularised
    projections in one batch, applied as regularize does after its own
    search (regularize.py:192-196): weight x g, su / g."""
    from .gss import g_scale_search_batch, sample_scale_tiles
    results = g_scale_search_batch([sample_scale_tiles(pm.reg.weight) for pm in prepared],
                                   tile_encoder)
    for pm, (g, _) in zip(prepared, results):
        g = float(g)
        if not g > 0.0:
            raise ValueError(f"global-scale search returned a non-positive scale: {g}")
        pm.reg.weight.mul_(g)
        pm.reg.su.div_(g)
        pm.reg.g_scale = g


def _finish_module(pm: _PreparedModule, lq: LDLQResult, K: int, cb: int,
                   shared_seconds: float) -> QuantizedModuleResult:
    """Back to the original basis and the metrics (layer_quant.py:216-265);
    ``elapsed_seconds`` = preparation + ``shared_seconds`` + this step."""
    t0 = time.time()
    W, reg = pm.W, pm.reg
    w_hat = weight_from_quantized(lq.weight_q, reg.su, reg.sv)
    diff = W - w_hat
    proxy_t, energy_t = _proxy_parts(W, w_hat, pm.H)
    # Every scalar of the module comes back in one device-to-host read
    # (float32 values widen to float64 exactly).
    (proxy, energy, mse, diff_norm, w_norm, tile_distortion, fact_res,
     h_norm) = torch.stack([t.to(torch.float64) for t in (
         proxy_t, energy_t, diff.pow(2).mean(), torch.linalg.norm(diff), torch.linalg.norm(W),
         (reg.weight - lq.weight_q).pow(2).mean(), *pm.fact_parts)]).tolist()
    metrics = ModuleMetrics(
        mse=mse,
        relative_frobenius_error=diff_norm / max(1e-12, w_norm),
        tile_distortion=tile_distortion,
        proxy_loss=proxy, normalized_proxy_loss=proxy / max(1e-12, energy),
        factorization_residual=fact_res / max(1e-12, h_norm), retries=pm.ldl.retries,
        g_scale=reg.g_scale,
        elapsed_seconds=pm.prep_seconds + shared_seconds + (time.time() - t0),
        encoder_seconds=lq.encoder_seconds, encoder_calls=lq.encoder_calls)
    return QuantizedModuleResult(name=pm.name, K=K, cb=cb, original_shape=tuple(W.shape),
                                 weight_orig=W, w_hat=w_hat, encoded=lq.encoded, su=reg.su,
                                 sv=reg.sv, metrics=metrics, regularize_result=reg,
                                 ldl_result=pm.ldl)


def quantize_linear_module(name: str, weight: torch.Tensor, H: torch.Tensor, K: int = 2,
                           cb: int = CB_MUL1, tile_encoder: Optional[TileEncoder] = None,
                           skip_g_scale: bool = True, buf_size_k: int = DEFAULT_BUF_SIZE_K,
                           block_size: int = DEFAULT_BLOCK_SIZE,
                           ldl_cache: Optional[dict] = None,
                           time_encoder: bool = False) -> QuantizedModuleResult:
    """Quantise one linear weight with LDLQ (layer_quant.py:130-265). The
    weight is (out, in) as in ``nn.Linear`` or already (in, out) = (k, n);
    ``H`` is (in, in). Runs on the device of ``H``, which must be a GPU. The
    default encoder uses codebook ``cb``; a given encoder must match K and
    cb. ``ldl_cache`` (a dict) lets calls that pass the same Hessian tensor
    share its factorisation. ``time_encoder`` measures
    ``metrics.encoder_seconds`` with HIP events around every encoder call,
    which costs a 4096 x 4096 layer about 3 % (0 is reported without it)."""
    if H.device.type != "cuda":
        raise ValueError("quantize_linear_module runs on the GPU; move H to a cuda device")
    if tile_encoder is None:
        tile_encoder = make_xpu_tile_encoder(K=K, device_index=H.device.index or 0, cb=cb)
    pm = _prepare_module(name, weight, H, K, cb, tile_encoder, skip_g_scale, block_size,
                         ldl_cache)
    t0 = time.time()
    lq = ldlq(weight=pm.reg.weight, L=pm.ldl.transformed, encode_tiles=tile_encoder,
              buf_size_k=buf_size_k, time_calls=time_encoder)
    return _finish_module(pm, lq, K, cb, time.time() - t0)


def quantize_decoder_layer(layer: torch.nn.Module, hessians: Dict[str, torch.Tensor], K: int = 2,
                           cb: int = CB_MUL1, device: Optional[torch.device] = None,
                           skip_g_scale: bool = True, buf_size_k: int = DEFAULT_BUF_SIZE_K,
                           block_size: int = DEFAULT_BLOCK_SIZE, memory_policy=None,
                           module_names: Optional[List[str]] = None,
                           lockstep: bool = True,
                           time_encoder: bool = False) -> LayerQuantizationReport:
    """Quantise every bias-free ``nn.Linear`` of a decoder layer (or the
    ``module_names`` subset) with one shared encoder and scratch arena
    (layer_quant.py:268-387).

    With ``lockstep`` (the default) the projections are prepared first and
    their LDLQ traversals run side by side (``ldlq_lockstep``): each encoder
    launch carries block b of every projection, e.g. 2176 tiles for
    q/k/v/o/gate/up of a 4096-wide layer instead of 64 to 768. The results
    equal the one-at-a-time order (``lockstep=False``, the reference's); a
    module's ``elapsed_seconds`` then includes the shared traversal and its
    ``encoder_seconds`` is its tile share of each call. Encoder time is
    measured only with ``time_encoder`` (HIP events around every call)."""
    from .gpu_quantizer import ScratchArena
    from .memory_policy import MemoryPolicy

    t_start = time.time()
    if device is None:
        device = torch.device("cuda:0")
    if device.type != "cuda":
        raise ValueError("quantize_decoder_layer runs on the GPU")
    policy = memory_policy or MemoryPolicy()
    arena = ScratchArena(device_index=device.index or 0, policy=policy)
    encoder = make_xpu_tile_encoder(K=K, device_index=device.index or 0, arena=arena, cb=cb)
    available = {name: m for name, m in layer.named_modules()
                 if isinstance(m, torch.nn.Linear) and m.bias is None}
    selected = list(available) if module_names is None else list(module_names)
    missing = [n for n in selected if n not in available]
    if missing:
        raise KeyError(f"requested modules are not bias-free nn.Linear submodules: {missing}")
    for name in selected:
        if name not in hessians:
            raise KeyError(f"Hessian missing for module {name}")
    torch.cuda.reset_peak_memory_stats(device)
    results: Dict[str, QuantizedModuleResult] = {}
    phases: Dict[str, float] = {}
    # Projections of one Hessian group (q/k/v, gate/up) share one factor.
    device_h = {id(hessians[n]): hessians[n].to(device) for n in selected}
    ldl_cache: dict = {}
    try:
        if lockstep:
            tp = time.time()
            # The global-scale search of every projection runs as one batch
            # after their regularisation (two encoder stages for the layer
            # instead of two per projection); each projection's scale equals
            # its own search's, since a candidate's MSE depends on its tiles
            # only.
            prepared = [_prepare_module(name, available[name].weight.data,
                                        device_h[id(hessians[name])], K, cb, encoder,
                                        True, block_size, ldl_cache)
                        for name in selected]
            if not skip_g_scale:
                _apply_global_scales(prepared, encoder)
            torch.cuda.synchronize(device)
            t0 = time.time()
            lqs = ldlq_lockstep([(pm.reg.weight, pm.ldl.transformed) for pm in prepared],
                                encoder, buf_size_k=buf_size_k, time_calls=time_encoder)
            shared = time.time() - t0
            for pm, lq in zip(prepared, lqs):
                results[pm.name] = _finish_module(pm, lq, K, cb, shared)
            phases = {"prepare_seconds": t0 - tp, "traversal_seconds": shared,
                      "finish_seconds": time.time() - t0 - shared}
        else:
            for name in selected:
                results[name] = quantize_linear_module(
                    name=name, weight=available[name].weight.data,
                    H=device_h[id(hessians[name])], K=K, cb=cb, tile_encoder=encoder,
                    skip_g_scale=skip_g_scale, buf_size_k=buf_size_k, block_size=block_size,
                    ldl_cache=ldl_cache, time_encoder=time_encoder)
                torch.cuda.synchronize(device)
    finally:
        arena.release()
        ldl_cache.clear()
    tiles = sum(r.original_shape[0] * r.original_shape[1] // 256 for r in results.values())
    return LayerQuantizationReport(
        K=K, codebook="mul1" if cb == CB_MUL1 else str(cb),
        total_elapsed_seconds=time.time() - t_start, module_results=results,
        total_proxy_loss=sum(r.metrics.proxy_loss for r in results.values()),
        mean_mse=float(sum(r.metrics.mse for r in results.values()) / max(1, len(results))),
        peak_device_memory_bytes=int(torch.cuda.max_memory_allocated(device)),
        scratch_arena_reused=True, device_index=device.index or 0, tiles=tiles,
        encoder_seconds=sum(r.metrics.encoder_seconds for r in results.values()),
        extra={"lockstep": bool(lockstep), **phases})
