"""EXL3 layer tensors on disk (reference: exl3_quant/serialization.py).

A quantised projection is stored as
  ``<prefix>.<layer>.<module>.trellis``  int16 (k/16, n/16, 16K): every tile's
                                         256 states packed (pack_trellis,
                                         then swap16_storage);
  ``.suh`` fp16 (k,), ``.svh`` fp16 (n,): the input / output scales;
  ``.mul1`` or ``.mcg`` int32 scalar:     the codebook marker (none = 3inst);
plus quantization_config.json and model.safetensors.index.json beside the
.safetensors file. Packing and unpacking run on the GPU (exl3_pack_trellis,
exl3_unpack_trellis), as does the decode back to weights (codebook
lookup, tensor-core un-permutation, Hadamard and scales); tensors handed to
safetensors are moved to the host.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any, Dict, Optional, Tuple, Union

import torch

from .hadamard import weight_from_quantized
from .trellis_format import CB_3INST, CB_MCG, CB_MUL1, tensor_core_perm

__all__ = ["pack_module_trellis", "unpack_module_trellis", "decode_weight_from_storage",
           "build_layer_tensors", "export_layer_safetensors", "load_and_verify_layer_safetensors"]

PRODUCER = "exl3_intel_arc_quantizer_amd"


def _ext():
    from .gpu_quantizer import build_quantize_extension
    return build_quantize_extension()


def _on_gpu(t: torch.Tensor) -> torch.Tensor:
    if t.device.type == "cuda":
        return t
    if not torch.cuda.is_available():
        raise RuntimeError("the trellis packing kernels need a GPU")
    return t.to(f"cuda:{torch.cuda.current_device()}")


def _codebook_name(cb: int) -> str:
    return "mul1" if cb == CB_MUL1 else ("mcg" if cb == CB_MCG else "3inst")


def pack_module_trellis(encoded: torch.Tensor, K: int) -> torch.Tensor:
    """(tiles_k, tiles_n, 256) states -> (tiles_k, tiles_n, 16K) int16 trellis
    words (serialization.py:40-62), on the input's device."""
    if encoded.dim() != 3 or encoded.shape[-1] != 256:
        raise ValueError(f"encoded states must have shape (tiles_k, tiles_n, 256), got "
                         f"{tuple(encoded.shape)}")
    if not 1 <= K <= 8:
        raise ValueError(f"K must be in 1..8, got {K}")
    tk, tn, _ = encoded.shape
    states = _on_gpu(encoded).to(torch.int16).reshape(tk * tn, 256).contiguous()
    packed = torch.empty((tk * tn, 16 * K), dtype=torch.int16, device=states.device)
    if tk * tn:
        _ext().pack_trellis(states, packed, K)
    return packed.view(tk, tn, 16 * K).to(encoded.device)


def unpack_module_trellis(trellis: torch.Tensor, K: int) -> torch.Tensor:
    """(tiles_k, tiles_n, 16K) int16 trellis words -> (tiles_k, tiles_n, 256)
    int16 states (serialization.py:65-84), on the input's device."""
    if trellis.dim() != 3:
        raise ValueError(f"trellis must be 3-D, got {tuple(trellis.shape)}")
    if trellis.shape[-1] != 16 * K:
        raise ValueError(f"Trellis last dimension {trellis.shape[-1]} does not match "
                         f"16 * K = {16 * K}")
    tk, tn, _ = trellis.shape
    words = _on_gpu(trellis).to(torch.int16).reshape(tk * tn, 16 * K).contiguous()
    states = torch.empty((tk * tn, 256), dtype=torch.int16, device=words.device)
    if tk * tn:
        _ext().unpack_trellis(words, states, K)
    return states.view(tk, tn, 256).to(trellis.device)


def decode_weight_from_storage(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                               K: int, cb: int = CB_MUL1) -> torch.Tensor:
    """Original-basis (k, n) float32 weight from stored EXL3 tensors
    (serialization.py:223-266): unpack, codebook values, tiles back to their
    original element order, then Hadamard and scales. On the trellis'
    device."""
    tk, tn, _ = trellis.shape
    dev_trellis = _on_gpu(trellis)
    device = dev_trellis.device
    states = unpack_module_trellis(dev_trellis, K).to(torch.int64) & 0xFFFF
    lut = torch.empty(65536, dtype=torch.float16, device=device)
    _ext().decode_codebook(cb, lut)
    vals = lut[states].to(torch.float32)                                  # (tk, tn, 256) TC order
    perm = torch.as_tensor(tensor_core_perm(), dtype=torch.long, device=device)
    tiles = torch.empty_like(vals)
    tiles[..., perm] = vals
    w_hat = tiles.view(tk, tn, 16, 16).permute(0, 2, 1, 3).reshape(tk * 16, tn * 16)
    w = weight_from_quantized(w_hat, suh.to(device).unsqueeze(1), svh.to(device).unsqueeze(0))
    return w.to(trellis.device)


def build_layer_tensors(module_results: Dict[str, Any], layer_idx: int = 0,
                        prefix: str = "model.layers",
                        norm_weights: Optional[Dict[str, torch.Tensor]] = None,
                        extra_tensors: Optional[Dict[str, torch.Tensor]] = None,
                        preserve_source_dtype: bool = False
                        ) -> Tuple[Dict[str, torch.Tensor], Dict[str, Any]]:
    """Host tensors and per-module metadata of one layer in the EXL3
    safetensors schema (serialization.py:87-178)."""
    tensors: Dict[str, torch.Tensor] = {}
    storage: Dict[str, Any] = {}
    base = f"{prefix}.{layer_idx}" if prefix else f"layers.{layer_idx}"
    for name, res in module_results.items():
        key = f"{base}.{name}"
        trellis = pack_module_trellis(res.encoded, K=res.K).cpu()
        suh = res.su.detach().flatten().to(torch.float16).cpu()
        svh = res.sv.detach().flatten().to(torch.float16).cpu()
        tensors[f"{key}.trellis"] = trellis
        tensors[f"{key}.suh"] = suh
        tensors[f"{key}.svh"] = svh
        if res.cb == CB_MUL1:
            tensors[f"{key}.mul1"] = torch.tensor(0, dtype=torch.int32)
        elif res.cb == CB_MCG:
            tensors[f"{key}.mcg"] = torch.tensor(0, dtype=torch.int32)
        storage[key] = {
            "quant_format": "exl3",
            "bits_per_weight": res.K,
            "codebook": _codebook_name(res.cb),
            "stored_tensors": {f"{key}.trellis": {"shape": list(trellis.shape)},
                               f"{key}.suh": {"shape": list(suh.shape)},
                               f"{key}.svh": {"shape": list(svh.shape)}},
        }
    for norm, w in (norm_weights or {}).items():
        w = w.detach().cpu()
        tensors[f"{base}.{norm}"] = w if preserve_source_dtype else w.to(torch.float16)
    for key, w in (extra_tensors or {}).items():
        if key in tensors:
            raise ValueError(f"pass-through tensor collides with an emitted tensor: {key}")
        tensors[key] = w.detach().cpu()
    return tensors, storage


def export_layer_safetensors(module_results: Dict[str, Any], output_dir: Union[str, Path],
                             filename: str = "model.safetensors", layer_idx: int = 0,
                             prefix: str = "model.layers",
                             norm_weights: Optional[Dict[str, torch.Tensor]] = None
                             ) -> Tuple[Path, Path]:
    """Write the layer's .safetensors, quantization_config.json and
    model.safetensors.index.json (serialization.py:181-220)."""
    from safetensors.torch import save_file

    if not module_results:
        raise ValueError("module_results is empty")
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    tensors, storage = build_layer_tensors(module_results, layer_idx=layer_idx, prefix=prefix,
                                           norm_weights=norm_weights)
    first = next(iter(module_results.values()))
    # The file-level codebook names MCG as such, as each module's storage
    # entry does (the reference's file level says "3inst" for it).
    meta = {"quant_format": "exl3", "producer": PRODUCER, "version": "1.0",
            "codebook": _codebook_name(first.cb), "bits": str(first.K)}
    st_file = out / filename
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(st_file), metadata=meta)
    qc_file = out / "quantization_config.json"
    qc_file.write_text(json.dumps({"quant_method": "exl3", "bits": first.K,
                                   "codebook": meta["codebook"], "tensor_storage": storage},
                                  indent=2))
    (out / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": meta, "weight_map": {k: filename for k in tensors}}, indent=2))
    return st_file, qc_file


def load_and_verify_layer_safetensors(safetensors_path: Union[str, Path],
                                      expected_results: Optional[Dict[str, Any]] = None,
                                      atol: float = 5e-3) -> Dict[str, torch.Tensor]:
    """Reload a layer file, decode every ``.trellis`` module (codebook from
    its marker tensor) and, given ``expected_results``, check each decoded
    weight against the module's ``w_hat`` (serialization.py:269-326).
    Returns the decoded weights by module key (host tensors)."""
    from safetensors import safe_open

    path = Path(safetensors_path)
    if not path.exists():
        raise FileNotFoundError(f"Safetensors file not found: {path}")
    with safe_open(str(path), framework="pt", device="cpu") as f:
        loaded = {k: f.get_tensor(k) for k in f.keys()}
    decoded: Dict[str, torch.Tensor] = {}
    for t_key in (k for k in loaded if k.endswith(".trellis")):
        mod = t_key[:-len(".trellis")]
        if f"{mod}.suh" not in loaded or f"{mod}.svh" not in loaded:
            raise KeyError(f"Missing suh or svh for {mod}")
        trellis = loaded[t_key]
        cb = (CB_MCG if f"{mod}.mcg" in loaded else
              CB_MUL1 if f"{mod}.mul1" in loaded else CB_3INST)
        w = decode_weight_from_storage(trellis, loaded[f"{mod}.suh"], loaded[f"{mod}.svh"],
                                       K=trellis.shape[-1] // 16, cb=cb).cpu()
        decoded[mod] = w
        for name, res in (expected_results or {}).items():
            if name in mod:
                diff = (w - res.w_hat.detach().float().cpu()).abs().max().item()
                if not diff < atol:
                    raise AssertionError(f"Mismatch in reloaded {name}: max diff {diff} "
                                         f"exceeds atol {atol}")
    return decoded
