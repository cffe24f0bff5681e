"""LDLQ tile-encoder adapter (reference: exl3_quant/ldlq.py:39-42,344-387).

A tile encoder takes a ``(tiles_n, 256)`` float32 batch already in
tensor-core order and returns ``(reconstructed, indices)``, both
``(tiles_n, 256)``: the reconstruction in tensor-core order (fp16 values as
float32) and the indices as 16-bit states in int16. ``make_xpu_tile_encoder``
keeps the reference's name and signature; the returned callable also
carries ``.K`` and ``.cb`` as the reference's does.

Unlike the reference adapter, which converts every call's tiles to numpy and
back (ldlq.py:370-380), this one keeps a CUDA input on the device: the
encoder's ``encode_tensor`` runs the HIP path and the outputs stay in HBM.
A CPU input is copied to the encoder's device and the outputs are returned
on the input's device.
"""

from __future__ import annotations

from typing import Callable

from .trellis_format import CB_MUL1

TileEncoder = Callable[["object"], "tuple"]


def make_xpu_tile_encoder(K: int = 2, device_index: int = 0, arena=None, sg_size: int = 32,
                          force_global_costs: bool = False,
                          traceback_mode: str = "gpu_resident") -> TileEncoder:
    """MI355X tile encoder (``XPUTrellisEncoder``, MUL1 codebook) as an LDLQ
    callback. The encoder and its ScratchArena are created once and reused
    for every call (ldlq.py:352-357)."""
    from .gpu_quantizer import XPUTrellisEncoder

    encoder = XPUTrellisEncoder(K=K, cb=CB_MUL1, arena=arena, device_index=device_index,
                                sg_size=sg_size, force_global_costs=force_global_costs)

    def encode(tiles):
        import torch

        if tiles.dim() != 2 or tiles.size(1) != 256:
            raise ValueError(f"expected (tiles_n, 256) tiles, got {tuple(tiles.shape)}")
        dev_tiles = tiles.detach().to(device=f"cuda:{device_index}", dtype=torch.float32)
        res = encoder.encode_tensor(dev_tiles.contiguous(), pre_permute=False,
                                    traceback_mode=traceback_mode, finalize=False)
        recon, idx = res["reconstructed_perm"], res["indices"]
        if tiles.device != recon.device:
            recon, idx = recon.to(tiles.device), idx.to(tiles.device)
        return recon, idx

    encode.K = K
    encode.cb = CB_MUL1
    encode.encoder = encoder
    return encode


make_gpu_tile_encoder = make_xpu_tile_encoder
