"""LDLQ tile-encoder adapter (reference: exl3_quant/ldlq.py:39-42,344-387).

A tile encoder takes a ``(tiles_n, 256)`` float32 batch already in
tensor-core order and returns ``(reconstructed, indices)``, both
``(tiles_n, 256)``: the reconstruction in tensor-core order (fp16 values as
float32) and the indices as 16-bit states in int16. ``make_xpu_tile_encoder``
keeps the reference's name and signature; the returned callable also
carries ``.K`` and ``.cb`` as the reference's does, and ``.fork()`` gives a
second adapter with its own scratch for calls on another stream.

Unlike the reference adapter, which converts every call's tiles to numpy and
back (ldlq.py:370-380), this one keeps a CUDA input on the device: the
encoder's ``encode_tensor`` runs the HIP path and the outputs stay in HBM.
A CPU input is copied to the encoder's device and the outputs are returned
on the input's device.

A CUDA input is encoded without any device-to-host round trip: the kernels
are queued on the current stream and the call returns, so the LDLQ loop's
host work overlaps the encoder. NaN inputs are counted on the device and
reported by ``encode.check_finite()``, which raises ``ValueError`` if any
call since the previous check saw one (``ldlq`` calls it when its traversal
ends). With ``asynchronous=False`` every call checks at once instead.
"""

from __future__ import annotations

from typing import Callable

from .trellis_format import CB_MUL1

TileEncoder = Callable[["object"], "tuple"]


def make_xpu_tile_encoder(K: int = 2, device_index: int = 0, arena=None, sg_size: int = 32,
                          force_global_costs: bool = False,
                          traceback_mode: str = "gpu_resident",
                          asynchronous: bool = True, cb: int = CB_MUL1) -> TileEncoder:
    """MI355X tile encoder (``XPUTrellisEncoder``) as an LDLQ callback. The
    encoder and its ScratchArena are created once and reused for every call
    (ldlq.py:352-357). ``cb`` defaults to MUL1, the reference adapter's only
    codebook."""
    import torch

    from .gpu_quantizer import XPUTrellisEncoder

    encoder = XPUTrellisEncoder(K=K, cb=cb, arena=arena, device_index=device_index,
                                sg_size=sg_size, force_global_costs=force_global_costs)
    run_async = asynchronous and traceback_mode == "gpu_resident"
    state = {"nan_count": None}

    def check_finite() -> None:
        counter = state["nan_count"]
        if counter is None:
            return
        seen = int(counter.item())
        if seen:
            counter.zero_()
            raise ValueError(f"NaN tile values are not supported ({seen} seen by the encoder)")

    def encode(tiles):
        if tiles.dim() != 2 or tiles.size(1) != 256:
            raise ValueError(f"expected (tiles_n, 256) tiles, got {tuple(tiles.shape)}")
        dev_tiles = tiles.detach().to(device=f"cuda:{device_index}", dtype=torch.float32)
        on_device = tiles.device == dev_tiles.device
        if run_async and state["nan_count"] is None:
            state["nan_count"] = torch.zeros(1, dtype=torch.int32, device=dev_tiles.device)
        res = encoder.encode_tensor(dev_tiles.contiguous(), pre_permute=False,
                                    traceback_mode=traceback_mode, finalize=False,
                                    synchronize=not run_async,
                                    nan_count=state["nan_count"] if run_async else None,
                                    traceback_policy=encode.traceback_policy)
        recon, idx = res["reconstructed_perm"], res["indices"]
        if not on_device:
            recon, idx = recon.to(tiles.device), idx.to(tiles.device)
            check_finite()
        return recon, idx

    def fork():
        """Another adapter with the same settings, its own scratch arena (same
        memory policy) and NaN counter: for calls queued on another stream
        while this one's are in flight."""
        from .gpu_quantizer import ScratchArena
        return make_xpu_tile_encoder(
            K=K, device_index=device_index,
            arena=ScratchArena(policy=encoder.arena.policy, device_index=device_index),
            sg_size=sg_size, force_global_costs=force_global_costs,
            traceback_mode=traceback_mode, asynchronous=asynchronous, cb=cb)

    encode.K = K
    encode.cb = cb
    # Traceback kernel of this adapter's calls ("auto", "rows", "stream";
    # None = the library's process default). Per adapter, so two lanes on
    # two streams can choose differently.
    encode.traceback_policy = None
    encode.encoder = encoder
    encode.check_finite = check_finite
    encode.fork = fork
    return encode


make_gpu_tile_encoder = make_xpu_tile_encoder
