"""ctypes binding of ``libexl3_hip.so`` and the extension facade.

``QuantizeExtension`` mirrors the functions of the reference's pybind module
``quantize_xpu_ext`` (csrc/quantize_xpu/quantize_xpu.cpp:302-357) with the
same names, argument order, defaults and error behaviour (``RuntimeError``
for rejected tensors, as its ``TORCH_CHECK``s raise), but takes torch-ROCm
device tensors (``cuda:i``) and calls the C-ABI declared in
``include/exl3_encoder.h``. Work is enqueued on the tensor's current torch
stream; nothing here synchronises.

There is no CPU fallback: loading fails loudly when the library is missing.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

from .build import LIB_PATH

_LIB = None

_c_int, _c_i64, _c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_version": (ctypes.c_char_p, []),
    "exl3_set_traceback_policy": (_c_int, [_c_int]),
    "exl3_decode_codebook": (_c_int, [_c_int, _c_vp, _c_vp]),
    "exl3_scratch_row_bytes": (_c_i64, [_c_int]),
    "exl3_scratch_edges_bytes": (_c_i64, [_c_int, _c_int, _c_i64]),
    "exl3_cost_row_slot": (_c_i64, [_c_int, _c_i64]),
    "exl3_quantize_tiles": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int,
                                     _c_int, _c_int, _c_int, _c_i64, _c_vp]),
    "exl3_quantize_tiles_tb": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                        _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_vp]),
    "exl3_quantize_tiles_noalloc": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int,
                                             _c_int, _c_vp]),
    "exl3_forward_pass": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int,
                                   _c_int, _c_int, _c_int, _c_vp]),
    "exl3_backward_pass": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_int,
                                    _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "exl3_prepare_tiles": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_vp, _c_vp]),
    "exl3_finalize_tiles": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                     _c_i64, _c_int, _c_int, _c_int, _c_vp]),
    "exl3_pack_trellis": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_vp]),
    "exl3_unpack_trellis": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_vp]),
    "exl3_probe_hfma": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_vp]),
    # include/exl3_layer.h
    "exl3_hadamard128": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_vp]),
    "exl3_hadamard128_scaled": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_vp, _c_vp,
                                         _c_vp]),
    "exl3_block_rms_from_slices": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]),
    "exl3_block_rms": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_vp, _c_i64,
                                _c_vp]),
    "exl3_block_rms_workspace": (_c_i64, [_c_i64, _c_i64, _c_int, _c_int]),
    "exl3_cholesky_diag_block": (_c_int, [_c_vp, _c_i64, _c_int, _c_i64, _c_vp, _c_vp]),
    "exl3_cholesky_block_order": (_c_int, []),
    "exl3_ldlq_gather": (_c_int, [_c_vp, _c_int, _c_i64, _c_vp, _c_vp]),
    "exl3_ldlq_scatter": (_c_int, [_c_vp, _c_int, _c_i64, _c_vp, _c_vp, _c_vp]),
}


def exported_symbols() -> list:
    """C-ABI entry points declared in include/exl3_encoder.h and
    include/exl3_layer.h."""
    return sorted(_SIGNATURES)


def load_library(path: Optional[Path] = None):
    """Load the native library (no build, no fallback)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    lib_path = Path(path) if path is not None else LIB_PATH
    if not lib_path.exists():
        raise RuntimeError(
            f"native encoder library {lib_path} is missing; build it with "
            "`python -m exl3_intel_arc_quantizer_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(lib_path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _LIB = lib
    return lib



TRACEBACK_POLICIES = {"auto": 0, "rows": 1, "stream": 2}


def _policy_code(policy: Optional[str]) -> int:
    """C-ABI code of a traceback policy name; None = the process default (-1)."""
    if policy is None:
        return -1
    if policy not in TRACEBACK_POLICIES:
        raise ValueError(f"policy must be one of {sorted(TRACEBACK_POLICIES)}, got {policy!r}")
    return TRACEBACK_POLICIES[policy]


def set_traceback_policy(policy: str) -> str:
    """Choose the default traceback kernel for later calls in this process
    that do not name one: "auto" (by batch size), "rows" (per-row tree
    loads) or "stream" (whole rows streamed through LDS); results are
    identical. Returns the previous default. ``quantize_tiles(...,
    traceback_policy=...)`` chooses per call without changing it."""
    if policy is None:
        raise ValueError("set_traceback_policy needs a policy name")
    prev = load_library().exl3_set_traceback_policy(_policy_code(policy))
    return {v: k for k, v in TRACEBACK_POLICIES.items()}[prev]

def last_error() -> str:
    return load_library().exl3_last_error().decode()


def _check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {last_error()}")


# ------------------------------------------------------------- validation

def _torch():
    import torch
    return torch


def _check_device_tensor(t, name: str, dtype, ndim: int) -> int:
    """TORCH_CHECK equivalents of check_xpu_tensor (quantize_xpu.cpp:73-83)."""
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU (cuda) tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} has wrong dtype")
    if t.dim() != ndim:
        raise RuntimeError(f"{name} must be {ndim}-D, got {t.dim()}-D")
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _check_buffer(t, name: str, dtype, shape, dev: int) -> None:
    """A device tensor of exactly ``shape`` on device ``dev``: every buffer a
    kernel indexes by the launch's sizes is checked before the launch."""
    if _check_device_tensor(t, name, dtype, len(shape)) != dev:
        raise RuntimeError(f"{name} must be on the same GPU device")
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _resolve_cb(mcg: bool, mul1: bool) -> int:
    """quantize_xpu.cpp:85-91."""
    if mcg and mul1:
        raise RuntimeError("mcg and mul1 cannot both be true (ambiguous codebook)")
    return 2 if mul1 else (1 if mcg else 0)


def _validate_common(K: int, cb: int, L: int, sg_size: int) -> None:
    """quantize_xpu.cpp:93-101. sg_size is accepted for API parity; wave64
    hardware has no sub-group width choice."""
    if not 1 <= K <= 8:
        raise RuntimeError(f"K must be in 1..8, got {K}")
    if L not in (256, 160):
        raise RuntimeError(f"tile length L must be 256 or 160, got {L}")
    if L == 160 and cb != 2:
        raise RuntimeError("tile length L=160 is only supported with mul1 (cb=2)")
    if sg_size not in (16, 32):
        raise RuntimeError(f"sg_size must be 16 or 32, got {sg_size}")


def _stream(device_index: int) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device_index).cuda_stream


def row_bytes(K: int) -> int:
    """Bytes of one scratch row at bitrate K."""
    return int(load_library().exl3_scratch_row_bytes(K))


def tile_rows(K: int, L: int = 256) -> int:
    """Scratch rows per tile (stored cost rows or ring rows, plus a header)."""
    lib = load_library()
    return int(lib.exl3_scratch_edges_bytes(K, L, 1) // lib.exl3_scratch_row_bytes(K))


def edges_shape(B: int, K: int, L: int = 256) -> tuple:
    """Shape of a uint8 ``temp_edges`` scratch tensor for B tiles."""
    return (B, tile_rows(K, L), row_bytes(K))


class QuantizeExtension:
    """Drop-in for the reference's ``quantize_xpu_ext`` module object."""

    def __init__(self, lib=None):
        self.lib = lib or load_library()

    # quantize_xpu.cpp:105-110
    def decode_codebook(self, cb: int, out_lut) -> None:
        torch = _torch()
        if not 0 <= cb <= 2:
            raise RuntimeError("cb must be 0, 1, or 2")
        dev = _check_device_tensor(out_lut, "out_lut", torch.float16, 1)
        if out_lut.size(0) != 65536:
            raise RuntimeError("out_lut must have length 65536")
        with torch.cuda.device(dev):
            _check(self.lib.exl3_decode_codebook(cb, out_lut.data_ptr(), _stream(dev)),
                   "decode_codebook")

    def _scratch_checks(self, temp_costs, temp_edges, K: int, L: int, dev: int) -> int:
        torch = _torch()
        if _check_device_tensor(temp_costs, "temp_costs", torch.float16, 3) != dev:
            raise RuntimeError("temp_costs must be on the same GPU device as input_tiles")
        if _check_device_tensor(temp_edges, "temp_edges", torch.uint8, 3) != dev:
            raise RuntimeError("temp_edges must be on the same GPU device as input_tiles")
        edges = 65536 >> K
        batch_cap = temp_costs.size(0)
        if batch_cap < 1:
            raise RuntimeError("temp_costs batch dimension B must be >= 1")
        if temp_costs.size(1) != 2 or temp_costs.size(2) != edges:
            raise RuntimeError("temp_costs must have shape (B, 2, 65536 >> K)")
        _, rows, rb = edges_shape(batch_cap, K, L)
        if (temp_edges.size(0) < batch_cap or temp_edges.size(1) != rows
                or temp_edges.size(2) != rb):
            raise RuntimeError(
                f"temp_edges must have shape (B, {rows}, {rb}) for K={K}, L={L} "
                "(cost-row scratch layout)")
        return batch_cap

    # quantize_xpu.cpp:112-167
    def quantize_tiles(self, input_tiles, output_tiles, output_indices, temp_costs, temp_edges,
                       K: int, mcg: bool, mul1: bool, sg_size: int = 32,
                       force_global_costs: bool = False, wave_cap_override: int = 0,
                       traceback_policy: Optional[str] = None) -> None:
        """The reference's arguments, plus ``traceback_policy`` (no counterpart
        there): the traceback kernel for this call only, "auto", "rows",
        "stream", or None for the process default."""
        torch = _torch()
        cb = _resolve_cb(mcg, mul1)
        tb = _policy_code(traceback_policy)
        dev = _check_device_tensor(input_tiles, "input_tiles", torch.float32, 2)
        if _check_device_tensor(output_tiles, "output_tiles", torch.float32, 2) != dev:
            raise RuntimeError("output_tiles must be on the same GPU device as input_tiles")
        if _check_device_tensor(output_indices, "output_indices", torch.int16, 2) != dev:
            raise RuntimeError("output_indices must be on the same GPU device as input_tiles")
        n, L = input_tiles.shape
        if n <= 0:
            raise RuntimeError(f"num_tiles must be positive, got {n}")
        _validate_common(K, cb, L, sg_size)
        batch_cap = self._scratch_checks(temp_costs, temp_edges, K, L, dev)
        if tuple(output_tiles.shape) != (n, L):
            raise RuntimeError("output_tiles shape must match input_tiles")
        if tuple(output_indices.shape) != (n, L):
            raise RuntimeError("output_indices shape must match input_tiles")
        with torch.cuda.device(dev):
            _check(self.lib.exl3_quantize_tiles_tb(
                input_tiles.data_ptr(), output_tiles.data_ptr(), output_indices.data_ptr(),
                temp_costs.data_ptr(), temp_edges.data_ptr(), batch_cap, n, K, cb, L,
                int(bool(force_global_costs)), int(wave_cap_override), tb, _stream(dev)),
                "quantize_tiles")

    # quantize_xpu.cpp:169-215
    def quantize_tiles_forward_pass(self, input_tiles, temp_costs, temp_edges, pre_states,
                                    K: int, mcg: bool, mul1: bool, roll: int, cost_slot: int = 0,
                                    sg_size: int = 32, force_global_costs: bool = False) -> None:
        torch = _torch()
        cb = _resolve_cb(mcg, mul1)
        dev = _check_device_tensor(input_tiles, "input_tiles", torch.float32, 2)
        if _check_device_tensor(pre_states, "pre_states", torch.int32, 1) != dev:
            raise RuntimeError("pre_states must be an int32 GPU tensor")
        n, L = input_tiles.shape
        _validate_common(K, cb, L, sg_size)
        batch_cap = self._scratch_checks(temp_costs, temp_edges, K, L, dev)
        if not 0 < n <= batch_cap:
            raise RuntimeError("num_tiles must be in 1..B")
        if pre_states.size(0) < n:
            raise RuntimeError("pre_states length must be >= num_tiles")
        if cost_slot not in (0, 1):
            raise RuntimeError("cost_slot must be 0 or 1")
        with torch.cuda.device(dev):
            _check(self.lib.exl3_forward_pass(
                input_tiles.data_ptr(), temp_costs.data_ptr(), temp_edges.data_ptr(),
                pre_states.data_ptr(), n, K, cb, L, int(roll), int(cost_slot),
                int(bool(force_global_costs)), _stream(dev)), "quantize_tiles_forward_pass")

    # quantize_xpu.cpp:217-259
    def quantize_tiles_backward_pass(self, temp_costs, temp_edges, output_tiles, output_indices,
                                     end_states, num_tiles: int, K: int, mcg: bool, mul1: bool,
                                     roll: int, cost_slot: int, write_output: bool,
                                     sg_size: int = 32) -> None:
        torch = _torch()
        cb = _resolve_cb(mcg, mul1)
        dev = _check_device_tensor(temp_costs, "temp_costs", torch.float16, 3)
        if _check_device_tensor(output_tiles, "output_tiles", torch.float32, 2) != dev:
            raise RuntimeError("output_tiles must be on the same GPU device")
        if _check_device_tensor(output_indices, "output_indices", torch.int16, 2) != dev:
            raise RuntimeError("output_indices must be on the same GPU device")
        if _check_device_tensor(end_states, "end_states", torch.int32, 1) != dev:
            raise RuntimeError("end_states must be an int32 GPU tensor")
        # The tile length is the one (256 or 160) whose scratch row count the
        # temp_edges tensor has; the two counts differ at every K.
        _validate_common(K, cb, 256, sg_size)
        if temp_edges.dim() != 3:
            raise RuntimeError("temp_edges must be 3-D (B, rows, row_bytes)")
        matches = [n for n in (256, 160) if tile_rows(K, n) == temp_edges.size(1)]
        if not matches:
            raise RuntimeError(f"temp_edges has {temp_edges.size(1)} rows, which fits neither "
                               f"L=256 ({tile_rows(K, 256)}) nor L=160 ({tile_rows(K, 160)}) "
                               f"at K={K}")
        L = matches[0]
        _validate_common(K, cb, L, sg_size)
        batch_cap = self._scratch_checks(temp_costs, temp_edges, K, L, dev)
        if not 0 < num_tiles <= batch_cap:
            raise RuntimeError("num_tiles must be in 1..B")
        if end_states.size(0) < num_tiles:
            raise RuntimeError("end_states length must be >= num_tiles")
        if write_output and (output_tiles.size(0) < num_tiles or output_tiles.size(1) != L
                             or output_indices.size(0) < num_tiles
                             or output_indices.size(1) != L):
            raise RuntimeError("output tensors must have shape (>= num_tiles, L)")
        with torch.cuda.device(dev):
            _check(self.lib.exl3_backward_pass(
                temp_costs.data_ptr(), temp_edges.data_ptr(), output_tiles.data_ptr(),
                output_indices.data_ptr(), end_states.data_ptr(), int(num_tiles), K, cb, L,
                int(roll), int(cost_slot), int(bool(write_output)), _stream(dev)),
                "quantize_tiles_backward_pass")

    # quantize_xpu.cpp:261-300, quantize_kernels.sycl:756-841
    def quantize_tiles_usm_host(self, input_tiles, temp_costs, output_tiles_cpu,
                                output_indices_cpu, lut_cpu, K: int, mcg: bool, mul1: bool,
                                sg_size: int = 32) -> list:
        """The reference's host-visible-edges variant: states and codebook
        values land in CPU tensors, and [search_s, trace_s] is returned. On
        MI355X the search and the traceback both run on the GPU (split
        forward/backward passes over an internal device scratch of
        temp_costs' batch size); the results are copied to the CPU tensors.
        ``lut_cpu`` is validated as in the reference and otherwise unused:
        the GPU decodes states in registers."""
        torch = _torch()
        cb = _resolve_cb(mcg, mul1)
        dev = _check_device_tensor(input_tiles, "input_tiles", torch.float32, 2)
        if _check_device_tensor(temp_costs, "temp_costs", torch.float16, 3) != dev:
            raise RuntimeError("temp_costs must be on the same GPU device")
        if not (output_tiles_cpu.device.type == "cpu" and output_tiles_cpu.is_contiguous()
                and output_tiles_cpu.dtype == torch.float32):
            raise RuntimeError("output_tiles_cpu must be a contiguous float32 CPU tensor")
        if not (output_indices_cpu.device.type == "cpu" and output_indices_cpu.is_contiguous()
                and output_indices_cpu.dtype == torch.int16):
            raise RuntimeError("output_indices_cpu must be a contiguous int16 CPU tensor")
        if not (lut_cpu.device.type == "cpu" and lut_cpu.is_contiguous()
                and lut_cpu.dtype == torch.float32 and lut_cpu.numel() == 65536):
            raise RuntimeError("lut_cpu must be a 65536-element float32 CPU tensor")
        n, L = input_tiles.shape
        _validate_common(K, cb, L, sg_size)
        if tuple(output_tiles_cpu.shape) != (n, L) or tuple(output_indices_cpu.shape) != (n, L):
            raise RuntimeError("output tensors must have shape (num_tiles, L)")
        B = temp_costs.size(0)
        if B < 1 or temp_costs.size(1) != 2 or temp_costs.size(2) != (65536 >> K):
            raise RuntimeError("temp_costs must have shape (B, 2, 65536 >> K)")
        search_s = trace_s = 0.0
        with torch.cuda.device(dev):
            edges = torch.empty(edges_shape(B, K, L), dtype=torch.uint8, device=f"cuda:{dev}")
            out_w = torch.empty((n, L), dtype=torch.float32, device=f"cuda:{dev}")
            out_i = torch.empty((n, L), dtype=torch.int16, device=f"cuda:{dev}")
            ends = torch.empty(B, dtype=torch.int32, device=f"cuda:{dev}")
            free = torch.full((B,), -1, dtype=torch.int32, device=f"cuda:{dev}")
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            for off in range(0, n, B):
                c = min(B, n - off)
                x = input_tiles[off:off + c]
                ev[0].record()
                self.quantize_tiles_forward_pass(x, temp_costs, edges, free, K, mcg, mul1,
                                                 L // 2, 0, sg_size)
                ev[1].record()
                self.quantize_tiles_backward_pass(temp_costs, edges, out_w[off:off + c],
                                                  out_i[off:off + c], ends, c, K, mcg, mul1,
                                                  L // 2, 0, False, sg_size)
                ev[2].record()
                self.quantize_tiles_forward_pass(x, temp_costs, edges, ends, K, mcg, mul1, 0, 1,
                                                 sg_size)
                ev[3].record()
                self.quantize_tiles_backward_pass(temp_costs, edges, out_w[off:off + c],
                                                  out_i[off:off + c], ends, c, K, mcg, mul1, 0, 1,
                                                  True, sg_size)
                ev[4].record()
                ev[4].synchronize()
                search_s += (ev[0].elapsed_time(ev[1]) + ev[2].elapsed_time(ev[3])) / 1e3
                trace_s += (ev[1].elapsed_time(ev[2]) + ev[3].elapsed_time(ev[4])) / 1e3
            output_tiles_cpu.copy_(out_w.cpu())
            output_indices_cpu.copy_(out_i.cpu())
        return [search_s, trace_s]

    # -------------------------------------------------- device-side helpers

    def prepare_tiles(self, raw, out, permute: bool, nan_count=None) -> None:
        """fp16-round (and optionally permute) ``raw`` into ``out``; a given
        ``nan_count`` (device int32, one element) gains one per NaN value."""
        torch = _torch()
        dev = _check_device_tensor(raw, "raw", torch.float32, 2)
        n, L = raw.shape
        _check_buffer(out, "out", torch.float32, (n, L), dev)
        counter = None
        if nan_count is not None:
            if (not isinstance(nan_count, torch.Tensor) or nan_count.dtype != torch.int32
                    or nan_count.device != raw.device or nan_count.numel() < 1):
                raise RuntimeError("nan_count must be an int32 tensor on the tiles' device")
            counter = nan_count.data_ptr()
        with torch.cuda.device(dev):
            _check(self.lib.exl3_prepare_tiles(raw.data_ptr(), out.data_ptr(), n, L,
                                               int(bool(permute)), counter, _stream(dev)),
                   "prepare_tiles")

    def finalize_tiles(self, x, raw, out_w, out_idx, packed, path_cost, distortion, recon_orig,
                       K: int, permuted: bool) -> None:
        torch = _torch()
        dev = _check_device_tensor(x, "x", torch.float32, 2)
        n, L = x.shape
        for t, name, dt, shape in ((out_w, "out_w", torch.float32, (n, L)),
                                   (out_idx, "out_idx", torch.int16, (n, L)),
                                   (path_cost, "path_cost", torch.float32, (n,)),
                                   (distortion, "distortion", torch.float32, (n,)),
                                   (recon_orig, "recon_orig", torch.int16, (n, L))):
            _check_buffer(t, name, dt, shape, dev)
        if packed is not None:
            _check_buffer(packed, "packed", torch.int16, (n, 16 * K), dev)
        if permuted:
            _check_buffer(raw, "raw", torch.float32, (n, L), dev)
        with torch.cuda.device(dev):
            _check(self.lib.exl3_finalize_tiles(
                x.data_ptr(), raw.data_ptr() if permuted else None, out_w.data_ptr(),
                out_idx.data_ptr(), packed.data_ptr() if packed is not None else None,
                path_cost.data_ptr(), distortion.data_ptr(), recon_orig.data_ptr(), n, K, L,
                int(bool(permuted)), _stream(dev)), "finalize_tiles")

    def pack_trellis(self, states, packed, K: int) -> None:
        torch = _torch()
        dev = _check_device_tensor(states, "states", torch.int16, 2)
        n = states.size(0)
        if states.size(1) != 256 or not 1 <= K <= 8:
            raise RuntimeError("pack_trellis expects (n, 256) states and K in 1..8")
        _check_buffer(packed, "packed", torch.int16, (n, 16 * K), dev)
        with torch.cuda.device(dev):
            _check(self.lib.exl3_pack_trellis(states.data_ptr(), packed.data_ptr(), n, K,
                                              _stream(dev)), "pack_trellis")

    def unpack_trellis(self, packed, states, K: int) -> None:
        """Packed (n, 16*K) int16 tiles back to (n, 256) int16 states."""
        torch = _torch()
        dev = _check_device_tensor(packed, "packed", torch.int16, 2)
        n = packed.size(0)
        if not 1 <= K <= 8 or packed.size(1) != 16 * K:
            raise RuntimeError("unpack_trellis expects (n, 16*K) words and K in 1..8")
        _check_buffer(states, "states", torch.int16, (n, 256), dev)
        with torch.cuda.device(dev):
            _check(self.lib.exl3_unpack_trellis(packed.data_ptr(), states.data_ptr(), n, K,
                                                _stream(dev)), "unpack_trellis")

    def probe_hfma(self, dh, cost, out, mode: int) -> None:
        """exl3_quant/xpu_probe.py ``probe_hfma`` (mode 0: fused, 1: two roundings)."""
        torch = _torch()
        dev = _check_device_tensor(dh, "dh", torch.float16, 1)
        _check_buffer(cost, "cost", torch.float16, tuple(dh.shape), dev)
        _check_buffer(out, "out", torch.float16, tuple(dh.shape), dev)
        with torch.cuda.device(dev):
            _check(self.lib.exl3_probe_hfma(dh.data_ptr(), cost.data_ptr(), out.data_ptr(),
                                            dh.numel(), int(mode), _stream(dev)), "probe_hfma")


# ------------------------------------------------- layer pipeline kernels

def _matrix(t, name: str) -> int:
    """A contiguous 2-D float32 GPU tensor; returns its device index."""
    return _check_device_tensor(t, name, _torch().float32, 2)


def hadamard128(x, out, side: int) -> None:
    """``out = H @ x`` per 128-row block (side 0) or ``x @ H`` per 128-column
    block (side 1), H the orthonormal Sylvester matrix of order 128
    (hadamard.py:73-96); ``out`` may be ``x``."""
    dev = _matrix(x, "x")
    _check_buffer(out, "out", x.dtype, tuple(x.shape), dev)
    rows, cols = x.shape
    torch = _torch()
    with torch.cuda.device(dev):
        _check(load_library().exl3_hadamard128(x.data_ptr(), out.data_ptr(), rows, cols,
                                               int(side), _stream(dev)), "hadamard128")


def hadamard128_scaled(x, out, side: int, divisor=None, slice_sumsq=None) -> None:
    """``out = (x / divisor[col]) @ H`` per 128-column block (side 1) or
    ``out = H @ (x / divisor[row])`` per 128-row block (side 0); with side 1
    ``slice_sumsq`` (rows x cols / 32 float32) receives the sums of squares
    of every 32-element slice of the output rows. ``out`` may be ``x``."""
    torch = _torch()
    dev = _matrix(x, "x")
    _check_buffer(out, "out", x.dtype, tuple(x.shape), dev)
    rows, cols = x.shape
    if divisor is not None:
        want = cols if side == 1 else rows
        if (not isinstance(divisor, torch.Tensor) or divisor.dtype != torch.float32
                or not divisor.is_contiguous() or divisor.device != x.device
                or divisor.numel() != want):
            raise RuntimeError(f"divisor must be a contiguous float32 tensor of {want} elements "
                               f"on {x.device}")
    if slice_sumsq is not None:
        if side != 1 or cols % 32:
            raise RuntimeError("slice sums of squares need side 1 and columns divisible by 32")
        _check_buffer(slice_sumsq, "slice_sumsq", torch.float32, (rows, cols // 32), dev)
    with torch.cuda.device(dev):
        _check(load_library().exl3_hadamard128_scaled(
            x.data_ptr(), out.data_ptr(), rows, cols, int(side),
            divisor.data_ptr() if divisor is not None else None,
            slice_sumsq.data_ptr() if slice_sumsq is not None else None, _stream(dev)),
            "hadamard128_scaled")


def block_rms_from_slices(slice_sumsq, out, n: int) -> None:
    """``out[o] = sqrt(sum_s slice_sumsq[o, s] / n)``, the slices added in
    order (the second pass of block_rms)."""
    torch = _torch()
    dev = _matrix(slice_sumsq, "slice_sumsq")
    outputs, slices = slice_sumsq.shape
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.float32 or not out.is_contiguous()
            or out.device != slice_sumsq.device or out.numel() != outputs):
        raise RuntimeError(f"out must be a contiguous float32 tensor of {outputs} elements")
    with torch.cuda.device(dev):
        _check(load_library().exl3_block_rms_from_slices(slice_sumsq.data_ptr(), out.data_ptr(),
                                                         outputs, int(n), slices, _stream(dev)),
               "block_rms_from_slices")


def block_rms(x, out, dim: int, blocksize: int = 32) -> None:
    """regularize.py:41-56 into ``out`` (``x.shape[1 - dim]`` elements,
    any shape)."""
    dev = _matrix(x, "x")
    rows, cols = x.shape
    n_out = cols if dim == 0 else rows
    torch = _torch()
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.float32 or not out.is_contiguous()
            or out.device != x.device or out.numel() != n_out):
        raise RuntimeError(f"out must be a contiguous float32 tensor of {n_out} elements on "
                           f"{x.device}")
    lib = load_library()
    need = int(lib.exl3_block_rms_workspace(rows, cols, int(dim), int(blocksize)))
    if need < 0:
        raise RuntimeError(f"block_rms: invalid dim {dim} or blocksize {blocksize}")
    with torch.cuda.device(dev):
        ws = torch.empty(max(need, 1), dtype=torch.float32, device=x.device)
        _check(lib.exl3_block_rms(x.data_ptr(), out.data_ptr(), rows, cols, int(dim),
                                  int(blocksize), ws.data_ptr(), ws.numel(), _stream(dev)),
               "block_rms")


def cholesky_block_order() -> int:
    return int(load_library().exl3_cholesky_block_order())


def cholesky_diag_block(a, j0: int, nb: int, info) -> None:
    """Factor the diagonal block ``a[j0:j0+nb, j0:j0+nb]`` of the square
    matrix ``a`` in place; a failed pivot k records ``j0 + k + 1`` in
    ``info`` (one int32 on the same device) unless it is already set."""
    torch = _torch()
    dev = _matrix(a, "a")
    n = a.shape[0]
    if a.shape[1] != n:
        raise RuntimeError(f"a must be square, got {tuple(a.shape)}")
    if not (0 <= j0 and 1 <= nb <= cholesky_block_order() and j0 + nb <= n):
        raise RuntimeError(f"block [{j0}, {j0 + nb}) does not fit a {n} x {n} matrix")
    if (not isinstance(info, torch.Tensor) or info.dtype != torch.int32
            or info.device != a.device or info.numel() < 1):
        raise RuntimeError("info must be an int32 tensor on a's device")
    with torch.cuda.device(dev):
        _check(load_library().exl3_cholesky_diag_block(a.data_ptr() + 4 * (j0 * n + j0), n, nb,
                                                       j0, info.data_ptr(), _stream(dev)),
               "cholesky_diag_block")


LDLQ_BLOCK_FIELDS = ("w", "comp", "wq", "err", "states", "n", "tile0", "reserved")


def check_ldlq_rows(rows, tiles: int) -> None:
    """Host check of one encoder call's ``exl3_ldlq_block`` rows before they
    are uploaded: every block's n is a positive multiple of 16, the first
    block starts at batch tile 0, each next one where the previous ends, and
    together they cover exactly ``tiles`` tiles. The kernels trust the table
    for their addresses, so a table that breaks this is refused here."""
    import numpy as np
    r = np.asarray(rows, dtype=np.int64).reshape(-1, len(LDLQ_BLOCK_FIELDS))
    check_ldlq_table(r, [(0, r.shape[0], tiles)])


def check_ldlq_table(rows, calls) -> None:
    """``check_ldlq_rows`` for a whole traversal at once: ``rows`` holds the
    ``exl3_ldlq_block`` rows of every call back to back and ``calls`` lists
    each call's (first row, row count, tiles), in order and covering every
    row."""
    import numpy as np
    r = np.asarray(rows, dtype=np.int64).reshape(-1, len(LDLQ_BLOCK_FIELDS))
    c = np.asarray(calls, dtype=np.int64).reshape(-1, 3)
    first, count, tiles = c[:, 0], c[:, 1], c[:, 2]
    if (count < 1).any():
        raise ValueError("an LDLQ call needs at least one block")
    if (not np.array_equal(first, np.concatenate([[0], np.cumsum(count)[:-1]]))
            or int(count.sum()) != r.shape[0]):
        raise ValueError("the calls must list the table's rows back to back")
    n = r[:, LDLQ_BLOCK_FIELDS.index("n")]
    tile0 = r[:, LDLQ_BLOCK_FIELDS.index("tile0")]
    if (n <= 0).any() or (n % 16).any():
        raise ValueError(f"block widths must be positive multiples of 16, got {n.tolist()}")
    # Each row's start within its call: the widths of the call's earlier rows.
    widths = n // 16
    ends = np.cumsum(widths)
    base = np.concatenate([[0], ends])[first]
    starts = ends - widths - np.repeat(base, count)
    call_bad = (np.add.reduceat((tile0 != starts).astype(np.int64), first) > 0) | (
        ends[first + count - 1] - base != tiles)
    if call_bad.any():
        i = int(np.flatnonzero(call_bad)[0])
        rows_i = slice(int(first[i]), int(first[i] + count[i]))
        raise ValueError(f"blocks must tile the batch back to back from 0 to {int(tiles[i])}: "
                         f"tile0 {tile0[rows_i].tolist()}, widths {widths[rows_i].tolist()}")
    for field in ("w", "comp", "wq", "err", "states"):
        if (r[:, LDLQ_BLOCK_FIELDS.index(field)] == 0).any():
            raise ValueError(f"NULL {field} address in an LDLQ block row")


def _ldlq_table(table, tiles_like, name: str) -> tuple:
    torch = _torch()
    dev = _check_device_tensor(tiles_like, name, tiles_like.dtype, 2)
    if tiles_like.size(1) != 256:
        raise RuntimeError(f"{name} must be (tiles, 256), got {tuple(tiles_like.shape)}")
    if (not isinstance(table, torch.Tensor) or table.dtype != torch.int64 or table.dim() != 2
            or table.size(1) != len(LDLQ_BLOCK_FIELDS) or not table.is_contiguous()
            or table.device != tiles_like.device or table.size(0) < 1):
        raise RuntimeError("the block table must be a contiguous (blocks, 8) int64 tensor on "
                           f"{tiles_like.device}")
    return dev, table.size(0), tiles_like.size(0)


def ldlq_gather(table, x) -> None:
    """Tile formation of one LDLQ encoder call (exl3_ldlq_gather): ``table``
    is the call's (blocks, 8) int64 ``exl3_ldlq_block`` rows on the device,
    whose addresses the caller has checked; ``x`` receives (tiles, 256)
    float32 tiles in tensor-core order."""
    torch = _torch()
    dev, nb, tiles = _ldlq_table(table, x, "x")
    if x.dtype != torch.float32:
        raise RuntimeError("x must be float32")
    with torch.cuda.device(dev):
        _check(load_library().exl3_ldlq_gather(table.data_ptr(), nb, tiles, x.data_ptr(),
                                               _stream(dev)), "ldlq_gather")


def ldlq_scatter(table, recon, idx) -> None:
    """Write-back of one LDLQ encoder call (exl3_ldlq_scatter) from the
    encoder's (tiles, 256) float32 reconstruction and int16 states."""
    torch = _torch()
    dev, nb, tiles = _ldlq_table(table, recon, "recon")
    if recon.dtype != torch.float32:
        raise RuntimeError("recon must be float32")
    _check_buffer(idx, "idx", torch.int16, tuple(recon.shape), dev)
    with torch.cuda.device(dev):
        _check(load_library().exl3_ldlq_scatter(table.data_ptr(), nb, tiles, recon.data_ptr(),
                                                idx.data_ptr(), _stream(dev)), "ldlq_scatter")


_EXT: Optional[QuantizeExtension] = None


def extension() -> QuantizeExtension:
    global _EXT
    if _EXT is None:
        _EXT = QuantizeExtension()
    return _EXT
