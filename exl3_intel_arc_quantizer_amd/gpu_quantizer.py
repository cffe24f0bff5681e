"""MI355X tile encoder and bounded scratch arena (PyTorch-ROCm front end).

Counterpart of the reference's exl3_quant/xpu_quantizer.py with the same
public names — ``build_quantize_extension``, ``get_build_timings``,
``verify_tile_encoding_quality``, ``ScratchArenaLogEntry``, ``ScratchArena``,
``BatchEncodingBreakdown``, ``XPUTrellisEncoder`` — so ldlq/layer_quant/
converter-style callers work unchanged, with ``cuda:i`` devices instead of
``xpu:i``. ``GPUTrellisEncoder`` is an alias of ``XPUTrellisEncoder``.

Every encoder result (states, reconstruction, packed words, path cost,
distortion) is computed by the HIP kernels of ``libexl3_hip.so``; the host
only moves arrays and builds the per-tile ``EncodingResult`` records. There
is no CPU fallback.

Deviations from the reference, all deliberate:

* scratch layout: ``temp_edges`` is ``uint8 (B, ROWS, ROW)``: every
  stride-th fp16 cost row, plus the header, see include/exl3_encoder.h;
  sized by the new ScratchEstimator;
* the arena's default batch capacity is 4096 tiles (the reference used 64 for
  the Arc iGPU), enough for eight waves of 1024-thread workgroups on 256 CUs;
* traceback placement: ``gpu_resident`` runs the fused encoder;
  ``gpu_resident_split``, ``d2h_cpu`` and ``usm_host`` run the split
  forward/traceback passes on the GPU (the host modes existed to work around
  a slow device traceback on Arc); all four give identical results;
* ``sg_size`` is validated and ignored (wave64); ``force_global_costs=True``
  selects the reference-structured generic kernel;
* NaN inputs are rejected with ``ValueError``: the reference's NaN handling
  (a NaN at branch 0 sticks) has no counterpart in the integer-key minimum,
  and its numpy and SYCL encoders already disagree on NaN
  (docs/algorithm_contract.md:292). Finite and infinite inputs are bit-exact.
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable, List, Optional, Tuple

import numpy as np

from . import build as _build
from ._native import QuantizeExtension, load_library
from .memory_policy import MemoryPolicy, MemoryPressureError, capture_snapshot
from .reference_encoder import EncodingResult
from .scratch_estimator import ScratchEstimator, scratch_row_bytes, tile_rows
from .trellis_format import (CB_3INST, CB_MCG, CB_MUL1, codebook_lut, tensor_core_perm,
                             tensor_core_perm_inv)

TRACEBACK_MODES = ("gpu_resident", "gpu_resident_split", "d2h_cpu", "usm_host")

_EXT: Optional[QuantizeExtension] = None
_COLD_BUILD_SECONDS = 0.0
_WARM_LOAD_SECONDS = 0.0


def build_quantize_extension(verbose: bool = False, force_rebuild: bool = False):
    """Load (or, with ``force_rebuild``, first compile) the native encoder
    (xpu_quantizer.py:65-98). Raises when the library is missing."""
    global _EXT, _COLD_BUILD_SECONDS, _WARM_LOAD_SECONDS
    if _EXT is not None and not force_rebuild:
        return _EXT
    t0 = time.perf_counter()
    if force_rebuild:
        _build.build_native(force=True, verbose=verbose)
        _COLD_BUILD_SECONDS = _build.last_build_seconds()
    lib = load_library()
    _EXT = QuantizeExtension(lib)
    if not force_rebuild:
        _WARM_LOAD_SECONDS = time.perf_counter() - t0
    return _EXT


def get_build_timings() -> dict:
    return {"cold_build_seconds": _COLD_BUILD_SECONDS, "warm_load_seconds": _WARM_LOAD_SECONDS}


def verify_tile_encoding_quality(result: EncodingResult, reference: EncodingResult,
                                 cost_atol: float = 0.0, distortion_rtol: float = 1e-4) -> dict:
    """Tie-aware comparison of two encodings (xpu_quantizer.py:108-169): ring
    continuity, exact codebook reconstruction, end-state consistency, path
    cost within ``cost_atol`` and distortion within ``distortion_rtol``."""
    L = len(result.output_indices)
    K = result.K
    mask = (65536 >> K) - 1
    idx = np.asarray(result.output_indices).astype(np.int64)
    nxt = np.roll(idx, -1)
    breaks = np.flatnonzero((idx & mask) != (nxt >> K))
    ring_valid = breaks.size == 0
    broken_step = int(breaks[0]) if breaks.size else -1
    lut = codebook_lut(result.cb)
    rec_exact = bool(np.array_equal(np.asarray(result.reconstructed_perm).view(np.uint16),
                                    lut[idx].view(np.uint16)))
    end_state_valid = (int(idx[L - 1]) & mask) == result.end_state
    indices_identical = bool(np.array_equal(result.output_indices, reference.output_indices))
    cost_diff = abs(float(result.path_cost) - float(reference.path_cost))
    cost_ok = cost_diff <= cost_atol
    ref_dist = max(1e-12, float(reference.distortion))
    dist_rel_diff = abs(float(result.distortion) - float(reference.distortion)) / ref_dist
    dist_ok = dist_rel_diff <= distortion_rtol or cost_diff == 0.0
    return {
        "passed": ring_valid and rec_exact and end_state_valid and cost_ok and dist_ok,
        "indices_identical": indices_identical,
        "ring_valid": ring_valid,
        "broken_step": broken_step,
        "rec_exact": rec_exact,
        "end_state_valid": end_state_valid,
        "cost_diff": cost_diff,
        "distortion_rel_diff": dist_rel_diff,
    }


@dataclass
class ScratchArenaLogEntry:
    """One arena action with its memory context (the reference's record,
    xpu_quantizer.py:172-185)."""

    action: str                     # "allocate", "reuse", "evict", "retry-shrink", "release"
    k: int
    tile_len: int
    requested_b: int
    admitted_b: int
    scratch_bytes: int
    distinct_staging_bytes: int
    outstanding_xpu_bytes: int
    usable_budget_bytes: int
    snapshot: dict


def _halvings(b: int):
    """Candidate batch sizes b, b // 2, ..., 1."""
    while b > 1:
        yield b
        b //= 2
    yield 1


@dataclass(frozen=True)
class _Refusal:
    """Why one candidate batch was not admitted, as plain data: no
    exception, traceback or tensor outlives the attempt."""

    message: str
    need_bytes: int
    usable_bytes: int
    snapshot: object
    context: str
    from_policy: bool


@dataclass
class _Slot:
    """The arena's resident scratch: one device byte buffer holding the
    terminal costs (B, 2, E) fp16 followed by B tiles of cost rows."""

    key: Tuple[int, int, int, int]          # (device, K, L, B)
    storage: object
    temp_costs: object
    temp_edges: object

    @classmethod
    def carve(cls, key, storage, est) -> "_Slot":
        import torch

        _, k, tile_len, b = key
        split = est.costs_bytes                 # b * 4E: a multiple of 1 KiB
        costs = storage[:split].view(torch.float16).view(b, 2, est.states)
        edges = storage[split:].view(b, tile_rows(k, tile_len), scratch_row_bytes(k))
        return cls(key, storage, costs, edges)

    @property
    def nbytes(self) -> int:
        return int(self.storage.numel())

    def serves(self, device: int, k: int, tile_len: int, b: int) -> bool:
        return self.key[:3] == (device, k, tile_len) and self.key[3] >= b


class ScratchArena:
    """Scratch for ``temp_costs`` / ``temp_edges`` with at most one resident
    slot (the contract of xpu_quantizer.py:188-506).

    * ``acquire`` returns ``(temp_costs, temp_edges, admitted_b)``. A slot of
      the same (device, K, L) with at least the requested batch is handed
      back; any other resident slot is evicted first, so at most one is ever
      held.
    * A slot is ONE device allocation, costs first, then the cost rows (sizes
      from ``ScratchEstimator``), so an admission asks the memory policy
      about a single figure and its single-allocation ceiling bounds the
      slot.
    * Candidate batches run from the request down to 1, halving. A candidate
      the policy refuses, or whose allocation, hook or post-commit check
      fails, is dropped (its buffer freed and the allocator's cache
      trimmed) before the next is tried. When even one tile is refused the
      call raises ``MemoryPressureError``, built from plain data so that
      holding it keeps no frame, buffer or earlier exception alive.
    * Reuse is stream-ordered when ``synchronize_reuse=False``: device-
      resident callers that launch everything on one stream need no host
      synchronisation to recycle the slot. The host-array API synchronises.
    * ``history`` records every action with its memory context; the counters
      count reuses, evictions, allocations and halvings.
    """

    def __init__(self, policy: Optional[MemoryPolicy] = None, device_index: int = 0,
                 default_cap_b: int = 4096):
        self.policy = policy or MemoryPolicy()
        self.device_index = device_index
        self.default_cap_b = default_cap_b
        self._slot: Optional[_Slot] = None
        self.history: List[ScratchArenaLogEntry] = []
        self.high_water_scratch_bytes = 0
        self.evictions = 0
        self.reuses = 0
        self.allocations = 0
        self.retries = 0

    @property
    def current_key(self) -> Optional[Tuple[int, int, int, int]]:
        return None if self._slot is None else self._slot.key

    @property
    def resident_bytes(self) -> int:
        return 0 if self._slot is None else self._slot.nbytes

    # ------------------------------------------------------------ helpers

    def _target(self, requested_b: Optional[int]) -> int:
        b = self.default_cap_b if requested_b is None else int(requested_b)
        if b < 1:
            raise ValueError(f"requested_b must be >= 1, got {b}")
        return b

    def _budget(self, staging: int):
        """Snapshot, bytes the process holds beyond this arena's slot plus
        host staging, and the policy's admissible bytes given those."""
        snap = capture_snapshot(self.device_index)
        outstanding = max(0, snap.device_allocated_bytes - self.resident_bytes) + staging
        return snap, outstanding, self.policy.usable_bytes(snap, outstanding_bytes=outstanding)

    def _note(self, action: str, k: int, tile_len: int, requested: int, admitted: int,
              nbytes: int, staging: int, snap, usable: int) -> None:
        self.history.append(ScratchArenaLogEntry(
            action=action, k=k, tile_len=tile_len, requested_b=requested, admitted_b=admitted,
            scratch_bytes=nbytes, distinct_staging_bytes=staging,
            outstanding_xpu_bytes=snap.device_allocated_bytes, usable_budget_bytes=usable,
            snapshot=snap.as_dict()))

    def _drop(self, action: str) -> None:
        """Free the resident slot after the device has finished with it."""
        import torch

        slot, self._slot = self._slot, None
        if slot is None:
            return
        _, k, tile_len, b = slot.key
        torch.cuda.synchronize(self.device_index)
        del slot
        torch.cuda.empty_cache()
        snap, _, usable = self._budget(0)
        self._note(action, k, tile_len, b, 0, 0, 0, snap, usable)

    def _commit(self, k: int, tile_len: int, b: int, staging: int,
                hook: Optional[Callable[[int], None]]):
        """Try one candidate batch: a new ``_Slot`` or a ``_Refusal``."""
        import torch

        est = ScratchEstimator.estimate_scratch(k=k, b=b, t=tile_len)
        snap, outstanding, usable = self._budget(staging)
        storage = None
        try:
            self.policy.check(est.total_bytes, snap, outstanding_bytes=outstanding,
                              context=f"K={k} B={b} scratch admit")
            if hook is not None:
                hook(b)
            storage = torch.empty(est.total_bytes, dtype=torch.uint8,
                                  device=f"cuda:{self.device_index}")
            self.policy.check_after_commit(capture_snapshot(self.device_index),
                                           pre_snapshot=snap, expected_bytes=est.total_bytes,
                                           context=f"K={k} B={b} post-commit")
        except MemoryPressureError as exc:
            refusal = _Refusal(str(exc), exc.need_bytes, exc.usable_bytes, exc.snapshot,
                               exc.context, True)
        except Exception as exc:  # noqa: BLE001 - allocator or hook failure: try a smaller B
            refusal = _Refusal(f"{type(exc).__name__}: {exc}", est.total_bytes, usable, snap,
                               f"K={k} B={b} allocation", False)
        else:
            slot = _Slot.carve((self.device_index, k, tile_len, b), storage, est)
            self.allocations += 1
            self.high_water_scratch_bytes = max(self.high_water_scratch_bytes, slot.nbytes)
            after, _, left = self._budget(staging)
            self._note("allocate", k, tile_len, b, b, slot.nbytes, staging, after, left)
            return slot
        if storage is not None:
            storage = None
            torch.cuda.empty_cache()
        return refusal

    # ------------------------------------------------------------ contract

    def adaptive_batch_capacity(self, k: int, tile_len: int = 256,
                                requested_b: Optional[int] = None,
                                distinct_staging_bytes: int = 0) -> int:
        """Largest batch, at most the request, whose slot the policy would
        admit now (the reference's P1-11 query, xpu_quantizer.py:234-269).
        Raises ``MemoryPressureError`` when not even one tile fits."""
        target = self._target(requested_b)
        per_tile = ScratchEstimator.estimate_scratch(k=k, b=1, t=tile_len).total_bytes
        snap, outstanding, usable = self._budget(distinct_staging_bytes)
        room = usable
        if self.policy.max_single_alloc_bytes is not None:
            room = min(room, self.policy.max_single_alloc_bytes)
        if room < per_tile:
            self.policy.check(per_tile, snap, outstanding_bytes=outstanding,
                              context=f"adaptive_batch_capacity K={k} B=1")
        return max(1, min(target, room // per_tile))

    def release(self) -> None:
        """Synchronise the device and free the resident slot, if any."""
        self._drop("release")

    def acquire(self, k: int, tile_len: int = 256, requested_b: Optional[int] = None,
                distinct_staging_bytes: int = 0,
                allocator_hook: Optional[Callable[[int], None]] = None,
                synchronize_reuse: bool = True):
        """``(temp_costs, temp_edges, admitted_b)`` for ``requested_b`` tiles
        (default ``default_cap_b``) of bitrate ``k`` and length ``tile_len``.
        ``allocator_hook(b)`` runs before each allocation attempt; an
        exception from it counts as an allocation failure at that b.
        ``distinct_staging_bytes`` (host memory the caller will hold beside
        the scratch) is charged against the budget."""
        import torch

        target = self._target(requested_b)
        slot = self._slot
        if slot is not None and slot.serves(self.device_index, k, tile_len, target):
            if synchronize_reuse:
                torch.cuda.synchronize(self.device_index)
            self.reuses += 1
            snap, _, usable = self._budget(distinct_staging_bytes)
            self._note("reuse", k, tile_len, target, target, slot.nbytes,
                       distinct_staging_bytes, snap, usable)
            return slot.temp_costs[:target], slot.temp_edges[:target], target
        if slot is not None:
            del slot
            self.evictions += 1
            self._drop("evict")

        refusal: Optional[_Refusal] = None
        for b in _halvings(target):
            outcome = self._commit(k, tile_len, b, distinct_staging_bytes, allocator_hook)
            if isinstance(outcome, _Slot):
                self._slot = outcome
                return outcome.temp_costs, outcome.temp_edges, b
            refusal = outcome
            if b > 1:
                self.retries += 1
                self._note("retry-shrink", k, tile_len, b, b // 2,
                           ScratchEstimator.estimate_scratch(k=k, b=b, t=tile_len).total_bytes,
                           distinct_staging_bytes, refusal.snapshot, refusal.usable_bytes)
        reason = refusal.message if refusal.from_policy else (
            f"no scratch for K={k}, L={tile_len}: every batch from {target} down to 1 tile "
            f"failed; at B=1: {refusal.message}")
        raise MemoryPressureError(reason, refusal.need_bytes, refusal.usable_bytes,
                                  refusal.snapshot, refusal.context) from None


@dataclass
class BatchEncodingBreakdown:
    """Batch output and timing split (xpu_quantizer.py:509-526)."""

    results: List[EncodingResult]
    reconstructed_tiles: np.ndarray      # (N, L) float16, original order when pre-permuted
    reconstructed_perm: np.ndarray       # (N, L) float16, kernel order
    output_indices: np.ndarray           # (N, L) uint16
    admitted_b: int
    num_chunks: int
    total_seconds: float
    search_seconds: float
    traceback_seconds: float
    transfer_seconds: float
    postprocess_seconds: float
    traceback_mode: str
    sg_size: int
    force_global_costs: bool
    packed: Optional[np.ndarray] = None          # (N, 16K) uint16 storage words
    path_costs: Optional[np.ndarray] = None      # (N,) float32
    distortions: Optional[np.ndarray] = None     # (N,) float32
    end_states: Optional[np.ndarray] = None      # (N,) int64


class XPUTrellisEncoder:
    """MI355X encoder with the reference's API (xpu_quantizer.py:529-994)."""

    def __init__(self, K: int = 2, cb: int = CB_MUL1, tile_len: int = 256,
                 arena: Optional[ScratchArena] = None, device_index: int = 0,
                 sg_size: int = 32, force_global_costs: bool = False,
                 wave_cap_override: int = 0):
        if not 1 <= K <= 8:
            raise ValueError(f"K must be between 1 and 8, got {K}")
        if cb not in (CB_3INST, CB_MCG, CB_MUL1):
            raise ValueError(f"Unknown codebook {cb}")
        if tile_len not in (256, 160):
            raise ValueError(f"tile_len must be 256 or 160, got {tile_len}")
        if tile_len == 160 and cb != CB_MUL1:
            raise ValueError("tile_len=160 is only supported with CB_MUL1")
        if sg_size not in (16, 32):
            raise ValueError(f"sg_size must be 16 or 32, got {sg_size}")
        self.K = K
        self.cb = cb
        self.L = tile_len
        self.edges = 65536 >> K
        self.device_index = device_index
        self.sg_size = sg_size
        self.force_global_costs = force_global_costs
        self.wave_cap_override = wave_cap_override
        self.arena = arena or ScratchArena(device_index=device_index)
        self._pinned_bufs = {}
        self._lut = None
        if self.L == 256:
            self.perm = tensor_core_perm()
            self.inv_perm = tensor_core_perm_inv()
        else:
            self.perm = None
            self.inv_perm = None

    @property
    def lut(self) -> np.ndarray:
        """fp16 codebook (decoded on the GPU on first use)."""
        if self._lut is None:
            self._lut = codebook_lut(self.cb, self.device_index)
        return self._lut

    @property
    def mcg_flag(self) -> bool:
        return self.cb == CB_MCG

    @property
    def mul1_flag(self) -> bool:
        return self.cb == CB_MUL1

    @property
    def device(self) -> str:
        return f"cuda:{self.device_index}"

    def _pinned(self, key: str, nbytes: int):
        """A page-locked host byte buffer of at least ``nbytes``, kept per
        encoder and reused by later calls (each call synchronises before it
        returns, so no copy is in flight when the buffer is refilled)."""
        import torch

        buf = self._pinned_bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1), dtype=torch.uint8, pin_memory=True)
            self._pinned_bufs[key] = buf
        return buf[:nbytes]

    def encode_tile(self, tile: np.ndarray, pre_permute: bool = True,
                    traceback_mode: str = "gpu_resident") -> EncodingResult:
        raw = np.asarray(tile, dtype=np.float32).reshape(-1)
        if raw.size != self.L:
            raise ValueError(f"Tile must have {self.L} elements, got {raw.size}")
        return self.encode_batch_detailed(raw.reshape(1, self.L), pre_permute=pre_permute,
                                          requested_b=1,
                                          traceback_mode=traceback_mode).results[0]

    def encode_batch(self, tiles: np.ndarray, pre_permute: bool = True,
                     requested_b: Optional[int] = None,
                     traceback_mode: str = "gpu_resident") -> List[EncodingResult]:
        return self.encode_batch_detailed(tiles, pre_permute=pre_permute,
                                          requested_b=requested_b,
                                          traceback_mode=traceback_mode).results

    # ------------------------------------------------------------ device API

    def _flatten(self, arr_shape) -> Tuple[int, int]:
        if len(arr_shape) == 2:
            return int(arr_shape[0]), int(arr_shape[1])
        if len(arr_shape) == 3 and tuple(arr_shape[1:]) == (16, 16) and self.L == 256:
            return int(arr_shape[0]), 256
        raise ValueError(f"Unsupported tiles shape {tuple(arr_shape)} for L={self.L}")

    def _check_mode(self, n: int, width: int, pre_permute: bool, mode: str) -> None:
        if n <= 0:
            raise ValueError(f"num_tiles must be positive, got {n}")
        if width != self.L:
            raise ValueError(f"Expected tile length {self.L}, got {width}")
        if pre_permute and self.L != 256:
            raise ValueError("pre_permute=True is only defined for L=256")
        if mode not in TRACEBACK_MODES:
            raise ValueError(f"Unknown traceback_mode {mode!r}")

    def _run_chunks(self, ext, x_dev, out_w, out_i, temp_costs, temp_edges, admitted_b, mode,
                    timings, synchronize=True, traceback_policy=None):
        """Encode x_dev (n, L) kernel-order tiles chunk by chunk."""
        import torch

        n = x_dev.shape[0]
        num_chunks = 0
        if mode == "gpu_resident":
            # One C-ABI call; the library chunks by the scratch capacity.
            ts = time.perf_counter()
            ext.quantize_tiles(x_dev, out_w, out_i, temp_costs[:admitted_b],
                               temp_edges[:admitted_b], self.K, self.mcg_flag, self.mul1_flag,
                               self.sg_size, self.force_global_costs, self.wave_cap_override,
                               traceback_policy=traceback_policy)
            if synchronize:
                torch.cuda.synchronize(self.device_index)
                timings["search"] += time.perf_counter() - ts
            return -(-n // admitted_b)
        pre = torch.full((admitted_b,), -1, dtype=torch.int32, device=x_dev.device)
        ends = torch.empty((admitted_b,), dtype=torch.int32, device=x_dev.device)
        for start in range(0, n, admitted_b):
            stop = min(start + admitted_b, n)
            cn = stop - start
            num_chunks += 1
            c_in = x_dev[start:stop]
            c_costs = temp_costs[:cn]
            c_edges = temp_edges[:cn]
            c_w = out_w[start:stop]
            c_i = out_i[start:stop]
            ts = time.perf_counter()
            ext.quantize_tiles_forward_pass(c_in, c_costs, c_edges, pre, self.K, self.mcg_flag,
                                            self.mul1_flag, self.L // 2, 0, self.sg_size,
                                            self.force_global_costs)
            torch.cuda.synchronize(self.device_index)
            tb = time.perf_counter()
            ext.quantize_tiles_backward_pass(c_costs, c_edges, c_w, c_i, ends, cn, self.K,
                                             self.mcg_flag, self.mul1_flag, self.L // 2, 0,
                                             False, self.sg_size)
            torch.cuda.synchronize(self.device_index)
            ts2 = time.perf_counter()
            ext.quantize_tiles_forward_pass(c_in, c_costs, c_edges, ends, self.K, self.mcg_flag,
                                            self.mul1_flag, 0, 1, self.sg_size,
                                            self.force_global_costs)
            torch.cuda.synchronize(self.device_index)
            tb2 = time.perf_counter()
            ext.quantize_tiles_backward_pass(c_costs, c_edges, c_w, c_i, ends, cn, self.K,
                                             self.mcg_flag, self.mul1_flag, 0, 1, True,
                                             self.sg_size)
            torch.cuda.synchronize(self.device_index)
            te = time.perf_counter()
            timings["search"] += (tb - ts) + (tb2 - ts2)
            timings["traceback"] += (ts2 - tb) + (te - tb2)
        return num_chunks

    def encode_tensor(self, tiles, pre_permute: bool = False, requested_b: Optional[int] = None,
                      traceback_mode: str = "gpu_resident", finalize: bool = True,
                      allocator_hook: Optional[Callable[[int], None]] = None,
                      synchronize: bool = True, nan_count=None,
                      traceback_policy: Optional[str] = None) -> dict:
        """Encode an (n, L) float32 device tensor, keeping every output on the
        device. Returns a dict of device tensors: ``x`` (kernel-order fp16
        inputs as f32), ``reconstructed_perm`` (f32, kernel order),
        ``indices`` (int16 states), and with ``finalize``: ``packed``,
        ``path_cost``, ``distortion``, ``reconstructed`` (fp16 bits as int16,
        original order).

        NaN inputs are counted by the prepare kernel. Without ``nan_count`` the
        count is read back at once and a NaN raises ``ValueError`` before any
        encoding. With ``nan_count`` (device int32) the count accumulates
        there and the caller checks it later; the batch is encoded anyway
        (its outputs are meaningless, every index stays a valid state).
        ``synchronize=False`` (``gpu_resident`` only) launches everything on
        the current stream and returns without waiting: host ``timings`` stay
        zero and the scratch buffers are reused in stream order.
        ``traceback_policy`` ("auto", "rows", "stream"; None = the process
        default) picks the traceback kernel of this call (``gpu_resident``);
        results are identical."""
        import torch

        if not isinstance(tiles, torch.Tensor) or tiles.device.type != "cuda":
            raise ValueError("encode_tensor expects a GPU tensor")
        n, width = self._flatten(tiles.shape)
        self._check_mode(n, width, pre_permute, traceback_mode)
        if not synchronize and traceback_mode != "gpu_resident":
            raise ValueError("synchronize=False requires traceback_mode='gpu_resident'")
        raw = tiles.reshape(n, width).to(torch.float32).contiguous()
        ext = build_quantize_extension()
        timings = {"search": 0.0, "traceback": 0.0}
        x = torch.empty_like(raw)
        if nan_count is None:
            counter = torch.zeros(1, dtype=torch.int32, device=raw.device)
            ext.prepare_tiles(raw, x, pre_permute, counter)
            if int(counter.item()):
                raise ValueError("NaN tile values are not supported (see module docstring)")
        else:
            ext.prepare_tiles(raw, x, pre_permute, nan_count)
        desired_b = min(n, requested_b if requested_b is not None else self.arena.default_cap_b)
        temp_costs, temp_edges, admitted_b = self.arena.acquire(
            k=self.K, tile_len=self.L, requested_b=desired_b, allocator_hook=allocator_hook,
            synchronize_reuse=synchronize)
        out_w = torch.empty((n, self.L), dtype=torch.float32, device=raw.device)
        out_i = torch.empty((n, self.L), dtype=torch.int16, device=raw.device)
        num_chunks = self._run_chunks(ext, x, out_w, out_i, temp_costs, temp_edges, admitted_b,
                                      traceback_mode, timings, synchronize, traceback_policy)
        res = {"x": x, "reconstructed_perm": out_w, "indices": out_i, "admitted_b": admitted_b,
               "num_chunks": num_chunks, "timings": timings}
        if finalize:
            tp = time.perf_counter()
            packed = (torch.empty((n, 16 * self.K), dtype=torch.int16, device=raw.device)
                      if self.L == 256 else None)
            path_cost = torch.empty(n, dtype=torch.float32, device=raw.device)
            distortion = torch.empty(n, dtype=torch.float32, device=raw.device)
            recon = torch.empty((n, self.L), dtype=torch.int16, device=raw.device)
            ext.finalize_tiles(x, raw, out_w, out_i, packed, path_cost, distortion, recon,
                               self.K, pre_permute)
            if synchronize:
                torch.cuda.synchronize(self.device_index)
                timings["finalize"] = time.perf_counter() - tp
            res.update(packed=packed, path_cost=path_cost, distortion=distortion,
                       reconstructed=recon)
        return res

    def encode_batch_detailed(self, tiles: np.ndarray, pre_permute: bool = True,
                              requested_b: Optional[int] = None,
                              traceback_mode: str = "gpu_resident",
                              allocator_hook: Optional[Callable[[int], None]] = None,
                              build_results: bool = True) -> BatchEncodingBreakdown:
        """Host-array API (xpu_quantizer.py:611-994). ``build_results=False``
        skips the per-tile ``EncodingResult`` records (arrays only)."""
        import torch

        arr = np.asarray(tiles, dtype=np.float32)
        n, width = self._flatten(arr.shape)
        self._check_mode(n, width, pre_permute, traceback_mode)
        flat = arr.reshape(n, width)
        if np.isnan(flat).any():
            raise ValueError("NaN tile values are not supported (see module docstring)")

        t_total0 = time.perf_counter()
        t0 = time.perf_counter()
        # Through a reused pinned buffer: DMA-speed copies both ways.
        staging = self._pinned("in", n * width * 4).view(torch.float32).view(n, width)
        staging.numpy()[...] = flat
        raw_dev = staging.to(self.device, non_blocking=True)
        torch.cuda.synchronize(self.device_index)
        t_transfer = time.perf_counter() - t0

        enc = self.encode_tensor(raw_dev, pre_permute=pre_permute, requested_b=requested_b,
                                 traceback_mode=traceback_mode, finalize=True,
                                 allocator_hook=allocator_hook)
        tx = time.perf_counter()
        outs = [("idx", enc["indices"]), ("rec_perm", enc["reconstructed_perm"].to(torch.float16)),
                ("rec", enc["reconstructed"]), ("path_cost", enc["path_cost"]),
                ("distortion", enc["distortion"])]
        if enc["packed"] is not None:
            outs.append(("packed", enc["packed"]))
        sizes = [-(-t.numel() * t.element_size() // 16) * 16 for _, t in outs]
        host_buf = self._pinned("out", sum(sizes))
        host, off = {}, 0
        for (name, t), size in zip(outs, sizes):
            view = host_buf[off:off + t.numel() * t.element_size()].view(t.dtype).view(t.shape)
            view.copy_(t, non_blocking=True)
            host[name] = view
            off += size
        torch.cuda.synchronize(self.device_index)
        idx = host["idx"].numpy().view(np.uint16).copy()
        rec_perm = host["rec_perm"].numpy().copy()
        rec = host["rec"].numpy().view(np.float16).copy()
        packed = (host["packed"].numpy().view(np.uint16).copy() if "packed" in host
                  else np.zeros((n, 0), dtype=np.uint16))
        path_cost = host["path_cost"].numpy().copy()
        distortion = host["distortion"].numpy().copy()
        t_transfer += time.perf_counter() - tx
        total_seconds = time.perf_counter() - t_total0
        del raw_dev, enc["x"]

        t_post0 = time.perf_counter()
        end_states = idx[:, self.L - 1].astype(np.int64) & (self.edges - 1)
        results: List[EncodingResult] = []
        if build_results:
            # Python scalars and per-tile row views converted in bulk (the
            # same values and views as indexing tile by tile, at a third of
            # the host time).
            dists, costs, ends = distortion.tolist(), path_cost.tolist(), end_states.tolist()
            L = float(self.L)
            results = [EncodingResult(
                output_indices=i_row, reconstructed=r_row, reconstructed_perm=rp_row,
                packed=p_row, end_state=e, distortion=d, mse=d / L, path_cost=c, K=self.K,
                cb=self.cb)
                for i_row, r_row, rp_row, p_row, e, d, c in zip(
                    list(idx), list(rec), list(rec_perm), list(packed), ends, dists, costs)]
        post = time.perf_counter() - t_post0 + enc["timings"].get("finalize", 0.0)
        return BatchEncodingBreakdown(
            results=results, reconstructed_tiles=rec, reconstructed_perm=rec_perm,
            output_indices=idx, admitted_b=enc["admitted_b"], num_chunks=enc["num_chunks"],
            total_seconds=total_seconds + (time.perf_counter() - t_post0),
            search_seconds=enc["timings"]["search"],
            traceback_seconds=enc["timings"]["traceback"], transfer_seconds=t_transfer,
            postprocess_seconds=post, traceback_mode=traceback_mode, sg_size=self.sg_size,
            force_global_costs=self.force_global_costs, packed=packed, path_costs=path_cost,
            distortions=distortion, end_states=end_states)


GPUTrellisEncoder = XPUTrellisEncoder
