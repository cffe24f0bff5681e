"""ctypes front end of ``oracle/libexl3_oracle.so`` — TEST INFRASTRUCTURE ONLY.

The C restatement (oracle/exl3_oracle.c) mirrors ReferenceTrellisEncoder
(exl3_quant/reference_encoder.py:99-324); this module gives it a batch API
that returns the same per-tile fields the reference's ``EncodingResult``
carries (indices, packed words, end state, path cost, reconstruction,
distortion), computed on the host.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .trellis_format_ref import swap16_storage, tensor_core_perm, tensor_core_perm_inv

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libexl3_oracle.so"
_LIB = None

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> Path:
    """Compile the C oracle with the committed Makefile."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.exl3o_codebook_lut.argtypes = [ctypes.c_int, _u16p]
        L.exl3o_codebook_lut.restype = None
        L.exl3o_half_from_double.argtypes = [ctypes.c_double]
        L.exl3o_half_from_double.restype = ctypes.c_uint16
        L.exl3o_fma_f16.argtypes = [_u16p, _u16p, _u16p, ctypes.c_int64]
        L.exl3o_fma_f16.restype = None
        L.exl3o_encode_tiles.argtypes = [_u16p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, _u16p, _u16p, _i32p, _u16p, _i32p,
                                         ctypes.c_int]
        L.exl3o_encode_tiles.restype = ctypes.c_int
        L.exl3o_forward_pass.argtypes = [_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, _u16p, _u16p,
                                         ctypes.c_void_p]
        L.exl3o_forward_pass.restype = ctypes.c_int
        L.exl3o_pack_tiles.argtypes = [_u16p, ctypes.c_int64, ctypes.c_int, _u16p]
        L.exl3o_pack_tiles.restype = None
        _LIB = L
    return _LIB


def default_threads() -> int:
    """OMP_NUM_THREADS when set (the GPU box pins it), else the CPUs this
    process may run on."""
    env = os.environ.get("EXL3_ORACLE_THREADS") or os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    if hasattr(os, "sched_getaffinity"):
        return len(os.sched_getaffinity(0))
    return os.cpu_count() or 1


def codebook_lut(cb: int) -> np.ndarray:
    out = np.empty(65536, dtype=np.uint16)
    lib().exl3o_codebook_lut(int(cb), out)
    return out.view(np.float16)


def fma_f16(dh: np.ndarray, cost: np.ndarray) -> np.ndarray:
    """fp16(dh*dh + cost) with one rounding, elementwise."""
    a = np.ascontiguousarray(dh, dtype=np.float16).view(np.uint16)
    c = np.ascontiguousarray(cost, dtype=np.float16).view(np.uint16)
    out = np.empty_like(a)
    lib().exl3o_fma_f16(a, c, out, a.size)
    return out.view(np.float16)


def forward_pass(tile16: np.ndarray, K: int, cb: int, roll: int, pre_state: int,
                 with_rows: bool = False):
    """One forward pass: returns (edges (L, E) uint16, terminal costs fp16) and,
    with ``with_rows``, the cost vector after every step (L, E) fp16 bits."""
    t = np.ascontiguousarray(tile16, dtype=np.float16).view(np.uint16)
    L = t.size
    E = 65536 >> K
    edges = np.empty((L, E), dtype=np.uint16)
    costs = np.empty(E, dtype=np.uint16)
    rows = np.empty((L, E), dtype=np.uint16) if with_rows else None
    rc = lib().exl3o_forward_pass(t, K, cb, L, roll, pre_state, edges, costs,
                                  rows.ctypes.data if with_rows else None)
    if rc != 0:
        raise RuntimeError(f"exl3o_forward_pass failed ({rc})")
    if with_rows:
        return edges, costs.view(np.float16), rows
    return edges, costs.view(np.float16)


def pack_tiles(states: np.ndarray, K: int) -> np.ndarray:
    """pack_trellis + swap16 for a (n, 256) batch."""
    s = np.ascontiguousarray(states, dtype=np.uint16).reshape(-1, 256)
    out = np.empty((s.shape[0], 16 * K), dtype=np.uint16)
    lib().exl3o_pack_tiles(s, s.shape[0], K, out)
    return out


@dataclass
class OracleBatch:
    """Batch outputs, field names as in the reference's EncodingResult."""

    output_indices: np.ndarray      # (n, L) uint16, kernel order
    reconstructed_perm: np.ndarray  # (n, L) fp16, kernel order
    reconstructed: np.ndarray       # (n, L) fp16, original order when pre-permuted
    packed: np.ndarray              # (n, 16K) uint16 (post-SWAP16), empty for L != 256
    end_state: np.ndarray           # (n,) int32
    path_cost: np.ndarray           # (n,) float32 value of fp16 c2[end_state]
    best_edge: np.ndarray           # (n,) int32 pass-1 terminal argmin
    distortion: np.ndarray          # (n,) float32
    inputs16: np.ndarray            # (n, L) fp16 kernel-order inputs that were encoded


def encode_tiles(tiles: np.ndarray, K: int, cb: int = 2, pre_permute: bool = False,
                 threads: int = 0) -> OracleBatch:
    """Encode a (n, L) float32 batch exactly as ReferenceTrellisEncoder.encode_tile
    does per tile (reference_encoder.py:253-324)."""
    raw = np.ascontiguousarray(tiles, dtype=np.float32)
    raw = raw.reshape(raw.shape[0], -1)
    n, L = raw.shape
    if pre_permute:
        if L != 256:
            raise ValueError("pre_permute requires L=256")
        x16 = raw[:, tensor_core_perm()].astype(np.float16)
    else:
        x16 = raw.astype(np.float16)
    x16 = np.ascontiguousarray(x16)
    idx = np.empty((n, L), dtype=np.uint16)
    rec = np.empty((n, L), dtype=np.uint16)
    end = np.empty(n, dtype=np.int32)
    pc = np.empty(n, dtype=np.uint16)
    best = np.empty(n, dtype=np.int32)
    threads = threads or default_threads()
    rc = lib().exl3o_encode_tiles(x16.view(np.uint16), n, K, cb, L, idx, rec, end, pc, best,
                                  threads)
    if rc != 0:
        raise RuntimeError(f"exl3o_encode_tiles failed ({rc})")
    rec16 = rec.view(np.float16)
    if L == 256:
        packed = pack_tiles(idx, K)
    else:
        packed = np.zeros((n, 0), dtype=np.uint16)
    if pre_permute:
        rec_orig = rec16[:, tensor_core_perm_inv()]
        orig = raw
    else:
        rec_orig = rec16
        orig = x16.astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        distortion = np.sum((orig - rec_orig.astype(np.float32)) ** 2, axis=1)
    return OracleBatch(
        output_indices=idx, reconstructed_perm=rec16, reconstructed=rec_orig, packed=packed,
        end_state=end, path_cost=pc.view(np.float16).astype(np.float32), best_edge=best,
        distortion=distortion.astype(np.float32), inputs16=x16)


__all__ = ["build", "codebook_lut", "fma_f16", "forward_pass", "pack_tiles", "encode_tiles",
           "OracleBatch", "swap16_storage"]
