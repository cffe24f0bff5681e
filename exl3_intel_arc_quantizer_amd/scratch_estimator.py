"""Scratch sizing for the MI355X encoder (cost-row layout).

Counterpart of exl3_quant/scratch_estimator.py:23-172 with the same class
and method names. The formula changes with the layout
(include/exl3_encoder.h, csrc/exl3_layout.h):

    S      = 65536 >> K                      edges per step
    row    = S * 2                           one fp16 cost per edge
    rows   = (T - 2) // stride + 1           every stride-th step
                                             (stride 8, 5, 3, 2, 1, 1, 1, 1)
           + ceil((16 + 2 T) / row)          header: fields and the T inputs
                                             (one row; two at K = 8)
    costs  = B * 2 * S * 2                   terminal fp16 costs of both passes
    edges  = B * rows * row

The reference's int16 layout, ``B * T * S * 2``, is still available by
passing ``bytes_per_edge`` explicitly (e.g. to compare the two). Per tile at
T = 256: K=1 2.06 MiB (reference 16 MiB), K=2 1.63 MiB (8 MiB), K=3 1.34 MiB
(4 MiB), K=4 1.01 MiB (2 MiB), K=5 1 MiB (1 MiB), K=6 512 KiB (512 KiB),
K=7 256 KiB (256 KiB), K=8 128.5 KiB (128 KiB).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

BYTES_PER_KIB = 1024
BYTES_PER_MIB = 1024 ** 2
BYTES_PER_GIB = 1024 ** 3

BYTES_PER_KB = 1000
BYTES_PER_MB = 1000 ** 2
BYTES_PER_GB = 1000 ** 3


HEADER_FIELD_BYTES = 16  # int32 terminal edge, end state, pre_state, spare


def uses_cost_rows(k: int) -> bool:
    """Every supported bitrate (K = 1..8) keeps fp16 cost rows."""
    return 1 <= k <= 8


def row_stride(k: int) -> int:
    """Steps between stored cost rows (exl3_layout.h row_stride)."""
    return {1: 8, 2: 5, 3: 3, 4: 2}.get(k, 1)


COST_BITS = 16  # one fp16 cost per edge and stored row


def scratch_row_bytes(k: int) -> int:
    """Bytes of one scratch row (exl3_scratch_row_bytes): E fp16 costs."""
    return (65536 >> k) * COST_BITS // 8


def tile_rows(k: int, t: int = 256) -> int:
    """Scratch rows per tile, header included (exl3_layout.h tile_rows)."""
    row = scratch_row_bytes(k)
    header = -(-(HEADER_FIELD_BYTES + 2 * t) // row)
    return (t - 2) // row_stride(k) + 1 + header


@dataclass(frozen=True)
class ScratchAllocation:
    """Memory breakdown of one scratch configuration (scratch_estimator.py:23-59)."""

    k: int
    states: int
    t: int
    b: int
    bytes_per_cost: int
    bits_per_edge: int
    costs_bytes: int
    edges_bytes: int
    total_bytes: int

    @property
    def costs_mib(self) -> float:
        return self.costs_bytes / BYTES_PER_MIB

    @property
    def costs_mb(self) -> float:
        return self.costs_bytes / BYTES_PER_MB

    @property
    def edges_gib(self) -> float:
        return self.edges_bytes / BYTES_PER_GIB

    @property
    def edges_gb(self) -> float:
        return self.edges_bytes / BYTES_PER_GB

    @property
    def total_gib(self) -> float:
        return self.total_bytes / BYTES_PER_GIB

    @property
    def total_gb(self) -> float:
        return self.total_bytes / BYTES_PER_GB


class ScratchEstimator:
    """Scratch estimator for the trellis encoder (scratch_estimator.py:62-172)."""

    @staticmethod
    def get_state_count(k: int) -> int:
        """S = 65536 >> K (scratch_estimator.py:66-74); the encoder accepts K in 1..8."""
        if k < 1 or k > 16:
            raise ValueError(f"Trellis parameter K must be between 1 and 16, got {k}")
        return 65536 >> k

    @classmethod
    def estimate_scratch(cls, k: int, t: int = 256, b: int = 256, bytes_per_cost: int = 2,
                         bytes_per_edge: Optional[int] = None) -> ScratchAllocation:
        """Scratch bytes for ``b`` tiles of length ``t``. ``bytes_per_edge=None``
        selects the layout of this encoder; an explicit value reproduces the
        reference's ``b*t*S*bytes_per_edge`` formula."""
        if b <= 0:
            raise ValueError(f"Batch size B must be positive, got {b}")
        if t <= 0:
            raise ValueError(f"Sequence length T must be positive, got {t}")
        states = cls.get_state_count(k)
        costs_bytes = b * 2 * states * bytes_per_cost
        if bytes_per_edge is None:
            if k > 8:
                raise ValueError(f"the encoder supports K in 1..8, got {k}")
            bits = COST_BITS
            edges_bytes = b * tile_rows(k, t) * scratch_row_bytes(k)
        else:
            bits = 8 * bytes_per_edge
            edges_bytes = b * t * states * bytes_per_edge
        return ScratchAllocation(k=k, states=states, t=t, b=b, bytes_per_cost=bytes_per_cost,
                                 bits_per_edge=bits, costs_bytes=costs_bytes,
                                 edges_bytes=edges_bytes, total_bytes=costs_bytes + edges_bytes)

    @classmethod
    def calculate_max_batch_size(
        cls,
        k: int,
        available_vram_bytes: int,
        vram_reserve_bytes: int = 8 * BYTES_PER_GIB,
        max_single_alloc_bytes: Optional[int] = None,
        t: int = 256,
        bytes_per_cost: int = 2,
        bytes_per_edge: Optional[int] = None,
    ) -> Tuple[int, ScratchAllocation]:
        """Largest B that fits ``available - reserve`` and the optional
        single-allocation ceiling (scratch_estimator.py:114-172). The MI355X
        defaults: 8 GiB reserve of 288 GB HBM3E, no single-allocation ceiling."""
        usable = available_vram_bytes - vram_reserve_bytes
        if usable <= 0:
            raise ValueError(
                f"Available VRAM ({available_vram_bytes / BYTES_PER_GIB:.2f} GiB) must exceed "
                f"reserve ({vram_reserve_bytes / BYTES_PER_GIB:.2f} GiB)")
        one = cls.estimate_scratch(k=k, t=t, b=1, bytes_per_cost=bytes_per_cost,
                                   bytes_per_edge=bytes_per_edge)
        max_b = usable // one.total_bytes
        if max_single_alloc_bytes is not None:
            max_b = min(max_b, max_single_alloc_bytes // one.edges_bytes)
        if max_b < 1:
            raise ValueError(
                f"Insufficient memory: minimum batch size B=1 requires "
                f"{one.total_bytes / BYTES_PER_MIB:.2f} MiB, which exceeds allowable memory budget.")
        return int(max_b), cls.estimate_scratch(k=k, t=t, b=int(max_b),
                                                bytes_per_cost=bytes_per_cost,
                                                bytes_per_edge=bytes_per_edge)
