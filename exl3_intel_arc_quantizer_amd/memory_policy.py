"""Reserve-based admission policy for encoder scratch on a discrete MI355X.

Counterpart of exl3_quant/memory_policy.py:194-421 with the same names
(``MemorySnapshot``, ``capture_snapshot``, ``MemoryPressureError``,
``MemoryPolicy``, env overrides). What changes for 288 GB of dedicated HBM3E:

* the binding figure is the device's free HBM (``torch.cuda.mem_get_info``);
  host RAM is a separate pool and no longer the tighter of two overlapping
  counters (the reference's integrated-GPU rule, memory_policy.py:210-215);
* the device counters fall when the process commits memory, so by default the
  live allocation is *not* subtracted a second time
  (``reflect_outstanding`` defaults to True; ``EXL3_MEMORY_REFLECT_OUTSTANDING=0``
  restores the reference's subtraction);
* the default reserve is 8 GiB (``EXL3_MEMORY_RESERVE_GIB`` /
  ``EXL3_MEMORY_RESERVE_BYTES`` override it, as in the reference).
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Optional

BYTES_PER_MIB = 1024 ** 2
BYTES_PER_GIB = 1024 ** 3

DEFAULT_RESERVE_BYTES = 8 * BYTES_PER_GIB
DEFAULT_SAFETY_SLACK_BYTES = 256 * BYTES_PER_MIB

ENV_RESERVE_BYTES = "EXL3_MEMORY_RESERVE_BYTES"
ENV_RESERVE_GIB = "EXL3_MEMORY_RESERVE_GIB"
ENV_REFLECT_OUTSTANDING = "EXL3_MEMORY_REFLECT_OUTSTANDING"

_MEMINFO_FIELDS = ("MemTotal", "MemFree", "MemAvailable", "Cached", "SwapTotal", "SwapFree",
                   "SwapCached")


def reflect_outstanding_counters() -> bool:
    """True unless EXL3_MEMORY_REFLECT_OUTSTANDING is set to a false value."""
    raw = os.environ.get(ENV_REFLECT_OUTSTANDING)
    if raw is None or not raw.strip():
        return True
    return raw.strip().lower() in ("1", "true", "yes", "on")


def default_reserve_bytes() -> int:
    """Configured reserve in bytes; the GiB form wins (memory_policy.py:78-92)."""
    raw_gib = os.environ.get(ENV_RESERVE_GIB)
    if raw_gib:
        try:
            return int(float(raw_gib) * BYTES_PER_GIB)
        except (TypeError, ValueError):
            pass
    raw_bytes = os.environ.get(ENV_RESERVE_BYTES)
    if raw_bytes:
        try:
            return int(raw_bytes)
        except (TypeError, ValueError):
            pass
    return DEFAULT_RESERVE_BYTES


def format_bytes(value: Optional[int]) -> str:
    if value is None:
        return "n/a"
    sign = "-" if value < 0 else ""
    value = abs(value)
    if value >= BYTES_PER_GIB:
        return f"{sign}{value / BYTES_PER_GIB:.2f} GiB"
    if value >= BYTES_PER_MIB:
        return f"{sign}{value / BYTES_PER_MIB:.1f} MiB"
    return f"{sign}{value} B"


def read_system_memory(path: str = "/proc/meminfo") -> dict:
    """Parse a /proc/meminfo-style file into byte counts (missing fields = 0)."""
    raw: dict = {}
    with open(path, "r", encoding="ascii") as handle:
        for line in handle:
            key, _, rest = line.partition(":")
            if key in _MEMINFO_FIELDS:
                raw[key] = int(rest.split()[0]) * 1024
    return {name: raw.get(name, 0) for name in _MEMINFO_FIELDS}


@dataclass(frozen=True)
class MemorySnapshot:
    """Host and device memory state at one point in time."""

    gpu_available: bool
    system_total_bytes: int
    system_available_bytes: int
    system_free_bytes: int
    cached_bytes: int
    swap_total_bytes: int
    swap_free_bytes: int
    device_free_bytes: int
    device_total_bytes: int
    device_allocated_bytes: int
    device_reserved_bytes: int

    @property
    def binding_available_bytes(self) -> int:
        """Free device HBM when a GPU is present, else host available memory."""
        if self.gpu_available:
            return self.device_free_bytes
        return self.system_available_bytes

    def as_dict(self) -> dict:
        d = {name: getattr(self, name) for name in self.__dataclass_fields__}
        d["binding_available_bytes"] = self.binding_available_bytes
        return d


def capture_snapshot(device_index: int = 0, meminfo_path: Optional[str] = None) -> MemorySnapshot:
    """Capture host (/proc/meminfo) and device (torch.cuda) counters; works
    without a GPU."""
    system = read_system_memory(meminfo_path or "/proc/meminfo")
    gpu_available = False
    free = total = allocated = reserved = 0
    try:
        import torch

        if torch.cuda.is_available():
            free, total = (int(v) for v in torch.cuda.mem_get_info(device_index))
            # One read of the allocator's nested counters (memory_allocated /
            # memory_reserved each rebuild the flattened statistics dict).
            stats = torch.cuda.memory_stats_as_nested_dict(device_index)
            allocated = int(stats.get("allocated_bytes", {}).get("all", {}).get("current", 0))
            reserved = int(stats.get("reserved_bytes", {}).get("all", {}).get("current", 0))
            gpu_available = True
    except Exception:  # pragma: no cover - broken driver / CPU-only host
        gpu_available = False
    return MemorySnapshot(
        gpu_available=gpu_available,
        system_total_bytes=system["MemTotal"],
        system_available_bytes=system["MemAvailable"],
        system_free_bytes=system["MemFree"],
        cached_bytes=system["Cached"],
        swap_total_bytes=system["SwapTotal"],
        swap_free_bytes=system["SwapFree"],
        device_free_bytes=free,
        device_total_bytes=total,
        device_allocated_bytes=allocated,
        device_reserved_bytes=reserved,
    )


class MemoryPressureError(RuntimeError):
    """Raised when an allocation would breach the reserve (memory_policy.py:272-291)."""

    def __init__(self, message: str, need_bytes: int, usable_bytes: int,
                 snapshot: MemorySnapshot, context: str = ""):
        super().__init__(message)
        self.need_bytes = need_bytes
        self.usable_bytes = usable_bytes
        self.snapshot = snapshot
        self.context = context

    def as_dict(self) -> dict:
        return {"error": "MemoryPressureError", "context": self.context,
                "need_bytes": self.need_bytes, "usable_bytes": self.usable_bytes,
                "message": str(self), "snapshot": self.snapshot.as_dict()}


@dataclass(frozen=True)
class MemoryPolicy:
    """Admission policy (memory_policy.py:294-421)."""

    reserve_bytes: int = field(default_factory=default_reserve_bytes)
    safety_slack_bytes: int = DEFAULT_SAFETY_SLACK_BYTES
    max_single_alloc_bytes: Optional[int] = None
    reflect_outstanding: bool = field(default_factory=reflect_outstanding_counters)

    def usable_bytes(self, snapshot: MemorySnapshot, outstanding_bytes: int = 0) -> int:
        if outstanding_bytes < 0:
            raise ValueError(f"outstanding_bytes must be non-negative, got {outstanding_bytes}")
        pending = 0 if self.reflect_outstanding else outstanding_bytes
        return max(0, snapshot.binding_available_bytes - self.reserve_bytes - pending)

    def check(self, need_bytes: int, snapshot: MemorySnapshot, outstanding_bytes: int = 0,
              context: str = "") -> int:
        if need_bytes < 0:
            raise ValueError(f"need_bytes must be non-negative, got {need_bytes}")
        usable = self.usable_bytes(snapshot, outstanding_bytes)
        if self.max_single_alloc_bytes is not None and need_bytes > self.max_single_alloc_bytes:
            raise MemoryPressureError(
                f"single-allocation ceiling exceeded{self._ctx(context)}: need "
                f"{format_bytes(need_bytes)} > ceiling {format_bytes(self.max_single_alloc_bytes)}",
                need_bytes, usable, snapshot, context)
        if need_bytes > usable:
            detail = (f"; outstanding {format_bytes(outstanding_bytes)} already committed"
                      if outstanding_bytes else "")
            raise MemoryPressureError(
                f"memory-pressure abort{self._ctx(context)}: need {format_bytes(need_bytes)} but "
                f"only {format_bytes(usable)} usable (binding available "
                f"{format_bytes(snapshot.binding_available_bytes)}, reserve "
                f"{format_bytes(self.reserve_bytes)}{detail})",
                need_bytes, usable, snapshot, context)
        return usable

    def check_after_commit(self, snapshot: MemorySnapshot,
                           pre_snapshot: Optional[MemorySnapshot] = None,
                           expected_bytes: int = 0, context: str = "post-commit") -> None:
        """Allocator growth must cover the request; the reserve floor must hold
        (memory_policy.py:366-408)."""
        if pre_snapshot is not None and expected_bytes > 0:
            growth = snapshot.device_allocated_bytes - pre_snapshot.device_allocated_bytes
            if growth < expected_bytes:
                raise MemoryPressureError(
                    f"allocator commitment failure{self._ctx(context)}: expected at least "
                    f"{format_bytes(expected_bytes)} allocated growth, observed only "
                    f"{format_bytes(growth)}",
                    expected_bytes, self.usable_bytes(snapshot), snapshot, context)
        floor = self.reserve_bytes - self.safety_slack_bytes
        if snapshot.binding_available_bytes < floor:
            raise MemoryPressureError(
                f"reserve breached{self._ctx(context)}: binding available "
                f"{format_bytes(snapshot.binding_available_bytes)} < floor {format_bytes(floor)} "
                f"(reserve {format_bytes(self.reserve_bytes)}, slack "
                f"{format_bytes(self.safety_slack_bytes)})",
                0, self.usable_bytes(snapshot), snapshot, context)

    def describe(self, snapshot: MemorySnapshot) -> dict:
        return {"reserve_bytes": self.reserve_bytes,
                "safety_slack_bytes": self.safety_slack_bytes,
                "max_single_alloc_bytes": self.max_single_alloc_bytes,
                "usable_bytes": self.usable_bytes(snapshot), "snapshot": snapshot.as_dict()}

    @staticmethod
    def _ctx(context: str) -> str:
        return f" [{context}]" if context else ""
