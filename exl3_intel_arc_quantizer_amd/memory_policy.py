"""Admission control for encoder scratch in a discrete GPU's HBM.

Public names follow the reference's exl3_quant/memory_policy.py:194-421
(``MemorySnapshot``, ``capture_snapshot``, ``MemoryPressureError``,
``MemoryPolicy`` and the environment switches), so arena code and scripts
written against it keep working. The model behind them is this build's own.

On an MI355X the scratch arena lives in the GPU's 288 GB of HBM3E, a pool
that the host never shares. One figure therefore decides admission: the
device's free HBM as the driver reports it (``hipMemGetInfo`` through
``torch.cuda.mem_get_info``). Host RAM and swap are still recorded in
every snapshot, because logs and scripts read them, but they never bind.
On a host without a GPU the host's available RAM stands in for the device
figure, so the same arithmetic can be tested on a CPU.

A request is admitted when it fits into

    admissible = free HBM - reserve - (outstanding, if counted)

* The reserve is headroom that the encoder leaves for everything else in
  the process: the layer driver's Hessians, GEMM workspaces, the caching
  allocator's slack. The default is 8 GiB. ``EXL3_MEMORY_RESERVE_GIB``
  (a float) or ``EXL3_MEMORY_RESERVE_BYTES`` (an integer) override it, and
  the GiB form takes precedence.
* The HBM counter already falls when this process commits memory, so by
  default the caller's outstanding bytes are not subtracted a second time.
  ``EXL3_MEMORY_REFLECT_OUTSTANDING=0`` subtracts them anyway, for drivers
  whose counters lag behind the allocator.
* An optional ceiling bounds any single buffer.

After an allocation, ``check_after_commit`` confirms that the allocator
really grew by the requested bytes and that free HBM did not sink below
the reserve (minus a slack for counter noise).
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Optional

BYTES_PER_MIB = 1 << 20
BYTES_PER_GIB = 1 << 30

DEFAULT_RESERVE_BYTES = 8 * BYTES_PER_GIB
DEFAULT_SAFETY_SLACK_BYTES = 256 * BYTES_PER_MIB

ENV_RESERVE_BYTES = "EXL3_MEMORY_RESERVE_BYTES"
ENV_RESERVE_GIB = "EXL3_MEMORY_RESERVE_GIB"
ENV_REFLECT_OUTSTANDING = "EXL3_MEMORY_REFLECT_OUTSTANDING"

# /proc/meminfo keys recorded in a snapshot (the file states them in kB).
_HOST_KEYS = ("MemTotal", "MemFree", "MemAvailable", "Cached", "SwapTotal", "SwapFree",
              "SwapCached")
_FALSE_WORDS = frozenset(("0", "false", "no", "off"))
_TRUE_WORDS = frozenset(("1", "true", "yes", "on"))


def reflect_outstanding_counters() -> bool:
    """Whether the free-HBM counter already includes this process's live
    allocations: True when ``EXL3_MEMORY_REFLECT_OUTSTANDING`` is unset,
    empty or one of 1 / true / yes / on, False for 0 / false / no / off.
    Any other value raises ``ValueError``: a misspelt switch must not
    silently admit more scratch than the operator asked for."""
    value = os.environ.get(ENV_REFLECT_OUTSTANDING, "").strip().lower()
    if value == "" or value in _TRUE_WORDS:
        return True
    if value in _FALSE_WORDS:
        return False
    raise ValueError(f"{ENV_REFLECT_OUTSTANDING}={value!r} is not one of "
                     f"{sorted(_TRUE_WORDS | _FALSE_WORDS)}")


def default_reserve_bytes() -> int:
    """The reserve from the environment (GiB form first, then bytes); an
    unset or unparsable value falls through to the next source and finally
    to DEFAULT_RESERVE_BYTES."""
    sources = ((ENV_RESERVE_GIB, lambda s: int(float(s) * BYTES_PER_GIB)),
               (ENV_RESERVE_BYTES, int))
    for name, parse in sources:
        text = os.environ.get(name)
        if not text:
            continue
        try:
            return parse(text)
        except ValueError:
            continue
    return DEFAULT_RESERVE_BYTES


def format_bytes(value: Optional[int]) -> str:
    """Binary-unit rendering for messages: ``2.50 GiB``, ``12.0 MiB``, ``512 B``."""
    if value is None:
        return "n/a"
    magnitude = abs(value)
    sign = "-" if value < 0 else ""
    for unit, size, digits in (("GiB", BYTES_PER_GIB, 2), ("MiB", BYTES_PER_MIB, 1)):
        if magnitude >= size:
            return f"{sign}{magnitude / size:.{digits}f} {unit}"
    return f"{sign}{magnitude} B"


def read_system_memory(path: str = "/proc/meminfo") -> dict:
    """Host memory counters in bytes from a /proc/meminfo-style file; keys
    the file lacks read as 0, keys this module does not record are dropped."""
    found = {}
    with open(path, "r", encoding="ascii") as handle:
        for line in handle:
            key, sep, rest = line.partition(":")
            if sep and key in _HOST_KEYS:
                found[key] = int(rest.split()[0]) << 10
                if len(found) == len(_HOST_KEYS):
                    break  # the scratch arena snapshots once per encoder call
    return {key: found.get(key, 0) for key in _HOST_KEYS}


def read_system_memory_windows() -> dict:
    """The reference reads host counters through GlobalMemoryStatusEx on
    Windows. ROCm builds of this encoder run on Linux only."""
    raise OSError("host memory counters through GlobalMemoryStatusEx exist on Windows only; "
                  "this build reads /proc/meminfo")


def read_system_memory_platform(meminfo_path: Optional[str] = None) -> dict:
    """Host memory counters from ``meminfo_path`` or the platform's source
    (/proc/meminfo on Linux)."""
    if meminfo_path is None and os.name == "nt":  # pragma: no cover
        return read_system_memory_windows()
    return read_system_memory(meminfo_path or "/proc/meminfo")


@dataclass(frozen=True)
class MemorySnapshot:
    """Memory counters at one instant. Device fields come from the HIP
    runtime and torch's caching allocator, host fields from /proc/meminfo."""

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
        """The figure admission is decided on: free HBM on a GPU host (the
        device's memory is its own pool), host available RAM otherwise."""
        return self.device_free_bytes if self.gpu_available else self.system_available_bytes

    def as_dict(self) -> dict:
        # Every field is a scalar: a shallow copy is the whole record.
        record = dict(vars(self))
        record["binding_available_bytes"] = self.binding_available_bytes
        return record


def _device_counters(device_index: int):
    """(free, total, allocated, reserved) bytes of one GPU, or None without one."""
    try:
        import torch
        if not torch.cuda.is_available():
            return None
        free, total = torch.cuda.mem_get_info(device_index)
        # One read of the allocator's statistics serves both counters.
        stats = torch.cuda.memory_stats_as_nested_dict(device_index)
        current = lambda name: int(stats.get(name, {}).get("all", {}).get("current", 0))  # noqa: E731
        return int(free), int(total), current("allocated_bytes"), current("reserved_bytes")
    except Exception:  # pragma: no cover - broken driver
        return None


def capture_snapshot(device_index: int = 0, meminfo_path: Optional[str] = None) -> MemorySnapshot:
    """Read the host and device counters now (a host without a GPU gives
    zero device fields and ``gpu_available=False``)."""
    host = read_system_memory_platform(meminfo_path)
    device = _device_counters(device_index)
    free, total, allocated, reserved = device if device is not None else (0, 0, 0, 0)
    return MemorySnapshot(
        gpu_available=device is not None,
        system_total_bytes=host["MemTotal"], system_available_bytes=host["MemAvailable"],
        system_free_bytes=host["MemFree"], cached_bytes=host["Cached"],
        swap_total_bytes=host["SwapTotal"], swap_free_bytes=host["SwapFree"],
        device_free_bytes=free, device_total_bytes=total,
        device_allocated_bytes=allocated, device_reserved_bytes=reserved)


class MemoryPressureError(RuntimeError):
    """A scratch request that the policy refused, with the numbers behind
    the refusal: bytes asked for, bytes admissible, the snapshot and the
    caller's context label."""

    def __init__(self, message: str, need_bytes: int, usable_bytes: int,
                 snapshot: MemorySnapshot, context: str = ""):
        super().__init__(message)
        self.need_bytes = need_bytes
        self.usable_bytes = usable_bytes
        self.snapshot = snapshot
        self.context = context

    def as_dict(self) -> dict:
        return {"error": type(self).__name__, "context": self.context,
                "need_bytes": self.need_bytes, "usable_bytes": self.usable_bytes,
                "message": str(self), "snapshot": self.snapshot.as_dict()}


def _non_negative(name: str, value: int) -> None:
    if value < 0:
        raise ValueError(f"{name} must be non-negative, got {value}")


def _label(kind: str, context: str) -> str:
    return f"{kind} [{context}]" if context else kind


@dataclass(frozen=True)
class MemoryPolicy:
    """Reserve-based admission of scratch buffers (see the module docstring)."""

    reserve_bytes: int = field(default_factory=default_reserve_bytes)
    safety_slack_bytes: int = DEFAULT_SAFETY_SLACK_BYTES
    max_single_alloc_bytes: Optional[int] = None
    reflect_outstanding: bool = field(default_factory=reflect_outstanding_counters)

    def usable_bytes(self, snapshot: MemorySnapshot, outstanding_bytes: int = 0) -> int:
        """Bytes that may still be committed without touching the reserve."""
        _non_negative("outstanding_bytes", outstanding_bytes)
        counted = 0 if self.reflect_outstanding else outstanding_bytes
        return max(0, snapshot.binding_available_bytes - self.reserve_bytes - counted)

    def _refusal(self, need: int, usable: int, snapshot: MemorySnapshot,
                 outstanding: int, context: str) -> Optional[str]:
        ceiling = self.max_single_alloc_bytes
        if ceiling is not None and need > ceiling:
            return (f"{_label('single-allocation ceiling exceeded', context)}: one buffer of "
                    f"{format_bytes(need)} is above the {format_bytes(ceiling)} ceiling")
        if need <= usable:
            return None
        counted = "" if self.reflect_outstanding or not outstanding else \
            f" - {format_bytes(outstanding)} outstanding"
        return (f"{_label('memory-pressure abort', context)}: {format_bytes(need)} requested, "
                f"{format_bytes(usable)} admissible = "
                f"{format_bytes(snapshot.binding_available_bytes)} free - "
                f"{format_bytes(self.reserve_bytes)} reserve{counted}")

    def check(self, need_bytes: int, snapshot: MemorySnapshot, outstanding_bytes: int = 0,
              context: str = "") -> int:
        """Admit ``need_bytes`` or raise MemoryPressureError; returns the
        admissible budget the request was measured against."""
        _non_negative("need_bytes", need_bytes)
        usable = self.usable_bytes(snapshot, outstanding_bytes)
        reason = self._refusal(need_bytes, usable, snapshot, outstanding_bytes, context)
        if reason is not None:
            raise MemoryPressureError(reason, need_bytes, usable, snapshot, context)
        return usable

    def check_after_commit(self, snapshot: MemorySnapshot,
                           pre_snapshot: Optional[MemorySnapshot] = None,
                           expected_bytes: int = 0, context: str = "post-commit") -> None:
        """Confirm a commitment: the caching allocator grew by at least
        ``expected_bytes`` since ``pre_snapshot`` (when both are given), and
        free memory is still above the reserve less the slack."""
        if pre_snapshot is not None and expected_bytes > 0:
            grew = snapshot.device_allocated_bytes - pre_snapshot.device_allocated_bytes
            if grew < expected_bytes:
                raise MemoryPressureError(
                    f"{_label('allocator commitment failure', context)}: the allocator grew by "
                    f"{format_bytes(grew)}, the buffers need {format_bytes(expected_bytes)}",
                    expected_bytes, self.usable_bytes(snapshot), snapshot, context)
        floor = self.reserve_bytes - self.safety_slack_bytes
        left = snapshot.binding_available_bytes
        if left < floor:
            raise MemoryPressureError(
                f"{_label('reserve breached', context)}: {format_bytes(left)} free after the "
                f"commitment, below the {format_bytes(self.reserve_bytes)} reserve less "
                f"{format_bytes(self.safety_slack_bytes)} slack",
                0, self.usable_bytes(snapshot), snapshot, context)

    def describe(self, snapshot: MemorySnapshot) -> dict:
        """The policy's settings and its budget on ``snapshot``."""
        return {"reserve_bytes": self.reserve_bytes,
                "safety_slack_bytes": self.safety_slack_bytes,
                "max_single_alloc_bytes": self.max_single_alloc_bytes,
                "usable_bytes": self.usable_bytes(snapshot), "snapshot": snapshot.as_dict()}
