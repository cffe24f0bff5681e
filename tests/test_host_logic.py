"""Host-side logic that needs no GPU: scratch sizing, memory policy, the
tensor-core permutation table, and argument validation of the encoder and
extension facade (reference tests/test_scratch.py, tests/test_memory_policy.py,
tests/test_xpu_quantizer.py:237-269)."""

from __future__ import annotations

import numpy as np
import pytest

from exl3_intel_arc_quantizer_amd import trellis_format
from exl3_intel_arc_quantizer_amd.gpu_quantizer import XPUTrellisEncoder
from exl3_intel_arc_quantizer_amd._native import QuantizeExtension
from exl3_intel_arc_quantizer_amd.memory_policy import (
    BYTES_PER_GIB, MemoryPolicy, MemoryPressureError, capture_snapshot, default_reserve_bytes,
    read_system_memory, reflect_outstanding_counters)
from exl3_intel_arc_quantizer_amd.scratch_estimator import (
    BYTES_PER_MIB, COST_BITS, ScratchEstimator, scratch_row_bytes)
from oracle import trellis_format_ref


def test_reference_formula_fixtures_still_reproducible():
    """tests/test_scratch.py:32-57 of the reference, via bytes_per_edge=2."""
    for k, states, edges_gib, costs_mib in ((1, 32768, 4.0, 32.0), (2, 16384, 2.0, 16.0),
                                            (3, 8192, 1.0, 8.0), (4, 4096, 0.5, 4.0)):
        a = ScratchEstimator.estimate_scratch(k=k, t=256, b=256, bytes_per_edge=2)
        assert a.states == states
        assert a.edges_gib == pytest.approx(edges_gib)
        assert a.costs_mib == pytest.approx(costs_mib)


# Stored cost rows (every stride-th of steps 0..254) plus the header, rows of
# E * 2 bytes; the header (16 bytes and 256 fp16 inputs) takes one row, two at
# K = 8 where a row is 512 bytes.
@pytest.mark.parametrize("k,per_tile", [(1, 33 * 65536), (2, 52 * 32768), (3, 86 * 16384),
                                        (4, 129 * 8192), (5, 256 * 4096), (6, 256 * 2048),
                                        (7, 256 * 1024), (8, 257 * 512)])
def test_layout_formula(k, per_tile):
    a = ScratchEstimator.estimate_scratch(k=k, t=256, b=10)
    assert a.edges_bytes == 10 * per_tile
    assert a.costs_bytes == 10 * 2 * (65536 >> k) * 2
    assert a.total_bytes == a.costs_bytes + a.edges_bytes
    assert scratch_row_bytes(k) * 8 == (65536 >> k) * COST_BITS
    assert a.bits_per_edge == COST_BITS


def test_estimator_validation_and_max_batch():
    with pytest.raises(ValueError):
        ScratchEstimator.estimate_scratch(k=0)
    with pytest.raises(ValueError):
        ScratchEstimator.estimate_scratch(k=3, b=0)
    with pytest.raises(ValueError):
        ScratchEstimator.estimate_scratch(k=3, t=-1)
    # 288 GB HBM, 8 GiB reserve, K=2: ~1.7 MiB per tile.
    max_b, alloc = ScratchEstimator.calculate_max_batch_size(k=2, available_vram_bytes=288 * 10 ** 9)
    assert alloc.total_bytes <= 288 * 10 ** 9 - 8 * BYTES_PER_GIB
    assert max_b == (288 * 10 ** 9 - 8 * BYTES_PER_GIB) // (52 * 32768 + 2 * 16384 * 2)
    max_b, _ = ScratchEstimator.calculate_max_batch_size(
        k=3, available_vram_bytes=64 * BYTES_PER_GIB, max_single_alloc_bytes=16 * BYTES_PER_MIB)
    assert max_b == 16 * BYTES_PER_MIB // (86 * 16384)
    with pytest.raises(ValueError):
        ScratchEstimator.calculate_max_batch_size(k=2, available_vram_bytes=BYTES_PER_GIB)


def test_meminfo_parsing_and_policy(tmp_path):
    p = tmp_path / "meminfo"
    p.write_text("MemTotal:       1000000 kB\nMemFree:         500000 kB\n"
                 "MemAvailable:    800000 kB\nCached: 100 kB\nBogus: 5 kB\n")
    sysmem = read_system_memory(str(p))
    assert sysmem["MemAvailable"] == 800000 * 1024 and sysmem["SwapTotal"] == 0
    snap = capture_snapshot(0, meminfo_path=str(p))
    pol = MemoryPolicy(reserve_bytes=100 * 1024 * 1024, reflect_outstanding=False)
    if not snap.gpu_available:
        assert snap.binding_available_bytes == 800000 * 1024
        usable = pol.usable_bytes(snap, outstanding_bytes=50 * 1024 * 1024)
        assert usable == 800000 * 1024 - 150 * 1024 * 1024
        with pytest.raises(MemoryPressureError) as ei:
            pol.check(10 ** 12, snap, context="unit")
        assert "unit" in str(ei.value) and ei.value.as_dict()["need_bytes"] == 10 ** 12
    ceiling = MemoryPolicy(reserve_bytes=0, max_single_alloc_bytes=10)
    with pytest.raises(MemoryPressureError):
        ceiling.check(11, snap)
    with pytest.raises(ValueError):
        pol.usable_bytes(snap, outstanding_bytes=-1)


def test_policy_env_overrides(monkeypatch):
    monkeypatch.setenv("EXL3_MEMORY_RESERVE_GIB", "1.5")
    assert default_reserve_bytes() == int(1.5 * BYTES_PER_GIB)
    monkeypatch.delenv("EXL3_MEMORY_RESERVE_GIB")
    monkeypatch.setenv("EXL3_MEMORY_RESERVE_BYTES", "12345")
    assert default_reserve_bytes() == 12345
    monkeypatch.delenv("EXL3_MEMORY_RESERVE_BYTES")
    assert default_reserve_bytes() == 8 * BYTES_PER_GIB
    assert reflect_outstanding_counters() is True
    for word, want in (("0", False), ("off", False), ("No", False), ("1", True),
                       (" TRUE ", True), ("on", True), ("", True)):
        monkeypatch.setenv("EXL3_MEMORY_REFLECT_OUTSTANDING", word)
        assert reflect_outstanding_counters() is want, word
    # A misspelt switch is an error, not a silent "on".
    for word in ("disable", "2", "tru"):
        monkeypatch.setenv("EXL3_MEMORY_REFLECT_OUTSTANDING", word)
        with pytest.raises(ValueError, match="EXL3_MEMORY_REFLECT_OUTSTANDING"):
            reflect_outstanding_counters()


def test_package_perm_matches_oracle():
    np.testing.assert_array_equal(trellis_format.tensor_core_perm(),
                                  trellis_format_ref.tensor_core_perm())
    np.testing.assert_array_equal(trellis_format.tensor_core_perm_inv(),
                                  trellis_format_ref.tensor_core_perm_inv())


def test_encoder_constructor_validation():
    """tests/test_xpu_quantizer.py:239-250 of the reference."""
    for kwargs in ({"K": 0}, {"K": 9}, {"K": 2, "cb": 99}, {"K": 2, "tile_len": 128},
                   {"K": 2, "cb": 1, "tile_len": 160}, {"K": 2, "sg_size": 8}):
        with pytest.raises(ValueError):
            XPUTrellisEncoder(**kwargs)
    enc = XPUTrellisEncoder(K=2)
    with pytest.raises(ValueError):
        enc.encode_tile(np.zeros(100, dtype=np.float32))
    with pytest.raises(ValueError):
        enc.encode_batch(np.zeros((0, 256), dtype=np.float32))
    with pytest.raises(ValueError):
        enc.encode_batch(np.zeros((2, 256), dtype=np.float32), traceback_mode="bad")
    with pytest.raises(ValueError):
        enc.encode_batch(np.full((1, 256), np.nan, dtype=np.float32))


def test_extension_validation_without_gpu():
    """quantize_xpu.cpp:73-101 checks raise RuntimeError."""
    import torch

    ext = QuantizeExtension()
    t = torch.zeros((1, 256), dtype=torch.float32)
    with pytest.raises(RuntimeError, match="ambiguous"):
        ext.quantize_tiles(t, t, t, t, t, 2, True, True)
    with pytest.raises(RuntimeError, match="GPU"):
        ext.quantize_tiles(t, t, t, t, t, 2, False, True)
    with pytest.raises(RuntimeError, match="cb must be"):
        ext.decode_codebook(7, torch.zeros(65536, dtype=torch.float16))


def _snap(device_free, system_available=64 * BYTES_PER_GIB, gpu=True, allocated=0):
    from exl3_intel_arc_quantizer_amd.memory_policy import MemorySnapshot
    return MemorySnapshot(gpu_available=gpu, system_total_bytes=128 * BYTES_PER_GIB,
                          system_available_bytes=system_available, system_free_bytes=0,
                          cached_bytes=0, swap_total_bytes=0, swap_free_bytes=0,
                          device_free_bytes=device_free if gpu else 0,
                          device_total_bytes=288 * 10 ** 9 if gpu else 0,
                          device_allocated_bytes=allocated, device_reserved_bytes=0)


def test_policy_binds_on_free_hbm():
    """memory_policy.py:194-421 with the discrete-HBM binding figure: free
    device memory on a GPU host (host RAM is a separate pool and does not
    bind, even when smaller), host available memory without a GPU."""
    assert _snap(200 * BYTES_PER_GIB, system_available=3 * BYTES_PER_GIB) \
        .binding_available_bytes == 200 * BYTES_PER_GIB
    assert _snap(0, system_available=10 * BYTES_PER_GIB, gpu=False) \
        .binding_available_bytes == 10 * BYTES_PER_GIB
    d = _snap(5).as_dict()
    assert d["binding_available_bytes"] == 5 and d["device_total_bytes"] == 288 * 10 ** 9


def test_policy_admission_boundary_and_outstanding():
    pol = MemoryPolicy(reserve_bytes=6 * BYTES_PER_GIB, reflect_outstanding=True)
    snap = _snap(10 * BYTES_PER_GIB)
    assert pol.usable_bytes(snap) == 4 * BYTES_PER_GIB
    assert pol.usable_bytes(_snap(3 * BYTES_PER_GIB)) == 0
    assert pol.check(4 * BYTES_PER_GIB, snap) == 4 * BYTES_PER_GIB      # exactly the budget
    with pytest.raises(MemoryPressureError) as ei:
        pol.check(4 * BYTES_PER_GIB + 1, snap, context="K=2 B=8")
    err = ei.value
    assert err.need_bytes == 4 * BYTES_PER_GIB + 1 and err.usable_bytes == 4 * BYTES_PER_GIB
    assert "memory-pressure abort [K=2 B=8]" in str(err) and "reserve" in str(err)
    assert err.as_dict()["context"] == "K=2 B=8"
    # The free-HBM counter already reflects live allocations by default;
    # with reflect_outstanding off they are subtracted and named.
    assert pol.usable_bytes(snap, outstanding_bytes=BYTES_PER_GIB) == 4 * BYTES_PER_GIB
    strict = MemoryPolicy(reserve_bytes=6 * BYTES_PER_GIB, reflect_outstanding=False)
    assert strict.usable_bytes(snap, outstanding_bytes=BYTES_PER_GIB) == 3 * BYTES_PER_GIB
    with pytest.raises(MemoryPressureError, match="1.00 GiB outstanding"):
        strict.check(3 * BYTES_PER_GIB + 1, snap, outstanding_bytes=BYTES_PER_GIB)
    with pytest.raises(ValueError):
        pol.check(-1, snap)


def test_policy_ceiling_and_post_commit():
    from exl3_intel_arc_quantizer_amd.memory_policy import BYTES_PER_MIB, format_bytes
    pol = MemoryPolicy(reserve_bytes=0, max_single_alloc_bytes=4 * BYTES_PER_GIB)
    snap = _snap(30 * BYTES_PER_GIB)
    pol.check(4 * BYTES_PER_GIB, snap)
    with pytest.raises(MemoryPressureError, match="single-allocation ceiling"):
        pol.check(4 * BYTES_PER_GIB + 1, snap)
    post = MemoryPolicy(reserve_bytes=6 * BYTES_PER_GIB, safety_slack_bytes=256 * BYTES_PER_MIB)
    post.check_after_commit(_snap(6 * BYTES_PER_GIB - 200 * BYTES_PER_MIB))   # within slack
    with pytest.raises(MemoryPressureError, match="reserve breached"):
        post.check_after_commit(_snap(6 * BYTES_PER_GIB - 300 * BYTES_PER_MIB))
    before, after = _snap(100 * BYTES_PER_GIB), _snap(99 * BYTES_PER_GIB, allocated=BYTES_PER_GIB)
    post.check_after_commit(after, pre_snapshot=before, expected_bytes=BYTES_PER_GIB)
    with pytest.raises(MemoryPressureError, match="allocator commitment failure"):
        post.check_after_commit(after, pre_snapshot=before, expected_bytes=BYTES_PER_GIB + 1)
    assert format_bytes(None) == "n/a" and format_bytes(512) == "512 B"
    assert format_bytes(3 * BYTES_PER_MIB // 2) == "1.5 MiB"
    assert format_bytes(-5 * BYTES_PER_GIB // 2) == "-2.50 GiB"
    assert post.describe(snap)["usable_bytes"] == 24 * BYTES_PER_GIB


def test_platform_memory_source(tmp_path):
    from exl3_intel_arc_quantizer_amd.memory_policy import (read_system_memory_platform,
                                                            read_system_memory_windows)
    live = read_system_memory_platform()
    assert live["MemTotal"] > 0 and live["MemAvailable"] <= live["MemTotal"]
    p = tmp_path / "m"
    p.write_text("MemTotal:       32 kB\nMemAvailable:   16 kB\n")
    assert read_system_memory_platform(str(p))["MemTotal"] == 32 * 1024
    with pytest.raises(OSError):
        read_system_memory_windows()
