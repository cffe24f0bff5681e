"""ScratchArena lifecycle on the GPU (reference tests/test_xpu_quantizer.py:
333-476, xpu_quantizer.py:172-506): bounded residency with eviction and
reuse across K, batch halving on allocation failure with the encoder still
bit-exact, clean rejection when even B = 1 cannot be admitted, the
single-allocation ceiling, no double residency during the halving retries
and no leaked scratch after a failed acquisition. Scratch sizes follow this
encoder's layout (ScratchEstimator.estimate_scratch), not the reference's
byte formula."""

from __future__ import annotations

import gc

import numpy as np
import pytest

from oracle import c_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def test_bounded_eviction_and_reuse_across_k(torch_mod):
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import ScratchArena, XPUTrellisEncoder
    from exl3_intel_arc_quantizer_amd.scratch_estimator import ScratchEstimator
    torch = torch_mod
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    start = torch.cuda.memory_allocated()
    arena = ScratchArena(default_cap_b=4)
    tiles = np.random.default_rng(15).normal(0.0, 1.0, size=(4, 256)).astype(np.float32)
    try:
        for K in (2, 2, 3, 4, 2, 3, 2):
            print(f"arena K={K}", flush=True)
            XPUTrellisEncoder(K=K, cb=2, arena=arena).encode_batch(tiles, requested_b=4)
            want = ScratchEstimator.estimate_scratch(k=K, b=4, t=256).total_bytes
            assert arena.resident_bytes == want, K
        assert arena.reuses == 1          # the second K = 2
        assert arena.evictions == 5       # every change of K
        assert arena.allocations == 6
    finally:
        arena.release()
    assert arena.resident_bytes == 0
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == start
    assert len(arena.history) >= 7
    assert {e.action for e in arena.history} >= {"allocate", "reuse", "release"}


def test_batch_halving_and_clean_rejection(torch_mod):
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import ScratchArena, XPUTrellisEncoder
    from exl3_intel_arc_quantizer_amd.memory_policy import (BYTES_PER_GIB, BYTES_PER_MIB,
                                                            MemoryPolicy, MemoryPressureError)
    from exl3_intel_arc_quantizer_amd.scratch_estimator import ScratchEstimator
    tiles = np.random.default_rng(13).normal(0.0, 1.0, size=(16, 256)).astype(np.float32)

    def fail_above_4(b):
        if b > 4:
            raise RuntimeError(f"simulated allocator failure at B={b}")

    arena = ScratchArena(default_cap_b=16)
    enc = XPUTrellisEncoder(K=3, cb=2, arena=arena)
    try:
        bd = enc.encode_batch_detailed(tiles, requested_b=16, allocator_hook=fail_above_4)
        assert bd.admitted_b == 4 and bd.num_chunks == 4
        assert arena.retries >= 2                      # 16 -> 8 -> 4
        assert [e.admitted_b for e in arena.history if e.action == "retry-shrink"] == [8, 4]
        ref = c_oracle.encode_tiles(tiles, K=3, cb=2, pre_permute=True)
        np.testing.assert_array_equal(bd.output_indices, ref.output_indices)
    finally:
        arena.release()

    # A reserve larger than the device leaves no room even for B = 1.
    impossible = ScratchArena(policy=MemoryPolicy(reserve_bytes=100_000 * BYTES_PER_GIB))
    with pytest.raises(MemoryPressureError):
        XPUTrellisEncoder(K=2, cb=2, arena=impossible).encode_batch(tiles, requested_b=4)
    assert impossible.resident_bytes == 0

    # A single-allocation ceiling caps B. A slot is one allocation (terminal
    # costs and cost rows together), so the ceiling counts a tile's whole
    # scratch: here 4 tiles' worth, and 3.5 tiles' worth admits 3 (query)
    # and 2 (halving from 16).
    per_b = ScratchEstimator.estimate_scratch(k=3, b=1, t=256).total_bytes
    for limit, query, halved in ((4 * per_b, 4, 4), (7 * per_b // 2, 3, 2)):
        ceiling = ScratchArena(policy=MemoryPolicy(reserve_bytes=4 * BYTES_PER_GIB,
                                                   max_single_alloc_bytes=limit))
        try:
            assert ceiling.adaptive_batch_capacity(k=3, requested_b=16) == query
            costs, edges, adm = ceiling.acquire(k=3, requested_b=16)
            assert adm == halved
            assert ceiling.resident_bytes == halved * per_b <= limit
            # Both views live in the one slot, costs first, rows after.
            assert costs.shape == (halved, 2, 65536 >> 3) and edges.shape[0] == halved
            assert edges.data_ptr() == costs.data_ptr() + costs.numel() * 2
        finally:
            ceiling.release()
    assert 4 * per_b < 64 * BYTES_PER_MIB
    tiny = ScratchArena(policy=MemoryPolicy(reserve_bytes=4 * BYTES_PER_GIB,
                                            max_single_alloc_bytes=per_b - 1))
    with pytest.raises(MemoryPressureError, match="ceiling"):
        tiny.adaptive_batch_capacity(k=3, requested_b=16)
    with pytest.raises(MemoryPressureError, match="ceiling"):
        tiny.acquire(k=3, requested_b=16)
    assert tiny.resident_bytes == 0 and tiny.retries == 4     # 16, 8, 4, 2 -> 1


def test_retry_path_holds_one_attempt_at_a_time(torch_mod):
    """A post-commit failure at B = 8 frees the B = 8 buffers before B = 4 is
    allocated, and the arena ends holding exactly B = 4's scratch."""
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import ScratchArena
    from exl3_intel_arc_quantizer_amd.memory_policy import MemoryPolicy, MemoryPressureError
    from exl3_intel_arc_quantizer_amd.scratch_estimator import ScratchEstimator
    torch = torch_mod
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    pre = torch.cuda.memory_allocated()

    class FailAtB8(MemoryPolicy):
        def check_after_commit(self, snapshot, pre_snapshot=None, expected_bytes=0, context=""):
            if "B=8" in context:
                raise MemoryPressureError("simulated post-commit failure at B=8", 0, 0, snapshot,
                                          context)
            return super().check_after_commit(snapshot, pre_snapshot, expected_bytes, context)

    arena = ScratchArena(policy=FailAtB8())
    seen = []
    try:
        _, _, adm = arena.acquire(k=3, requested_b=8,
                                  allocator_hook=lambda b: seen.append(
                                      (b, torch.cuda.memory_allocated())))
        assert adm == 4
        assert [b for b, _ in seen] == [8, 4]
        # Nothing of the B = 8 attempt is left when B = 4 allocates.
        assert seen[1][1] == seen[0][1] <= pre
        want = ScratchEstimator.estimate_scratch(k=3, b=4, t=256).total_bytes
        assert torch.cuda.memory_allocated() == seen[1][1] + want
        assert arena.resident_bytes == want
    finally:
        arena.release()


def test_failed_acquisition_frees_all_scratch(torch_mod):
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import ScratchArena
    from exl3_intel_arc_quantizer_amd.memory_policy import MemoryPolicy, MemoryPressureError
    torch = torch_mod
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    pre = torch.cuda.memory_allocated()

    class AlwaysFail(MemoryPolicy):
        def check_after_commit(self, snapshot, pre_snapshot=None, expected_bytes=0, context=""):
            raise MemoryPressureError("simulated post-commit failure", 0, 0, snapshot, context)

    arena = ScratchArena(policy=AlwaysFail())
    with pytest.raises(MemoryPressureError, match="simulated post-commit failure") as info:
        arena.acquire(k=3, requested_b=1)
    assert torch.cuda.memory_allocated() == pre
    assert arena.resident_bytes == 0
    assert "simulated" in str(info.value)
