"""Host logic of the LDLQ traversal (exl3_intel_arc_quantizer_amd/ldlq.py) on
the CPU, with a deterministic grid quantiser standing in for the tile
encoder: the torch traversal against the numpy oracle's (ldlq.py:163-309),
and ldlq_lockstep against separate runs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ldlq_ref


def _grid_np(tiles):
    return np.round(tiles * 4.0) / np.float32(4.0), np.zeros(tiles.shape, np.uint16)


def _grid_torch(tiles):
    q = torch.round(tiles * 4.0) / 4.0
    # A state that depends on the tile values, so a misrouted block shows.
    return q, (q * 4.0).to(torch.int16)


def _problem(k, n, seed):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((k, n)).astype(np.float32)
    X = rng.standard_normal((4 * k, k)).astype(np.float32)
    H = (X.T @ X) / np.float32(X.shape[0]) + np.float32(0.05) * np.eye(k, dtype=np.float32)
    L, _, _ = ldlq_ref.block_ldl(H.astype(np.float32))
    return W, L


def test_ldlq_matches_oracle_traversal():
    from exl3_intel_arc_quantizer_amd.ldlq import ldlq
    W, L = _problem(256, 128, 1)
    got = ldlq(torch.from_numpy(W), torch.from_numpy(L), _grid_torch, buf_size_k=64)
    want, _ = ldlq_ref.ldlq(W, L, _grid_np, buf=64)
    np.testing.assert_allclose(got.weight_q.numpy(), want, rtol=0, atol=1e-6)
    assert got.encoder_calls == 16 and got.encoded.shape == (16, 8, 256)


def test_lockstep_equals_separate_runs():
    from exl3_intel_arc_quantizer_amd.ldlq import ldlq, ldlq_lockstep
    probs = [_problem(256, 128, 2), _problem(128, 256, 3), _problem(256, 384, 4)]
    calls = []

    def grid(tiles):
        calls.append(tiles.shape[0])
        return _grid_torch(tiles)

    tp = [(torch.from_numpy(W), torch.from_numpy(L)) for W, L in probs]
    together = ldlq_lockstep(tp, grid, buf_size_k=64)
    # 16 steps; the 128-row problem stops after 8.
    assert calls == [8 + 16 + 24] * 8 + [8 + 24] * 8
    for (W, L), res in zip(tp, together):
        alone = ldlq(W, L, _grid_torch, buf_size_k=64)
        assert torch.equal(res.weight_q, alone.weight_q)
        assert torch.equal(res.encoded, alone.encoded)
        assert res.encoder_calls == alone.encoder_calls == W.shape[0] // 16


def test_ldlq_rejects_bad_shapes_and_encoder_output():
    from exl3_intel_arc_quantizer_amd.ldlq import ldlq, ldlq_lockstep
    W, L = _problem(128, 128, 5)
    Wt, Lt = torch.from_numpy(W), torch.from_numpy(L)
    with pytest.raises(ValueError, match="multiple of 128"):
        ldlq(Wt[:, :64], Lt, _grid_torch)
    with pytest.raises(ValueError, match="L must be"):
        ldlq(Wt, Lt[:64, :64], _grid_torch)
    with pytest.raises(ValueError, match="buf_size_k"):
        ldlq(Wt, Lt, _grid_torch, buf_size_k=24)
    with pytest.raises(ValueError, match="encode_tiles must return"):
        ldlq(Wt, Lt, lambda t: (t[:-1], t[:-1]))
    assert ldlq_lockstep([], _grid_torch) == []


def test_lockstep_schedule_balances_calls():
    """lockstep_schedule: as many calls as the longest walk has blocks, every
    walk advancing exactly once per block, in order; a 9B-class layer's
    projections (q, k, v, o, gate, up: 256 blocks; down: 768) spread over
    768 calls of at most 1024 tiles instead of 256 calls of 2432 and 512
    of 256."""
    from exl3_intel_arc_quantizer_amd.ldlq import LOCKSTEP_ROUND_TILES, lockstep_schedule
    blocks = [256, 256, 256, 256, 256, 256, 768]
    tiles = [256, 64, 64, 256, 768, 768, 256]
    sched = lockstep_schedule(blocks, tiles)
    assert len(sched) == 768
    assert [sum(w in call for call in sched) for w in range(7)] == blocks
    loads = [sum(tiles[w] for w in call) for call in sched]
    assert max(loads) == 1024 and min(loads) == 896
    assert all(call == sorted(set(call)) for call in sched)
    rng = np.random.default_rng(7)
    for _ in range(50):
        nw = int(rng.integers(1, 9))
        b = [int(x) for x in rng.integers(1, 40, nw)]
        t = [int(x) for x in rng.integers(1, 900, nw)]
        sched = lockstep_schedule(b, t)
        assert len(sched) == max(b)
        assert [sum(w in call for call in sched) for w in range(nw)] == b
        target = max(LOCKSTEP_ROUND_TILES,
                     -(-(-(-sum(x * y for x, y in zip(b, t)) // max(b))) // LOCKSTEP_ROUND_TILES)
                     * LOCKSTEP_ROUND_TILES)
        left = list(b)
        for c, call in enumerate(sched):
            forced = [w for w in range(nw) if left[w] == len(sched) - c]
            assert set(forced) <= set(call)
            load = sum(t[w] for w in call)
            assert load <= max(target, sum(t[w] for w in forced) + max(t)), (b, t, c)
            for w in call:
                left[w] -= 1
    assert lockstep_schedule([], []) == []


def test_lanes_and_union_of_intervals():
    """The two-lane split (longest walks, the rest) and the union length the
    overlapping encoder calls are scaled to."""
    from exl3_intel_arc_quantizer_amd.ldlq import _lanes_of, _union_seconds

    def walk(b, t):
        return type("W", (), {"blocks": [0] * b, "tiles_n": t})()

    nine_b = [walk(256, 256), walk(256, 64), walk(256, 64), walk(256, 256), walk(256, 768),
              walk(256, 768), walk(768, 256)]
    assert _lanes_of(nine_b) == [[6], [0, 1, 2, 3, 4, 5]]
    assert _lanes_of([walk(16, 8), walk(16, 32)]) == [[0, 1]]
    assert _union_seconds([(0.0, 1.0), (0.5, 2.0), (3.0, 4.0), (3.5, 3.6)]) == pytest.approx(3.0)
    assert _union_seconds([]) == 0.0


def _block(n, tile0, w=1):
    return [w, 2, 3, 4, 5, n, tile0, 0]


def test_block_table_check_covers_every_call():
    """check_ldlq_table (the host guard of the GPU traversal's block table,
    one vectorised pass for every call) accepts back-to-back blocks and
    names the first call that breaks a rule: a block start, a call's total,
    a width, an empty or misplaced call, a NULL address; check_ldlq_rows is
    the same check for one call."""
    from exl3_intel_arc_quantizer_amd._native import check_ldlq_rows, check_ldlq_table
    good = [_block(48, 0), _block(32, 3), _block(64, 0)]
    check_ldlq_table(good, [(0, 2, 5), (2, 1, 4)])
    check_ldlq_rows(good[:2], 5)
    cases = [
        ([_block(48, 0), _block(32, 2), _block(64, 0)], [(0, 2, 5), (2, 1, 4)], "0 to 5"),
        (good, [(0, 2, 6), (2, 1, 4)], "0 to 6"),
        ([_block(48, 0), _block(32, 3), _block(64, 1)], [(0, 2, 5), (2, 1, 4)], "0 to 4"),
        ([_block(40, 0), _block(32, 3), _block(64, 0)], [(0, 2, 5), (2, 1, 4)], "multiples of 16"),
        (good, [(0, 2, 5), (1, 1, 4)], "back to back"),
        (good, [(0, 0, 0), (0, 2, 5), (2, 1, 4)], "at least one block"),
        ([_block(48, 0), _block(32, 3), _block(64, 0, w=0)], [(0, 2, 5), (2, 1, 4)], "NULL w"),
    ]
    for rows, calls, msg in cases:
        with pytest.raises(ValueError, match=msg):
            check_ldlq_table(rows, calls)
    with pytest.raises(ValueError, match="0 to 4"):
        check_ldlq_rows(good[:2], 4)
