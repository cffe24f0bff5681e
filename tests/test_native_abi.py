"""The C-ABI library loads on the CPU, exports every symbol the public header
declares, and its host-only entry points behave (no GPU work is launched)."""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from exl3_intel_arc_quantizer_amd import _native, scratch_estimator
from exl3_intel_arc_quantizer_amd.build import LIB_PATH

from .conftest import REPO_ROOT

HEADERS = sorted((REPO_ROOT / "include").glob("*.h"))


def _declared_symbols():
    names = set()
    for header in HEADERS:
        text = header.read_text()
        names |= set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(exl3_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_library_built_in_tree():
    assert LIB_PATH.exists(), "run __graft_entry__.build() first"


def test_header_symbols_are_exported():
    lib = ctypes.CDLL(str(LIB_PATH))
    declared = _declared_symbols()
    assert len(HEADERS) == 2 and len(declared) >= 17
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/*.h but not exported"
    assert declared == _native.exported_symbols()


def test_version_and_empty_error():
    lib = _native.load_library()
    assert lib.exl3_version().decode().startswith("exl3-mi355x")


@pytest.mark.parametrize("K", range(1, 9))
def test_row_bytes_match_estimator(K):
    lib = _native.load_library()
    assert lib.exl3_scratch_row_bytes(K) == scratch_estimator.scratch_row_bytes(K)
    for L in (256, 160):
        assert (lib.exl3_scratch_edges_bytes(K, L, 3)
                == scratch_estimator.ScratchEstimator.estimate_scratch(k=K, t=L, b=3).edges_bytes)


@pytest.mark.parametrize("K", range(1, 9))
def test_cost_row_slots_are_a_permutation(K):
    """Every edge owns exactly one cost position of a stored row."""
    lib = _native.load_library()
    E = 65536 >> K
    step = max(1, E // 4096)
    edges = np.arange(0, E, step)
    slots = np.array([lib.exl3_cost_row_slot(K, int(e)) for e in edges])
    assert slots.min() >= 0 and slots.max() < E
    if step == 1:
        assert np.array_equal(np.sort(slots), np.arange(E))
    else:
        assert np.unique(slots).size == edges.size
    assert lib.exl3_cost_row_slot(K, E) == -1


@pytest.mark.parametrize("K", [1, 5, 6, 7])
def test_cost_row_positions_are_group_major(K):
    """Cost rows hold predecessor edge x = (k << (16-2K)) | h at (h << K) | k."""
    lib = _native.load_library()
    ks = 16 - 2 * K
    rng = np.random.default_rng(K)
    for x in rng.integers(0, 65536 >> K, size=64):
        k, h = int(x) >> ks, int(x) & ((1 << ks) - 1)
        assert lib.exl3_cost_row_slot(K, int(x)) == (h << K) | k


def _predecessors(edges, K):
    """Predecessor edges of each edge, branch k = 0 .. 2^K - 1 last:
    state (k << (16 - K)) | e, predecessor state >> K."""
    k = np.arange(1 << K)
    return ((k[None, :] << (16 - K)) | np.asarray(edges)[:, None]).reshape(-1) >> K


@pytest.mark.parametrize("K,stride,run", [(2, 5, 1024), (3, 3, 512), (4, 2, 64)])
def test_cost_rows_keep_traceback_trees_together(K, stride, run):
    """A stored row serves `stride` steps; the traceback reads, per stored
    row, the 2^(K stride) costs `stride` predecessor steps below one edge.
    The row layout keeps each edge's 2^K predecessors in one aligned run in
    branch order and a whole tree in aligned runs of `run` positions, and
    puts the LDS neighbours x, x + 1 (x even) at positions t and t + E/2
    (the forward pass stores both from one dword read)."""
    lib = _native.load_library()
    E = 65536 >> K
    pos = np.array([lib.exl3_cost_row_slot(K, x) for x in range(E)])
    assert np.array_equal(np.sort(pos), np.arange(E))
    edge_at = np.argsort(pos)
    assert np.array_equal(edge_at[E // 2:], edge_at[:E // 2] + 1)
    assert not (edge_at[:E // 2] & 1).any()
    rng = np.random.default_rng(K)
    for e in rng.integers(0, E, size=32):
        sib = pos[_predecessors([e], K)]
        assert sib[0] % (1 << K) == 0 and np.array_equal(sib, sib[0] + np.arange(1 << K))
        leaves = [int(e)]
        for _ in range(stride):
            leaves = _predecessors(leaves, K)
        p = np.sort(pos[leaves]).reshape(-1, run)
        assert (p[:, 0] % run == 0).all() and (p == p[:, :1] + np.arange(run)).all()


@pytest.mark.parametrize("K,cb,L,msg", [
    (0, 2, 256, "K must be in 1..8"),
    (9, 2, 256, "K must be in 1..8"),
    (2, 3, 256, "cb must be 0, 1, or 2"),
    (2, 2, 128, "tile length L must be 256 or 160"),
    (2, 1, 160, "L=160 is only supported with mul1"),
])
def test_quantize_rejects_bad_arguments_before_any_gpu_work(K, cb, L, msg):
    lib = _native.load_library()
    rc = lib.exl3_quantize_tiles(None, None, None, None, None, 1, 1, K, cb, L, 0, 0, None)
    assert rc != 0
    assert msg in lib.exl3_last_error().decode()


def test_forward_and_backward_reject_bad_arguments():
    lib = _native.load_library()
    assert lib.exl3_forward_pass(None, None, None, None, 1, 2, 2, 256, 300, 0, 0, None) != 0
    assert "roll" in lib.exl3_last_error().decode()
    assert lib.exl3_forward_pass(None, None, None, None, 1, 2, 2, 256, 0, 2, 0, None) != 0
    assert "cost_slot" in lib.exl3_last_error().decode()
    assert lib.exl3_backward_pass(None, None, None, None, None, 0, 2, 2, 256, 0, 0, 0,
                                  None) != 0
    assert "num_tiles" in lib.exl3_last_error().decode()
    assert lib.exl3_decode_codebook(5, None, None) != 0
    assert lib.exl3_pack_trellis(None, None, 0, 2, None) != 0
    assert lib.exl3_prepare_tiles(None, None, 1, 160, 1, None, None) != 0
    assert "pre_permute" in lib.exl3_last_error().decode()
    # Valid shapes with NULL device buffers are refused, never launched.
    assert lib.exl3_decode_codebook(2, None, None) != 0
    assert lib.exl3_prepare_tiles(None, None, 4, 256, 0, None, None) != 0
    assert b"NULL" in lib.exl3_last_error()
    assert lib.exl3_pack_trellis(None, None, 4, 2, None) != 0
    assert lib.exl3_unpack_trellis(None, None, 4, 2, None) != 0
    assert lib.exl3_probe_hfma(None, None, None, 4, 0, None) != 0
    assert lib.exl3_probe_hfma(None, None, None, 4, 7, None) != 0
    assert b"mode" in lib.exl3_last_error()
    assert lib.exl3_finalize_tiles(None, None, None, None, None, None, None, None, 4, 2, 256, 0,
                                   None) != 0
    assert lib.exl3_forward_pass(None, None, None, None, 4, 2, 2, 256, 0, 0, 0, None) != 0
    assert lib.exl3_backward_pass(None, None, None, None, None, 4, 2, 2, 256, 0, 0, 1, None) != 0
    assert lib.exl3_quantize_tiles(None, None, None, None, None, 4, 4, 2, 2, 256, 0, 0, None) != 0
    assert b"NULL" in lib.exl3_last_error()


def test_traceback_policy_switch():
    """exl3_set_traceback_policy only records the choice (no GPU work)."""
    lib = _native.load_library()
    assert lib.exl3_set_traceback_policy(3) == -1
    assert b"policy" in lib.exl3_last_error()
    assert _native.set_traceback_policy("rows") == "auto"
    assert _native.set_traceback_policy("stream") == "rows"
    assert _native.set_traceback_policy("auto") == "stream"
    with pytest.raises(ValueError):
        _native.set_traceback_policy("fast")


def test_per_call_traceback_choice_is_checked_on_the_host():
    """exl3_quantize_tiles_tb rejects a traceback choice outside -1..2 before
    any launch (dummy non-NULL pointers never reach a kernel), leaves the
    process default alone, and the Python facade rejects an unknown name
    before it looks at the tensors."""
    import torch
    lib = _native.load_library()
    p = 16
    assert _native.set_traceback_policy("rows") == "auto"
    try:
        for bad in (3, -2):
            assert lib.exl3_quantize_tiles_tb(p, p, p, p, p, 4, 4, 4, 2, 256, 0, 0, bad,
                                              None) != 0
            assert b"traceback must be -1, 0, 1 or 2" in lib.exl3_last_error()
        assert _native.set_traceback_policy("auto") == "rows"
    finally:
        _native.set_traceback_policy("auto")
    t = torch.zeros((1, 256), dtype=torch.float32)
    with pytest.raises(ValueError, match="policy must be one of"):
        _native.QuantizeExtension().quantize_tiles(t, t, t, t, t, 2, False, True,
                                                   traceback_policy="fast")


def test_layer_entry_points_reject_bad_arguments():
    """include/exl3_layer.h: every argument check runs on the host, before
    any launch (dummy non-NULL pointers never reach a kernel here)."""
    lib = _native.load_library()
    err = lambda: lib.exl3_last_error().decode()  # noqa: E731
    assert lib.exl3_hadamard128(None, None, 128, 128, 0, None) != 0 and "NULL" in err()
    assert lib.exl3_hadamard128(1, 1, 100, 128, 0, None) != 0 and "divisible by 128" in err()
    assert lib.exl3_hadamard128(1, 1, 128, 100, 1, None) != 0 and "divisible by 128" in err()
    assert lib.exl3_hadamard128(1, 1, 128, 128, 2, None) != 0 and "side" in err()
    assert lib.exl3_hadamard128(1, 1, 0, 128, 0, None) != 0 and "empty" in err()
    assert lib.exl3_block_rms_workspace(256, 384, 0, 32) == 384 * 8
    assert lib.exl3_block_rms_workspace(100, 70, 1, 32) == 100 * 3
    assert lib.exl3_block_rms_workspace(100, 70, 2, 32) == -1
    assert lib.exl3_block_rms(1, 1, 100, 70, 1, 32, 1, 299, None) != 0 and "workspace" in err()
    assert lib.exl3_block_rms(1, 1, 100, 70, 3, 32, 1, 10 ** 6, None) != 0 and "dim" in err()
    assert lib.exl3_block_rms(1, 1, 100, 70, 0, 0, 1, 10 ** 6, None) != 0 and "blocksize" in err()
    assert lib.exl3_block_rms(1, 1, 100, 70, 0, 32, None, 10 ** 6, None) != 0 and "NULL" in err()
    assert lib.exl3_cholesky_block_order() == 128
    assert lib.exl3_cholesky_diag_block(1, 256, 0, 0, 1, None) != 0 and "order" in err()
    assert lib.exl3_cholesky_diag_block(1, 256, 129, 0, 1, None) != 0 and "order" in err()
    assert lib.exl3_cholesky_diag_block(1, 64, 128, 0, 1, None) != 0 and "lda" in err()
    assert lib.exl3_cholesky_diag_block(1, 256, 128, -1, 1, None) != 0 and "offset" in err()
    assert lib.exl3_cholesky_diag_block(1, 256, 128, 0, None, None) != 0 and "NULL" in err()
    assert lib.exl3_ldlq_gather(1, 0, 16, 1, None) != 0 and "no blocks" in err()
    assert lib.exl3_ldlq_gather(1, 1, 0, 1, None) != 0 and "tile count" in err()
    assert lib.exl3_ldlq_gather(None, 1, 16, 1, None) != 0 and "NULL" in err()
    assert lib.exl3_ldlq_scatter(1, 1, 16, 1, None, None) != 0 and "NULL" in err()
    assert lib.exl3_ldlq_scatter(1, 1, -3, 1, 1, None) != 0 and "tile count" in err()


def test_ldlq_block_table_fields_match_the_header():
    """_native.LDLQ_BLOCK_FIELDS lists exl3_ldlq_block's int64 fields in the
    header's order (the ldlq driver builds the table row by row)."""
    text = (REPO_ROOT / "include" / "exl3_layer.h").read_text()
    body = text[text.index("typedef struct exl3_ldlq_block {"):text.index("} exl3_ldlq_block;")]
    fields = re.findall(r"int64_t (\w+);", body)
    assert tuple(fields) == _native.LDLQ_BLOCK_FIELDS
