"""The oracle (numpy and C restatements) against the reference's own outputs.

The golden vectors in tests/golden/ were produced by the reference's
``ReferenceTrellisEncoder`` (exl3_quant/reference_encoder.py) and
``codebook_lut`` (exl3_quant/trellis_format.py) by tests/golden/make_golden.py.
"""

from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest

from oracle import c_oracle
from oracle.reference_encoder import ReferenceTrellisEncoder
from oracle.trellis_format_ref import codebook_lut

from .conftest import GOLDEN, load_golden


def _lut_meta():
    return json.loads((GOLDEN / "codebook_lut.json").read_text())


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_full_table_hash(cb):
    meta = _lut_meta()[str(cb)]
    for lut in (codebook_lut(cb), c_oracle.codebook_lut(cb)):
        u = np.ascontiguousarray(lut).view(np.uint16)
        assert hashlib.sha256(u.tobytes()).hexdigest() == meta["sha256"]
        assert int(np.unique(lut.astype(np.float64)).size) == meta["distinct_levels"]


def _assert_batch_matches(ob, g, sel=None, K=None):
    sel = slice(None) if sel is None else sel
    np.testing.assert_array_equal(ob.output_indices, g["output_indices"][sel])
    np.testing.assert_array_equal(ob.end_state, g["end_state"][sel])
    np.testing.assert_array_equal(ob.path_cost.astype(np.float64), g["path_cost"][sel])
    np.testing.assert_array_equal(ob.distortion.astype(np.float64), g["distortion"][sel])
    if "packed" in g:
        width = ob.packed.shape[1]
        np.testing.assert_array_equal(ob.packed, g["packed"][sel][:, :width])
    if "reconstructed" in g:
        np.testing.assert_array_equal(ob.reconstructed.view(np.uint16), g["reconstructed"][sel])


def test_c_oracle_config1():
    g = load_golden("c1_k2_mul1")
    ob = c_oracle.encode_tiles(g["tiles"], K=2, cb=2, pre_permute=False)
    _assert_batch_matches(ob, g)


def test_c_oracle_k_sweep_all_codebooks_and_orders():
    g = load_golden("k_sweep")
    for K in range(1, 9):
        for cb in (0, 1, 2):
            for pp in (False, True):
                sel = (g["K"] == K) & (g["cb"] == cb) & (g["pre_permute"] == pp)
                ob = c_oracle.encode_tiles(g["tiles"][sel], K=K, cb=cb, pre_permute=pp)
                _assert_batch_matches(ob, g, sel)


@pytest.mark.parametrize("name", ["heavy_tail", "edge_cases", "l160"])
def test_c_oracle_other_sets(name):
    g = load_golden(name)
    Ks = np.atleast_1d(g["K"])
    pps = np.atleast_1d(g["pre_permute"]) if g["pre_permute"].ndim else None
    n = g["tiles"].shape[0]
    for K in np.unique(Ks):
        for pp in ((False, True) if pps is not None else (bool(g["pre_permute"]),)):
            sel = Ks == K if Ks.size == n else np.ones(n, bool)
            if pps is not None:
                sel = sel & (pps == pp)
            if not sel.any():
                continue
            with np.errstate(over="ignore", invalid="ignore"):
                ob = c_oracle.encode_tiles(g["tiles"][sel], K=int(K), cb=int(g["cb"]),
                                           pre_permute=pp)
            _assert_batch_matches(ob, g, sel)


@pytest.mark.parametrize("row", [0, 17, 40, 63])
def test_numpy_oracle_config1_tiles(row):
    """The numpy restatement, op for op, on single tiles (slow: ~1 s/tile)."""
    g = load_golden("c1_k2_mul1")
    res = ReferenceTrellisEncoder(K=2, cb=2).encode_tile(g["tiles"][row], pre_permute=False)
    np.testing.assert_array_equal(res.output_indices, g["output_indices"][row])
    np.testing.assert_array_equal(res.packed, g["packed"][row])
    assert res.end_state == g["end_state"][row]
    assert res.path_cost == g["path_cost"][row]
    assert res.distortion == g["distortion"][row]


@pytest.mark.parametrize("K,cb,pp", [(1, 2, True), (3, 0, False), (5, 1, True), (8, 2, False)])
def test_numpy_oracle_sweep_tiles(K, cb, pp):
    g = load_golden("k_sweep")
    rows = np.flatnonzero((g["K"] == K) & (g["cb"] == cb) & (g["pre_permute"] == pp))
    res = ReferenceTrellisEncoder(K=K, cb=cb).encode_tile(g["tiles"][rows[0]], pre_permute=pp)
    np.testing.assert_array_equal(res.output_indices, g["output_indices"][rows[0]])
    np.testing.assert_array_equal(res.packed, g["packed"][rows[0]][:16 * K])
    assert res.path_cost == g["path_cost"][rows[0]]


def test_forward_pass_pins():
    """forward / argmin_cost / backward individually (reference_encoder.py:130-251)."""
    g = load_golden("forward_pass")
    i = 0
    while f"case{i}_tile" in g:
        K, roll, pre, best, end = (int(v) for v in g[f"case{i}_meta"])
        tile16 = g[f"case{i}_tile"].view(np.float16)
        edges, costs = c_oracle.forward_pass(tile16, K=K, cb=2, roll=roll, pre_state=pre)
        np.testing.assert_array_equal(costs.view(np.uint16), g[f"case{i}_costs"])
        assert hashlib.sha256(edges.tobytes()).hexdigest() == str(g[f"case{i}_edges_sha256"])
        enc = ReferenceTrellisEncoder(K=K, cb=2)
        assert enc.argmin_cost(costs) == best
        got_end, _, _ = enc.backward(edges, roll=roll, write=False, edge=best)
        assert got_end == end
        i += 1
    assert i == 4
