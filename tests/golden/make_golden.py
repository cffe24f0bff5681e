"""Generate the golden encoder vectors from the reference's own CPU encoder.

This script is the only place that executes reference code. It runs in the
build container (where the reference checkout is mounted read-only) and writes
small ``.npz`` fixtures next to itself; the fixtures, not the reference, are
what the test-suite and the GPU box see.

Reference functions pinned here (they have no closed form; every other part
of the path is pinned by closed forms, invariants or known answers):

* ``ReferenceTrellisEncoder.encode_tile`` (reference_encoder.py:253-324),
  i.e. ``forward`` (:130-204), ``argmin_cost`` (:206-214) and ``backward``
  (:216-251) on concrete inputs, including which branch wins exact ties;
* the K=5..8 behaviour that no reference device test exercises;
* the edge-case tiles of tests/test_xpu_quantizer.py:163-174;
* the L=160 rows of tests/test_xpu_quantizer.py:117-131;
* ``codebook_lut`` as a full-table hash (trellis_format.py:41-81).

Usage (container only)::

    python tests/golden/make_golden.py [--reference /root/reference] [--jobs 8]
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from multiprocessing import Pool
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

_ENC_CACHE: dict = {}


def _encoder(K: int, cb: int, L: int):
    from exl3_quant.reference_encoder import ReferenceTrellisEncoder

    key = (K, cb, L)
    if key not in _ENC_CACHE:
        _ENC_CACHE[key] = ReferenceTrellisEncoder(K=K, cb=cb, tile_len=L)
    return _ENC_CACHE[key]


def _init_worker(ref_root: str) -> None:
    if ref_root not in sys.path:
        sys.path.insert(0, ref_root)


def _encode_job(job):
    tile, K, cb, L, pre_permute = job
    res = _encoder(K, cb, L).encode_tile(tile, pre_permute=pre_permute)
    return {
        "output_indices": np.asarray(res.output_indices, dtype=np.uint16),
        "reconstructed": np.asarray(res.reconstructed, dtype=np.float16).view(np.uint16),
        "reconstructed_perm": np.asarray(res.reconstructed_perm, dtype=np.float16).view(np.uint16),
        "packed": np.asarray(res.packed, dtype=np.uint16),
        "end_state": int(res.end_state),
        "path_cost": float(res.path_cost),
        "distortion": float(res.distortion),
        "mse": float(res.mse),
    }


def _forward_job(job):
    """Pin forward/argmin/backward individually on one tile."""
    tile16, K, cb, roll, pre_state = job
    enc = _encoder(K, cb, 256)
    edges = np.zeros((enc.L, enc.edges), dtype=np.uint16)
    costs = enc.forward(tile16, roll=roll, pre_state=pre_state, temp_edges=edges)
    best = enc.argmin_cost(costs)
    end_state, _, _ = enc.backward(edges, roll=roll, write=False, edge=best)
    return {
        "costs": np.asarray(costs, dtype=np.float16).view(np.uint16),
        "edges_sha256": hashlib.sha256(np.ascontiguousarray(edges).tobytes()).hexdigest(),
        "edges_rows_head": np.ascontiguousarray(edges[:4, :64]),
        "best_edge": int(best),
        "end_state": int(end_state),
    }


def _stack(results, tiles, meta):
    out = {"tiles": np.asarray(tiles, dtype=np.float32)}
    for name in ("output_indices", "reconstructed", "reconstructed_perm", "packed"):
        arrs = [r[name] for r in results]
        if all(a.size == arrs[0].size for a in arrs):
            out[name] = np.stack(arrs)
        else:
            # Ragged (packed words depend on K): zero-pad, keep the lengths.
            width = max(a.size for a in arrs)
            padded = np.zeros((len(arrs), width), dtype=arrs[0].dtype)
            for i, a in enumerate(arrs):
                padded[i, :a.size] = a
            out[name] = padded
            out[name + "_len"] = np.asarray([a.size for a in arrs], dtype=np.int64)
    for name in ("end_state", "path_cost", "distortion", "mse"):
        out[name] = np.asarray([r[name] for r in results],
                               dtype=np.float64 if name != "end_state" else np.int64)
    for key, value in meta.items():
        out[key] = np.asarray(value)
    return out


def build_jobs():
    """Every fixture set: (name, [(tile, K, cb, L, pre_permute)], meta)."""
    sets = []

    # Config 1 of the benchmark: 64 tiles N(0,1) seed 0, K=2, mul1, kernel order.
    rng = np.random.default_rng(0)
    c1 = rng.standard_normal((64, 256), dtype=np.float32).astype(np.float16).astype(np.float32)
    sets.append(("c1_k2_mul1", [(t, 2, 2, 256, False) for t in c1],
                 {"K": 2, "cb": 2, "L": 256, "pre_permute": False}))

    # K sweep x codebook x permute: 2 tiles per combination, N(0, 1.15).
    sweep_tiles, sweep_jobs, sweep_k, sweep_cb, sweep_pp = [], [], [], [], []
    for K in range(1, 9):
        for cb in (0, 1, 2):
            for pp in (False, True):
                seed = 1000 + 100 * K + 10 * cb + int(pp)
                t = np.random.default_rng(seed).normal(0.0, 1.15, size=(2, 256)).astype(np.float32)
                for tile in t:
                    sweep_tiles.append(tile)
                    sweep_jobs.append((tile, K, cb, 256, pp))
                    sweep_k.append(K)
                    sweep_cb.append(cb)
                    sweep_pp.append(pp)
    sets.append(("k_sweep", sweep_jobs,
                 {"K": sweep_k, "cb": sweep_cb, "pre_permute": sweep_pp, "L": 256}))

    # Heavy-tailed tiles at K=2..6 (mul1, kernel order): N(0,1) with 1% x4.
    ht_jobs, ht_k = [], []
    for K in (2, 3, 4, 5, 6):
        r = np.random.default_rng(2000 + K)
        t = r.standard_normal((4, 256), dtype=np.float32)
        mask = r.random((4, 256)) < 0.01
        t = np.where(mask, t * 4.0, t).astype(np.float16).astype(np.float32)
        for tile in t:
            ht_jobs.append((tile, K, 2, 256, False))
            ht_k.append(K)
    sets.append(("heavy_tail", ht_jobs, {"K": ht_k, "cb": 2, "L": 256, "pre_permute": False}))

    # Edge-case tiles (tests/test_xpu_quantizer.py:163-174) plus degenerate ones.
    r77 = np.random.default_rng(77)
    cases = {
        "zeros": np.zeros(256, dtype=np.float32),
        "constant": np.full(256, 0.5, dtype=np.float32),
        "outliers": np.where(np.arange(256) % 17 == 0, 25.0,
                             r77.normal(0.0, 0.5, size=256)).astype(np.float32),
        "alternating": np.tile(np.array([-1.5, 1.5], dtype=np.float32), 128),
        "huge": np.full(256, 60000.0, dtype=np.float32),
        "overflow_inf": np.full(256, 1.0e6, dtype=np.float32),
        "mixed_inf": np.where(np.arange(256) % 5 == 0, np.float32(np.inf),
                              np.float32(0.25)).astype(np.float32),
        "subnormal": (np.random.default_rng(5).integers(-40, 40, size=256) * 2.0 ** -24).astype(np.float32),
        "ramp": np.linspace(-4.0, 4.0, 256, dtype=np.float32),
    }
    ec_jobs, ec_names, ec_k, ec_pp = [], [], [], []
    for K in (2, 4, 6):
        for pp in (True, False):
            for name, tile in cases.items():
                ec_jobs.append((tile, K, 2, 256, pp))
                ec_names.append(name)
                ec_k.append(K)
                ec_pp.append(pp)
    sets.append(("edge_cases", ec_jobs,
                 {"name": ec_names, "K": ec_k, "pre_permute": ec_pp, "cb": 2, "L": 256}))

    # L = 160 rows (mul1 only, kernel order).
    l_jobs, l_k = [], []
    for K in (2, 3, 4):
        t = np.random.default_rng(160 + K).normal(0.0, 1.0, size=(2, 160)).astype(np.float32)
        for tile in t:
            l_jobs.append((tile, K, 2, 160, False))
            l_k.append(K)
    sets.append(("l160", l_jobs, {"K": l_k, "cb": 2, "L": 160, "pre_permute": False}))
    return sets


def build_forward_jobs():
    jobs, meta = [], []
    for K, roll, pre in ((3, 128, -1), (4, 0, 1234), (2, 128, -1), (6, 0, 777)):
        tile16 = np.random.default_rng(31 + K).normal(0.0, 0.8, size=256).astype(np.float16)
        jobs.append((tile16, K, 2, roll, pre))
        meta.append((K, roll, pre, tile16))
    return jobs, meta


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--jobs", type=int, default=os.cpu_count() or 1)
    args = ap.parse_args()

    _init_worker(args.reference)
    from exl3_quant.trellis_format import codebook_lut

    luts = {}
    for cb in (0, 1, 2):
        lut = codebook_lut(cb)
        u = lut.view(np.uint16)
        luts[str(cb)] = {
            "sha256": hashlib.sha256(u.tobytes()).hexdigest(),
            "distinct_levels": int(np.unique(lut.astype(np.float64)).size),
            "min_bits": int(lut[np.argmin(lut.astype(np.float64))].view(np.uint16)),
            "max_bits": int(lut[np.argmax(lut.astype(np.float64))].view(np.uint16)),
            "head_bits": [int(x) for x in u[:16]],
        }
    (HERE / "codebook_lut.json").write_text(json.dumps(luts, indent=1) + "\n")

    with Pool(args.jobs, initializer=_init_worker, initargs=(args.reference,)) as pool:
        for name, jobs, meta in build_jobs():
            t0 = time.perf_counter()
            results = pool.map(_encode_job, jobs, chunksize=1)
            np.savez_compressed(HERE / f"{name}.npz",
                                **_stack(results, [j[0] for j in jobs], meta))
            print(f"{name}: {len(jobs)} tiles in {time.perf_counter() - t0:.1f}s", flush=True)

        fjobs, fmeta = build_forward_jobs()
        fres = pool.map(_forward_job, fjobs, chunksize=1)
        out = {}
        for i, (res, (K, roll, pre, tile16)) in enumerate(zip(fres, fmeta)):
            out[f"case{i}_tile"] = tile16.view(np.uint16)
            out[f"case{i}_costs"] = res["costs"]
            out[f"case{i}_edges_head"] = res["edges_rows_head"]
            out[f"case{i}_meta"] = np.asarray([K, roll, pre, res["best_edge"], res["end_state"]],
                                              dtype=np.int64)
            out[f"case{i}_edges_sha256"] = np.asarray(res["edges_sha256"])
        np.savez_compressed(HERE / "forward_pass.npz", **out)
        print("forward_pass: done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
