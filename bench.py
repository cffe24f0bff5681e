#!/usr/bin/env python
"""Encoder throughput on one MI355X: encoded 16x16 tiles/s and the fraction of
the packed-fp16 VALU roofline, with the CPU oracle timed beside it.

Workload: one 1024x1024 matrix of i.i.d. N(0,1)
fp16 values (seed 1), cut into 4096 16x16 tiles as the LDLQ loop forms them
(16-row blocks, tensor-core permutation), encoded at K=4 with the MUL1
codebook; K=2 is measured on the same matrix and reported beside it.
Synthetic data, inputs resident in HBM before the timed region. One step =
the full device-side encode of the batch: pass-1 forward, traceback, pass-2
forward, traceback (exl3_quantize_tiles) plus the finalize kernel (packing,
path cost, distortion). ``--sweep`` adds K=2..6 on the 4096x4096
heavy-tailed matrix of configs[2] (65536 tiles).

Roofline: algorithmic work per forward-pass launch = tiles * 256 steps *
65536 candidates * 3 fp16 element-ops (subtract, FMA, compare-select);
``achieved`` divides it by the forward kernel's mean duration measured with
HIP events on the stream the kernel runs on. Peak = 256 CU * 64 lanes * 2
(packed fp16) * 2.4 GHz = 78.64 T fp16 element-ops/s (the published
157.3 TFLOP/s fp16 vector rate counts each FMA twice).

``traffic``: HBM bytes per forward launch from the committed rocprofv3 PMC
summary (profiles/forward_pass_pmc_configs1.md): FETCH_SIZE x 2 + WRITE_SIZE
x 1.0 per dispatch, the factors a 1 GiB device copy reads on the same
counters; null when the summary has no row for the kernel.

    python bench.py [--steps 10] [--warmup 2] [--sweep] [--no-cpu-baseline]
    python bench.py --profile-forward --k-list 4,2   # forward launches only
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = ("encoded 16x16 tiles/sec at K=2 and K=4, 1 MI355X; % of fp16 VALU/LDS roofline")
PEAK_ELEM_OPS = 256 * 64 * 2 * 2.4e9          # fp16 element-ops/s
OPS_PER_TILE_PASS = 256 * 65536 * 3            # one forward pass


def config2_tiles() -> np.ndarray:
    rng = np.random.default_rng(1)
    W = rng.standard_normal((1024, 1024), dtype=np.float32).astype(np.float16).astype(np.float32)
    return W.reshape(64, 16, 64, 16).transpose(0, 2, 1, 3).reshape(4096, 256)


def config3_tiles() -> np.ndarray:
    rng = np.random.default_rng(2)
    W = rng.standard_normal((4096, 4096), dtype=np.float32)
    W = np.where(rng.random(W.shape) < 0.01, 4.0 * W, W)
    W = W.astype(np.float16).astype(np.float32)
    return W.reshape(256, 16, 256, 16).transpose(0, 2, 1, 3).reshape(65536, 256)


class DeviceBatch:
    """A batch prepared on the device with its scratch, ready to encode."""

    def __init__(self, raw_np, K, torch, ext, batch_cap=None):
        from exl3_intel_arc_quantizer_amd._native import edges_shape
        self.torch, self.ext, self.K = torch, ext, K
        self.n = raw_np.shape[0]
        self.raw = torch.from_numpy(raw_np).cuda()
        self.x = torch.empty_like(self.raw)
        ext.prepare_tiles(self.raw, self.x, True)
        cap = batch_cap or self.n
        self.cap = cap
        self.costs = torch.empty((cap, 2, 65536 >> K), dtype=torch.float16, device="cuda")
        self.edges = torch.empty(edges_shape(cap, K), dtype=torch.uint8, device="cuda")
        self.out_w = torch.empty((self.n, 256), dtype=torch.float32, device="cuda")
        self.out_i = torch.empty((self.n, 256), dtype=torch.int16, device="cuda")
        self.packed = torch.empty((self.n, 16 * K), dtype=torch.int16, device="cuda")
        self.pc = torch.empty(self.n, dtype=torch.float32, device="cuda")
        self.dist = torch.empty(self.n, dtype=torch.float32, device="cuda")
        self.rec = torch.empty((self.n, 256), dtype=torch.int16, device="cuda")
        self.pre = torch.full((cap,), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()

    def step(self):
        self.ext.quantize_tiles(self.x, self.out_w, self.out_i, self.costs, self.edges, self.K,
                                False, True)
        self.ext.finalize_tiles(self.x, self.raw, self.out_w, self.out_i, self.packed, self.pc,
                                self.dist, self.rec, self.K, True)

    def forward_only(self, n):
        self.ext.quantize_tiles_forward_pass(self.x[:n], self.costs[:n], self.edges[:n],
                                             self.pre[:n], self.K, False, True, 0, 1)


def time_steps(batch, steps, warmup, torch):
    for _ in range(warmup):
        batch.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        batch.step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


PMC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "forward_pass_pmc_configs1.md")


def pmc_traffic(K, tiles):
    """HBM bytes per forward launch of `tiles` tiles at bitrate K from the
    committed PMC summary (rows `| traffic | K | tiles | bytes |`), scaled
    linearly in the tile count; None if absent."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 4 and cells[0] == "traffic" and cells[1] == str(K):
                    return int(round(float(cells[3]) * tiles / float(cells[2])))
    except OSError:
        return None
    return None


def forward_kernel_name(K):
    """The forward kernel the fast path launches for bitrate K."""
    if 1 <= K <= 7:
        return f"acs_forward_rows<K={K}>"
    return "acs_forward_generic"


def forward_kernel_roofline(batch, torch, reps=3):
    """Mean duration of one forward-pass launch over the whole batch, timed
    with HIP events recorded on the launch stream."""
    n = min(batch.n, batch.cap)
    batch.forward_only(n)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        batch.forward_only(n)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    ops = n * OPS_PER_TILE_PASS
    achieved = ops / (ms * 1e-3)
    return {"bound": "valu", "achieved": round(achieved / 1e12, 3),
            "peak": round(PEAK_ELEM_OPS / 1e12, 3), "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_ELEM_OPS, 4), "traffic": pmc_traffic(batch.K, n),
            "kernel": forward_kernel_name(batch.K), "launch_ms": round(ms, 3),
            "tiles_per_launch": n,
            "ops_note": "fp16 element-ops: tiles*256 steps*65536 candidates*3 (sub, FMA, "
                        "compare-select); peak 256 CU*64 lanes*2 halves*2.4 GHz",
            "traffic_note": "HBM bytes per launch: rocprofv3 FETCH_SIZE*2 + WRITE_SIZE*1.0 "
                            "(copy-kernel calibration), profiles/forward_pass_pmc_configs1.md"}


def _numpy_encode_one(args):
    tile, K = args
    from oracle.reference_encoder import ReferenceTrellisEncoder
    ReferenceTrellisEncoder(K=K, cb=2).encode_tile(tile, pre_permute=True)
    return 0


def cpu_baseline_numpy(tiles, K, cores):
    """The numpy restatement of the reference encoder (oracle/reference_encoder.py,
    op for op the reference's reference_encoder.py), one tile per task on a
    pool of `cores` processes, on a bounded sample of the same workload. Run
    before the GPU is initialised (the pool forks)."""
    import multiprocessing as mp
    n = 4 * cores
    ctx = mp.get_context("fork")
    pool = ctx.Pool(cores)
    try:
        pool.map(_numpy_encode_one, [(tiles[0], K)] * cores)       # imports, warm
        t0 = time.perf_counter()
        pool.map(_numpy_encode_one, [(tiles[i], K) for i in range(n)], chunksize=1)
        dt = time.perf_counter() - t0
    finally:
        # Let the workers exit and reap them, so none outlives the benchmark.
        pool.close()
        pool.join()
    return {"value": round(n / dt, 3), "unit": "tiles/s", "cores": cores, "kind": "port",
            "sample": f"first {n} tiles of the benchmark matrix at K={K} ({dt:.1f} s, numpy "
                      "restatement of reference_encoder.py, one process per core)"}


def cpu_baseline(tiles, K):
    """The C oracle (oracle/libexl3_oracle.so, a port of the reference's CPU
    encoder) on a bounded sample of the same workload, all host cores."""
    from oracle import c_oracle
    cores = c_oracle.default_threads()
    n = 16 * cores                                   # ~10 s of CPU work
    sample = tiles[:n]
    c_oracle.encode_tiles(sample[:1], K=K, cb=2, pre_permute=True, threads=1)  # load + warm
    t0 = time.perf_counter()
    c_oracle.encode_tiles(sample, K=K, cb=2, pre_permute=True, threads=cores)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tiles/s", "cores": cores, "kind": "port",
            "sample": f"first {n} tiles of the benchmark matrix at K={K} "
                      f"({dt:.1f} s, C restatement of reference_encoder.py, OpenMP)"}


def _synthetic_activations(rng, tokens, width, outlier_frac=0.05):
    """N(0, 1) activations with a seeded fraction of channels scaled x10."""
    X = rng.standard_normal((tokens, width), dtype=np.float32)
    chans = rng.choice(width, size=int(round(outlier_frac * width)), replace=False)
    X[:, chans] *= 10.0
    return X


def run_layer_config(torch, K=4, gss=False):
    """one 4096x4096 linear layer, W ~ N(0, 0.02^2) (seed 3),
    Hessian X^T X / 8192 from bf16 activations [8192, 4096] (seed 4, 5 % of
    channels x10), damped 1 %, Hadamard-rotated inside the driver, LDLQ with
    buf_size_k = 128 at K = 4 (256 encoder calls of 256 tiles). The reported
    wall time is the median of three runs after a 256x256 warm-up layer."""
    from exl3_intel_arc_quantizer_amd.layer_quant import (hessian_from_activations,
                                                          quantize_linear_module)
    W = torch.from_numpy((np.random.default_rng(3).standard_normal((4096, 4096),
                                                                   dtype=np.float32) * 0.02))
    X = torch.from_numpy(_synthetic_activations(np.random.default_rng(4), 8192, 4096))
    X = X.to(torch.bfloat16).cuda()
    H, damp = hessian_from_activations(X)
    del X
    quantize_linear_module("warmup", W[:256, :256].cuda(), H[:256, :256].contiguous(), K=K,
                           skip_g_scale=not gss)
    torch.cuda.synchronize()
    # A 0.2 s run is sensitive to clock ramp and host jitter: time three
    # full-size runs and report the median one.
    runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        res = quantize_linear_module("layer", W.cuda(), H, K=K, skip_g_scale=not gss)
        torch.cuda.synchronize()
        runs.append((time.perf_counter() - t0, res))
    runs.sort(key=lambda r: r[0])
    wall, res = runs[1]
    m = res.metrics
    tiles = 4096 * 4096 // 256
    return {"metric": "LDLQ-driven 4096x4096 layer, K=4, 1 MI355X: wall time", "value": round(wall, 3),
            "unit": "s", "higher_is_better": False, "n_gpus": 1, "dtype": "fp16", "data": "synthetic",
            "config": {"workload": "configs[3]", "K": K, "buf_size_k": 128, "tiles": tiles,
                       "encoder_calls": m.encoder_calls, "global_scale_search": gss},
            "g_scale": m.g_scale,
            "tiles_per_s": round(tiles / wall, 1),
            "runs_seconds": [round(r[0], 3) for r in runs],
            "encoder_seconds": round(m.encoder_seconds, 3),
            "encoder_share": round(m.encoder_seconds / wall, 4),
            "proxy_loss": m.proxy_loss, "normalized_proxy_loss": m.normalized_proxy_loss,
            "mse": m.mse, "factorization_residual": m.factorization_residual,
            "damping": damp,
            "cpu_path_parity": "proxy within 1e-3 of the CPU path on 256x256 layers "
                               "(tests/test_gpu_layer.py); measured once at full size "
                               "with a shared float64-built H: 5.1e-4 relative"}


def run_decoder_config(torch, K=4, cpu_tiles_per_s=None, lockstep=True, gss=False):
    """a 9B-class decoder layer (hidden 4096; q, o 4096x4096;
    k, v 1024x4096; gate, up 12288x4096; down 4096x12288), random-init weights
    (torch seed 5), Hessians per shared-input group from synthetic bf16
    activations [16384, width] (seeds 6..9, 5 % of channels x10), K = 4:
    753,664 tiles in 2,304 encoder calls."""
    from exl3_intel_arc_quantizer_amd.layer_quant import (hessian_from_activations,
                                                          hessian_groups,
                                                          quantize_decoder_layer)
    nn = torch.nn
    torch.manual_seed(5)
    layer = nn.Module()
    layer.self_attn = nn.Module()
    layer.mlp = nn.Module()
    for name, (o, i) in {"q_proj": (4096, 4096), "k_proj": (1024, 4096), "v_proj": (1024, 4096),
                         "o_proj": (4096, 4096)}.items():
        setattr(layer.self_attn, name, nn.Linear(i, o, bias=False))
    for name, (o, i) in {"gate_proj": (12288, 4096), "up_proj": (12288, 4096),
                         "down_proj": (4096, 12288)}.items():
        setattr(layer.mlp, name, nn.Linear(i, o, bias=False))
    layer = layer.cuda()
    names = [n for n, m in layer.named_modules() if isinstance(m, nn.Linear)]
    hess = {}
    t_hess = 0.0
    for seed, (key, members) in enumerate(hessian_groups(names).items(), start=6):
        width = 12288 if key == "mlp.down_proj" else 4096
        X = torch.from_numpy(_synthetic_activations(np.random.default_rng(seed), 16384, width))
        X = X.to(torch.bfloat16).cuda()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        H, _ = hessian_from_activations(X)
        torch.cuda.synchronize()
        t_hess += time.perf_counter() - t0
        for mname in members:
            hess[mname] = H
    # A model conversion runs this once per layer; the first layer of a
    # process also pays rocSOLVER / hipBLASLt kernel loading, so the timed
    # run is the second conversion of the same shapes (the steady state).
    first = quantize_decoder_layer(layer, hess, K=K, lockstep=lockstep, skip_g_scale=not gss)
    first_wall = first.total_elapsed_seconds
    del first
    rep = quantize_decoder_layer(layer, hess, K=K, lockstep=lockstep, skip_g_scale=not gss)
    wall = rep.total_elapsed_seconds
    calls = sum(r.metrics.encoder_calls for r in rep.module_results.values())
    out = {"metric": "9B-class decoder layer conversion, K=4, 1 MI355X: wall time",
           "value": round(wall, 3), "unit": "s", "higher_is_better": False, "n_gpus": 1,
           "dtype": "fp16", "data": "synthetic",
           "config": {"workload": "configs[4]", "K": K, "tiles": rep.tiles,
                      "module_encoder_calls": calls, "lockstep": lockstep,
                      "global_scale_search": gss},
           "tiles_per_s": round(rep.tiles / wall, 1),
           "encoder_seconds": round(rep.encoder_seconds, 3),
           "encoder_share": round(rep.encoder_seconds / wall, 4),
           "hessian_seconds": round(t_hess, 3),
           "first_layer_seconds": round(first_wall, 3),
           "phases": {k: round(v, 3) for k, v in rep.extra.items() if k.endswith("_seconds")},
           "total_proxy_loss": rep.total_proxy_loss, "mean_mse": rep.mean_mse,
           "peak_device_memory_bytes": rep.peak_device_memory_bytes,
           "modules": {n: {"shape_kn": list(r.original_shape),
                           "seconds": round(r.metrics.elapsed_seconds, 3),
                           "encoder_seconds": round(r.metrics.encoder_seconds, 3),
                           "normalized_proxy_loss": r.metrics.normalized_proxy_loss,
                           "g_scale": r.metrics.g_scale}
                       for n, r in rep.module_results.items()}}
    if cpu_tiles_per_s:
        out["cpu_encoder_extrapolated_seconds"] = round(rep.tiles / cpu_tiles_per_s, 1)
    return out


def run_host_api(torch, tiles, K=4, steps=5):
    """configs[1] through the reference's host-array API
    (XPUTrellisEncoder.encode_batch_detailed, xpu_quantizer.py:707-909):
    numpy tiles in, numpy states / packed words / path costs / distortions
    out, so PCIe transfers and host result assembly are inside the timing
    (per-tile EncodingResult objects skipped: build_results=False)."""
    from exl3_intel_arc_quantizer_amd.gpu_quantizer import XPUTrellisEncoder
    enc = XPUTrellisEncoder(K=K, cb=2)
    try:
        enc.encode_batch_detailed(tiles, pre_permute=True, build_results=False)
        t0 = time.perf_counter()
        for _ in range(steps):
            bd = enc.encode_batch_detailed(tiles, pre_permute=True, build_results=False)
        dt = (time.perf_counter() - t0) / steps
    finally:
        enc.arena.release()
    return {"metric": "configs[1] tiles/s through the host-array API (PCIe and host assembly "
                      "included), K=4, 1 MI355X",
            "value": round(tiles.shape[0] / dt, 1), "unit": "tiles/s", "higher_is_better": True,
            "n_gpus": 1, "steps": steps, "ms_per_step": round(dt * 1e3, 3), "dtype": "fp16",
            "data": "synthetic", "config": {"workload": "configs[1]", "K": K,
                                            "tiles": int(tiles.shape[0])},
            "breakdown_ms": {k: round(v * 1e3, 3) for k, v in (
                ("transfer", bd.transfer_seconds), ("search", bd.search_seconds),
                ("traceback", bd.traceback_seconds), ("post_process", bd.postprocess_seconds),
                ("total", bd.total_seconds))}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--sweep", action="store_true", help="also run K=2..6 on configs[2]")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--k-list", default="4,2",
                    help="bitrates to time on configs[1]; the first is the headline value")
    ap.add_argument("--profile-forward", action="store_true",
                    help="only the forward launches the roofline is measured on (one warm-up "
                         "and three timed per K), for rocprofv3 runs")
    ap.add_argument("--layer", action="store_true",
                    help="configs[3]: LDLQ-driven 4096x4096 layer (prints its own JSON line)")
    ap.add_argument("--decoder", action="store_true",
                    help="configs[4]: 9B-class decoder layer conversion (its own JSON line)")
    ap.add_argument("--host-api", action="store_true",
                    help="configs[1] through encode_batch_detailed (numpy in/out; PCIe-inclusive)")
    ap.add_argument("--gss", action="store_true",
                    help="with --layer / --decoder: run the global-scale search (skip_g_scale=False)")
    ap.add_argument("--sequential", action="store_true",
                    help="with --decoder: one projection at a time (the reference's order)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 1 GiB device copy (known-size kernel for PMC byte "
                         "counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the encoder "
              "would shard by tiles (each GPU a contiguous slice of the batch, outputs gathered "
              "once)", file=sys.stderr)
        return 2

    tiles = config2_tiles()
    k_list = [int(k) for k in args.k_list.split(",")]
    head = k_list[0]
    cpu = cpu_np = None
    if args.host_api:
        import torch
        print(json.dumps(run_host_api(torch, tiles)), flush=True)
        return 0
    if args.layer or args.decoder:
        import torch
        if args.decoder and not args.no_cpu_baseline:
            cpu = cpu_baseline(tiles, 4)
        line = (run_layer_config(torch, gss=args.gss) if args.layer else
                run_decoder_config(torch, cpu_tiles_per_s=cpu["value"] if cpu else None,
                                   lockstep=not args.sequential, gss=args.gss))
        print(json.dumps(line), flush=True)
        return 0
    if not args.no_cpu_baseline and not args.profile_forward:
        # Host baselines first: nothing has touched the GPU yet.
        cpu = cpu_baseline(tiles, head)
        cpu_np = cpu_baseline_numpy(tiles, head, cpu["cores"])
        print(f"# CPU baselines at K={head}: C {cpu['value']} tiles/s, numpy {cpu_np['value']} "
              f"tiles/s on {cpu['cores']} cores", file=sys.stderr, flush=True)

    import torch

    from exl3_intel_arc_quantizer_amd.gpu_quantizer import build_quantize_extension
    ext = build_quantize_extension()

    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("# calibration copy: 3 x 1 GiB read + 1 GiB written", file=sys.stderr, flush=True)
        del src, dst
        torch.cuda.empty_cache()

    if args.profile_forward:
        for K in k_list:
            b = DeviceBatch(tiles, K, torch, ext)
            for _ in range(8):                   # clocks up, as after the timed steps
                b.forward_only(b.n)
            rf = forward_kernel_roofline(b, torch)
            print(f"# K={K}: forward {rf['launch_ms']} ms over {b.n} tiles = "
                  f"{100 * rf['frac']:.1f}% of VALU peak", file=sys.stderr, flush=True)
            del b
            torch.cuda.empty_cache()
        return 0
    results = {}
    for K in k_list:
        b = DeviceBatch(tiles, K, torch, ext)
        sec = time_steps(b, args.steps, args.warmup, torch)
        results[K] = {"tiles_per_s": b.n / sec, "ms_per_step": sec * 1e3,
                      "roofline": forward_kernel_roofline(b, torch)}
        print(f"# K={K}: {b.n / sec:,.0f} tiles/s, {sec * 1e3:.2f} ms/step, forward "
              f"{results[K]['roofline']['launch_ms']} ms = "
              f"{100 * results[K]['roofline']['frac']:.1f}% of VALU peak", file=sys.stderr,
              flush=True)
        del b
        torch.cuda.empty_cache()

    sweep = None
    if args.sweep:
        sweep = {}
        big = config3_tiles()
        for K in (2, 3, 4, 5, 6):
            b = DeviceBatch(big, K, torch, ext, batch_cap=8192)
            sec = time_steps(b, max(1, args.steps // 5), 1, torch)
            rf = forward_kernel_roofline(b, torch, reps=1)
            sweep[K] = {"tiles_per_s": round(big.shape[0] / sec, 1),
                        "valu_frac": rf["frac"], "forward_ms_8192_tiles": rf["launch_ms"]}
            print(f"# sweep K={K}: {big.shape[0] / sec:,.0f} tiles/s, VALU {100 * rf['frac']:.1f}%",
                  file=sys.stderr, flush=True)
            del b
            torch.cuda.empty_cache()

    main_k = results[head]
    line = {
        "metric": METRIC,
        "value": round(main_k["tiles_per_s"], 1),
        "unit": "tiles/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_k["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "configs[1]: 1024x1024 N(0,1) fp16 matrix (seed 1), 4096 tiles "
                               f"in LDLQ order, K={head}, MUL1, L=256",
                   "tiles": 4096, "K": head, "codebook": "mul1"},
        "roofline": main_k["roofline"],
        "cpu_baseline": cpu,
        "cpu_baseline_numpy": cpu_np,
    }
    for K in k_list[1:]:
        line[f"k{K}"] = {"value": round(results[K]["tiles_per_s"], 1), "unit": "tiles/s",
                         "ms_per_step": round(results[K]["ms_per_step"], 3),
                         "roofline": results[K]["roofline"]}
    if sweep is not None:
        line["sweep_configs2"] = sweep
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
