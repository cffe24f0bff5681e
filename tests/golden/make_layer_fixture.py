"""Write tests/golden/layer_configs3.npz: configs[3] through the CPU pipeline.

The CPU pipeline is oracle/ldlq_ref.quantize_linear_module (numpy float32
restatement of layer_quant.py:130-265: regularize, Hadamard, block LDL, LDLQ
with buf_size_k = 128, the proxy of layer_quant.py:104-127) with the C
oracle encoder (oracle/libexl3_oracle.so) as the tile encoder, K = 4, on the
inputs of tests/layer_configs.py. It runs in this container only, once: the
4096 x 4096 layer is 65,536 tiles at about 6 tiles/s per core (3 h on 8
cores). The GPU test (tests/test_gpu_layer_full.py) repeats the layer on the
GPU and compares against what is stored here:

* proxy and normalised proxy of the CPU pipeline;
* SHA-256 of H (float32 bytes), to report whether the GPU built the same H;
* SHA-256 of all states (uint16 (256, 256, 256), block row, tile, position)
  and one per block row;
* states of tiles 0 and 128 of every block row (256 x 2 x 256 uint16);
* rows 0, 1024, 2048, 3072 of the reconstructed weight w_hat (k, n).

    python tests/golden/make_layer_fixture.py [--threads N] [--full-out PATH]
"""

from __future__ import annotations

import argparse
import hashlib
import os
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

SAMPLE_TILES = (0, 128)
W_HAT_ROWS = (0, 1024, 2048, 3072)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=0, help="C oracle threads (0: all CPUs)")
    ap.add_argument("--full-out", default=None,
                    help="also save every state and w_hat to this .npz (not committed)")
    args = ap.parse_args()
    if args.threads:
        os.environ["EXL3_ORACLE_THREADS"] = str(args.threads)

    from oracle import c_oracle, ldlq_ref
    from tests.layer_configs import C3_K, configs3_hessian_cpu, configs3_weight

    c_oracle.build()
    t0 = time.time()
    W = configs3_weight()
    H, damp = configs3_hessian_cpu()
    print(f"H ready in {time.time() - t0:.1f} s, damping {damp!r}", flush=True)

    inner = ldlq_ref.c_oracle_encoder(C3_K)
    calls = [0]

    def counting(tiles):
        calls[0] += 1
        if calls[0] % 8 == 0:
            print(f"encoder call {calls[0]} / 256 at {time.time() - t0:.0f} s", flush=True)
        return inner(tiles)

    original = ldlq_ref.c_oracle_encoder
    ldlq_ref.c_oracle_encoder = lambda K: counting
    try:
        w_hat, encoded, proxy, norm = ldlq_ref.quantize_linear_module(
            np.ascontiguousarray(W.T), H, C3_K)
    finally:
        ldlq_ref.c_oracle_encoder = original
    encoded = np.ascontiguousarray(np.asarray(encoded, dtype=np.uint16))
    assert encoded.shape == (256, 256, 256), encoded.shape
    block_sha = np.stack([np.frombuffer(hashlib.sha256(encoded[b].tobytes()).digest(), np.uint8)
                          for b in range(encoded.shape[0])])
    out = HERE / "layer_configs3.npz"
    np.savez(out,
             proxy=np.float64(proxy), normalized_proxy=np.float64(norm),
             damping=np.float64(damp),
             h_sha256=np.array(hashlib.sha256(H.tobytes()).hexdigest()),
             states_sha256=np.array(hashlib.sha256(encoded.tobytes()).hexdigest()),
             block_sha256=block_sha,
             sample_tiles=np.array(SAMPLE_TILES, dtype=np.int32),
             states_sample=encoded[:, list(SAMPLE_TILES), :],
             w_hat_row_index=np.array(W_HAT_ROWS, dtype=np.int32),
             w_hat_rows=np.ascontiguousarray(w_hat[list(W_HAT_ROWS)], dtype=np.float32))
    if args.full_out:
        np.savez(args.full_out, encoded=encoded, w_hat=w_hat.astype(np.float32))
    print(f"done in {time.time() - t0:.0f} s: proxy {proxy!r} normalised {norm!r} -> {out}",
          flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
