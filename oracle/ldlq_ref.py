"""CPU oracle for the LDLQ layer driver — TEST INFRASTRUCTURE ONLY.

numpy float32 restatement of the reference's layer pipeline around the tile
encoder: blockwise Hadamard (exl3_quant/hadamard.py:34-140), regularize
(regularize.py:41-211), block_ldl (ldlq.py:76-142), ldlq (ldlq.py:163-309),
the proxy loss (layer_quant.py:95-127) and quantize_linear_module
(layer_quant.py:130-265) with the C oracle as tile encoder. Only tests/ and
bench.py's baseline may use it.

Pinned by tests/test_oracle_ldlq.py: the Hadamard closed form
((-1)^popcount(i & j) / sqrt(128)) and orthonormality; the regularize round
trip through weight_from_quantized; block_ldl's factor (L L^T = H) and fold
(transformed column block x diagonal block of L = L's column block,
identity diagonal); the LDLQ feedback identity (every block's encoder
input equals W_b + L[below, b]^T (W - W_q)[below], checked with a recording
encoder); the proxy against an explicit trace.
"""

from __future__ import annotations

import numpy as np

HAD_DIM = 128
CODEBOOK_SCALE = np.float32(1.24371088)
ZERO_FLOOR = np.float32(0.1)
EPS = np.float32(1e-10)


def hadamard(n: int = HAD_DIM) -> np.ndarray:
    """Orthonormal Sylvester matrix (hadamard.py:34-70), float32."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return (h / np.sqrt(n)).astype(np.float32)


def had_l(x: np.ndarray) -> np.ndarray:
    """H @ x per 128-row block (hadamard.py:73-83)."""
    k, n = x.shape
    h = hadamard()
    return np.einsum("ij,bjn->bin", h, x.reshape(k // HAD_DIM, HAD_DIM, n),
                     dtype=np.float32).reshape(k, n)


def had_r(x: np.ndarray) -> np.ndarray:
    """x @ H per 128-column block (hadamard.py:86-96)."""
    k, n = x.shape
    h = hadamard()
    return np.einsum("kbj,ji->kbi", x.reshape(k, n // HAD_DIM, HAD_DIM), h,
                     dtype=np.float32).reshape(k, n)


def block_rms(x: np.ndarray, axis: int) -> np.ndarray:
    """sqrt(mean of squares) over 32-slices in order (regularize.py:41-56), keepdims."""
    n = x.shape[axis]
    sq = None
    for s in range(0, n, 32):
        blk = np.take(x, np.arange(s, min(s + 32, n)), axis=axis)
        part = np.square(blk).sum(axis=axis, keepdims=True, dtype=np.float32)
        sq = part if sq is None else sq + part
    return np.sqrt(sq / np.float32(n)).astype(np.float32)


def regularize(W: np.ndarray, H_diag: np.ndarray):
    """regularize.py:74-211 with su = sv = 1, skip_g_scale: returns
    (weight, su (k,1), sv (1,n), apply_out_scales)."""
    k, n = W.shape
    d = np.sort(np.sqrt(H_diag.astype(np.float32)))[::-1]
    skew = float(d[: d.shape[0] // 50].sum() / d.sum())
    apply_out = skew < 0.15
    work = W.astype(np.float32).copy()
    out_scales = block_rms(work, axis=0)
    mean = float(out_scales.mean())
    if mean > 1e-30:
        out_scales = out_scales / np.float32(mean)
    zero_out = np.abs(out_scales) < 1e-30
    su = np.ones((k, 1), np.float32)
    sv = np.ones((1, n), np.float32)
    if apply_out:
        out_scales[zero_out] = ZERO_FLOOR
        sv = (sv * out_scales + EPS).astype(np.float32)
    work = work / sv
    sv[zero_out] = 0.0
    work = had_r(work)
    in_scales = block_rms(work, axis=1)
    in_scales[np.abs(in_scales) < 1e-30] = ZERO_FLOOR
    su = (su * in_scales / (-CODEBOOK_SCALE) + EPS).astype(np.float32)
    work = work / su
    work = had_l(work)
    return work.astype(np.float32), su, sv, apply_out


def weight_from_quantized(w_hat: np.ndarray, su: np.ndarray, sv: np.ndarray) -> np.ndarray:
    """H_l, x su, H_r, x sv (hadamard.py:129-140)."""
    return had_r(had_l(w_hat) * su) * sv


def block_ldl(H: np.ndarray, block_size: int = 16, sigma_reg: float = 0.025,
              max_retries: int = 10):
    """ldlq.py:76-142: returns (transformed, chol, retries)."""
    n = H.shape[0]
    work = H.astype(np.float32).copy()
    for attempt in range(max_retries + 1):
        try:
            chol = np.linalg.cholesky(work).astype(np.float32)
            break
        except np.linalg.LinAlgError:
            if attempt == max_retries:
                raise
            work[np.diag_indices(n)] += np.float32(2.0 * sigma_reg * np.diag(work).mean())
    transformed = chol.copy()
    for b in range(n // block_size):
        s = slice(b * block_size, (b + 1) * block_size)
        transformed[:, s] = chol[:, s] @ np.linalg.inv(chol[s, s]).astype(np.float32)
    for b in range(n // block_size):
        s = slice(b * block_size, (b + 1) * block_size)
        transformed[s, s] = np.eye(block_size, dtype=np.float32)
    return transformed, chol, attempt


def tc_perm() -> np.ndarray:
    from oracle.trellis_format_ref import tensor_core_perm
    return tensor_core_perm()


def ldlq(W: np.ndarray, L: np.ndarray, encode, buf: int = 128):
    """ldlq.py:163-309. ``encode`` maps (tiles_n, 256) float32 tensor-core
    order tiles to (reconstruction float32, uint16 states)."""
    k, n = W.shape
    tn = n // 16
    perm = tc_perm()
    inv = np.argsort(perm)
    prod = np.zeros((k, n), np.float32)
    Wq = np.zeros((k, n), np.float32)
    enc = np.zeros((k // 16, tn, 256), np.uint16)
    for j in range(k, 0, -buf):
        i = j - buf
        for bj in range(buf, 0, -16):
            r0, r1 = i + bj - 16, i + bj
            if r1 < j:
                prod[r0:r1] += L[r1:j, r0:r1].T @ (W[r1:j] - Wq[r1:j])
            rows = W[r0:r1] + prod[r0:r1]
            tiles = rows.reshape(16, tn, 16).transpose(1, 0, 2).reshape(tn, 256)[:, perm]
            qw, qi = encode(np.ascontiguousarray(tiles, dtype=np.float32))
            Wq[r0:r1] = qw[:, inv].reshape(tn, 16, 16).transpose(1, 0, 2).reshape(16, n)
            enc[r0 // 16] = qi
        prod += L[i:j].T @ (W[i:j] - Wq[i:j])
    return Wq, enc


def c_oracle_encoder(K: int):
    """Tile encoder backed by the C oracle (fp16 rounding as the reference's
    wrapper, xpu_quantizer.py:654-655, then encode_tile with pre_permute=False)."""
    from oracle import c_oracle

    def encode(tiles):
        t16 = tiles.astype(np.float16).astype(np.float32)
        b = c_oracle.encode_tiles(t16, K=K, cb=2, pre_permute=False)
        return b.reconstructed_perm.astype(np.float32), b.output_indices
    return encode


def proxy_loss(W: np.ndarray, W_hat: np.ndarray, H: np.ndarray):
    """sum((H E) * E) and its ratio to sum((H W) * W) (layer_quant.py:104-127)."""
    E = (W - W_hat).astype(np.float32)
    proxy = float(((H @ E) * E).sum(dtype=np.float64))
    energy = float(((H @ W) * W).sum(dtype=np.float64))
    return proxy, proxy / max(1e-12, energy)


def quantize_linear_module(weight_kn: np.ndarray, H: np.ndarray, K: int, buf: int = 128):
    """layer_quant.py:130-265 for a (k, n) weight: returns (w_hat, encoded, proxy, norm_proxy)."""
    W = weight_kn.astype(np.float32)
    reg_w, su, sv, _ = regularize(W, np.diag(H))
    Hw = had_r(had_l(H.astype(np.float32)))
    transformed, _, _ = block_ldl(Hw)
    Wq, enc = ldlq(reg_w, transformed, c_oracle_encoder(K), buf)
    w_hat = weight_from_quantized(Wq, su, sv)
    proxy, norm = proxy_loss(W, w_hat, H.astype(np.float32))
    return w_hat, enc, proxy, norm
