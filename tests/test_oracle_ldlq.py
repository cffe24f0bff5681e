"""CPU checks that pin the LDLQ layer oracle (oracle/ldlq_ref.py) by
closed forms and invariants, each chosen so that a dropped term, a wrong
sign, a transposed factor or a reordered transform fails."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ldlq_ref


def _spd(n, seed, outliers=True):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((4 * n, n)).astype(np.float32)
    if outliers:
        X[:, rng.random(n) < 0.05] *= 10.0
    H = (X.T @ X) / np.float32(X.shape[0])
    H[np.diag_indices(n)] += np.float32(0.01 * np.diag(H).mean())
    return H.astype(np.float32)


def test_hadamard_closed_form():
    """hadamard.py:34-70: Sylvester entries (-1)^popcount(i & j) / sqrt(128),
    orthonormal and symmetric; had_l is its own inverse."""
    h = ldlq_ref.hadamard()
    i, j = np.meshgrid(np.arange(128), np.arange(128), indexing="ij")
    pop = np.vectorize(lambda v: bin(v).count("1"))(i & j)
    np.testing.assert_allclose(h, ((-1.0) ** pop) / np.sqrt(128.0), rtol=0, atol=1e-7)
    np.testing.assert_allclose(h @ h.T, np.eye(128), atol=1e-5)
    x = np.random.default_rng(1).standard_normal((256, 128)).astype(np.float32)
    np.testing.assert_allclose(ldlq_ref.had_l(ldlq_ref.had_l(x)), x, atol=1e-5)
    np.testing.assert_allclose(ldlq_ref.had_r(x)[:, :128], x[:, :128] @ h, atol=1e-5)


def test_regularize_round_trip_and_scales():
    """regularize.py:74-211 undone by weight_from_quantized (hadamard.py:129-140):
    the order (/sv, H_r, /su, H_l) and every scale are pinned by the round trip."""
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    W[:, 7] *= 30.0                                      # a loud output channel
    H = _spd(256, 3)
    reg_w, su, sv, apply_out = ldlq_ref.regularize(W, np.diag(H))
    np.testing.assert_allclose(ldlq_ref.weight_from_quantized(reg_w, su, sv), W,
                               rtol=2e-3, atol=2e-6)
    # block_rms is the plain RMS up to float32 rounding.
    np.testing.assert_allclose(ldlq_ref.block_rms(W, axis=0)[0],
                               np.sqrt((W.astype(np.float64) ** 2).mean(axis=0)), rtol=1e-5)
    # Skew heuristic: a diagonal whose top 2% holds most of the mass turns
    # the output scales off.
    skewed = np.ones(256, np.float32)
    skewed[:5] = 1e6
    assert ldlq_ref.regularize(W, skewed)[3] is False
    assert apply_out is True


@pytest.mark.parametrize("name", ["columns", "tiny", "dead", "skew_below", "skew_above"])
def test_regularize_closed_forms(name):
    """regularize.py:83-211: scale values fixed by the definition (see
    tests/regularize_cases.py): su = RMS / -1.24371088 + 1e-10 with the sign,
    constant and 1e-10 placement pinned, sv = column RMS / mean RMS, zero
    rows and columns, the 0.15 skew cutoff over the top 2 % of the diagonal."""
    from .regularize_cases import cases, check
    case = cases()[name]
    reg_w, su, sv, apply_out = ldlq_ref.regularize(case["W"], case["H_diag"])
    back = ldlq_ref.weight_from_quantized(reg_w, su, sv)
    check(name, case, reg_w, su, sv, apply_out, back)


def test_block_ldl_factor_and_fold():
    """ldlq.py:76-142: L L^T = H; transformed = L with each column block
    times the inverse of its diagonal block, diagonal blocks identity."""
    H = _spd(64, 4)
    T, chol, retries = ldlq_ref.block_ldl(H)
    assert retries == 0
    np.testing.assert_allclose(chol @ chol.T, H, rtol=1e-4, atol=1e-4 * np.abs(H).max())
    for b in range(4):
        s = slice(16 * b, 16 * b + 16)
        np.testing.assert_array_equal(T[s, s], np.eye(16, dtype=np.float32))
        rows = np.r_[0:16 * b, 16 * b + 16:64]
        np.testing.assert_allclose(T[rows, s] @ chol[s, s], chol[rows, s], atol=1e-4)
    # Shifted just below positive definite (by 2 % of mean(diag)): the damping
    # retries (2 sigma mean(diag) each) recover it in one or two steps.
    lam = np.linalg.eigvalsh(H.astype(np.float64)).min()
    bad = (H - np.float32(lam + 0.02 * np.diag(H).mean()) * np.eye(64, dtype=np.float32))
    _, chol_bad, retries = ldlq_ref.block_ldl(bad.astype(np.float32))
    assert 1 <= retries <= 2


def test_ldlq_feedback_identity():
    """ldlq.py:163-309: block b's encoder input equals
    W_b + L[rows below b, b]^T (W - W_q)[rows below b] for the final W_q,
    whatever the encoder does (checked with a recording grid quantiser)."""
    rng = np.random.default_rng(5)
    k, n = 256, 128
    W = rng.standard_normal((k, n)).astype(np.float32)
    L, _, _ = ldlq_ref.block_ldl(_spd(k, 6))
    seen = []

    def grid(tiles):
        seen.append(tiles.copy())
        return np.round(tiles * 4.0) / np.float32(4.0), np.zeros(tiles.shape, np.uint16)

    Wq, _ = ldlq_ref.ldlq(W, L, grid, buf=128)
    inv = np.argsort(ldlq_ref.tc_perm())
    E = W - Wq
    order = [r0 for j in range(k, 0, -128) for r0 in range(j - 16, j - 128 - 1, -16)]
    assert len(order) == len(seen) == k // 16
    for r0, tiles in zip(order, seen):
        got = tiles[:, inv].reshape(n // 16, 16, 16).transpose(1, 0, 2).reshape(16, n)
        want = W[r0:r0 + 16] + L[r0 + 16:, r0:r0 + 16].T @ E[r0 + 16:]
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    # With H = I the factor is the identity: no feedback at all.
    Wq_eye, _ = ldlq_ref.ldlq(W, np.eye(k, dtype=np.float32), grid, buf=64)
    np.testing.assert_array_equal(Wq_eye, np.round(W * 4.0) / np.float32(4.0))


def test_proxy_is_the_hessian_trace():
    """layer_quant.py:104-127: sum((H E) * E) = tr(E^T H E)."""
    rng = np.random.default_rng(7)
    H = _spd(32, 8)
    W = rng.standard_normal((32, 16)).astype(np.float32)
    W_hat = W + 0.01 * rng.standard_normal((32, 16)).astype(np.float32)
    p, norm = ldlq_ref.proxy_loss(W, W_hat, H)
    E = (W - W_hat).astype(np.float64)
    assert p == pytest.approx(np.trace(E.T @ H.astype(np.float64) @ E), rel=1e-5)
    assert norm == pytest.approx(p / np.trace(W.T.astype(np.float64) @ H @ W), rel=1e-5)
