"""Closed-form cases for regularize (regularize.py:83-211 of the reference),
shared by the oracle's CPU test and the GPU test of the product. Each case
gives a weight W (k, n), the Hessian diagonal and the scale values that the
definition fixes, computed here from the definition in float64:

* ``columns``: column c of W is a_c times random signs, a_c cycling through
  0.5, 1, 2, 4. The column RMS is a_c exactly and their mean 1.875 exactly,
  so sv = a_c / 1.875 (+1e-10, below float32 resolution at these values).
  After W / sv every entry has magnitude 1.875; the right transform is
  orthonormal per 128-column block, so every row RMS is 1.875 and
  su = -1.875 / 1.24371088. A flipped sign or a wrong codebook constant in
  su, or a mean over the wrong count in the RMS, fails.
* ``tiny``: all entries +-1e-12. su = 1e-10 - 1e-12 / 1.24371088, which is
  positive: the 1e-10 is added after the division. Adding it anywhere else
  gives a negative su.
* ``dead``: column 5 and row 17 of a Gaussian W are zero. The dead column
  is divided by 0.1 (+1e-10) and stored as sv = 0; the dead row's RMS is
  replaced by 0.1, so su[17] = 0.1 / -1.24371088 + 1e-10.
* ``skew_below`` / ``skew_above``: a Hessian diagonal whose top 5 of 256
  entries (the top 2 %, 256 // 50) have sqrt 8.8 / 8.92 and the rest 1:
  skew = 5 L / (5 L + 251) = 0.14915 / 0.15088, either side of the 0.15
  cutoff, so the output scales apply / do not (sv stays the caller's ones).
"""

from __future__ import annotations

import numpy as np

K, N = 256, 384
CB = 1.24371088
EPS = 1e-10


def _signs(rng, shape):
    return np.where(rng.random(shape) < 0.5, -1.0, 1.0).astype(np.float32)


def cases():
    """name -> dict(W, H_diag, expected: dict of float64 arrays / bools)."""
    rng = np.random.default_rng(77)
    out = {}
    a = np.tile(np.array([0.5, 1.0, 2.0, 4.0], np.float32), N // 4)
    W = _signs(rng, (K, N)) * a[None, :]
    ones = np.ones(K, np.float32)
    out["columns"] = dict(W=W, H_diag=ones, expected=dict(
        apply_out=True, sv=(a.astype(np.float64) / 1.875).reshape(1, N),
        su=np.full((K, 1), -1.875 / CB)))

    W = (_signs(rng, (K, N)) * np.float32(1e-12)).astype(np.float32)
    out["tiny"] = dict(W=W, H_diag=ones, expected=dict(
        apply_out=True, su=np.full((K, 1), EPS - 1e-12 / CB)))

    W = rng.standard_normal((K, N)).astype(np.float32)
    W[:, 5] = 0.0
    W[17, :] = 0.0
    out["dead"] = dict(W=W, H_diag=ones, expected=dict(
        apply_out=True, dead_col=5, dead_row=17, su_dead=0.1 / -CB + EPS))

    for name, L in (("skew_below", 8.8), ("skew_above", 8.92)):
        diag = np.ones(K, np.float32)
        diag[[3, 50, 99, 140, 201]] = np.float32(L * L)
        W = rng.standard_normal((K, N)).astype(np.float32)
        W[:, 11] *= 20.0
        out[name] = dict(W=W, H_diag=diag, expected=dict(
            apply_out=name == "skew_below", skew=5 * L / (5 * L + 251)))
    return out


def check(name, case, weight, su, sv, apply_out, W_back):
    """Assert the closed-form values of ``case`` on one implementation's
    outputs (numpy arrays: transformed weight, su (K, 1), sv (1, N), the
    apply flag, and the weight rebuilt by weight_from_quantized)."""
    exp = case["expected"]
    W = case["W"]
    assert bool(apply_out) == exp["apply_out"], name
    assert np.isfinite(weight).all(), name
    su = np.asarray(su, np.float64).reshape(K, 1)
    sv = np.asarray(sv, np.float64).reshape(1, N)
    if "sv" in exp:
        np.testing.assert_allclose(sv, exp["sv"], rtol=1e-7, err_msg=name)
    if "su" in exp:
        np.testing.assert_allclose(su, exp["su"], rtol=2e-6, err_msg=name)
        assert np.all(np.sign(su) == np.sign(exp["su"])), name
    if name == "dead":
        assert sv[0, exp["dead_col"]] == 0.0
        np.testing.assert_allclose(su[exp["dead_row"], 0], exp["su_dead"], rtol=1e-6)
        assert np.all(sv[0, np.arange(N) != exp["dead_col"]] > 0)
    if name == "skew_above":
        np.testing.assert_array_equal(sv, np.ones((1, N)))
    if name == "skew_below":
        assert sv[0, 11] > 5.0 * np.median(sv)
    # Decoding (H_l, x su, H_r, x sv) returns the weight.
    scale = np.abs(W).max()
    np.testing.assert_allclose(W_back, W, rtol=0, atol=2e-5 * scale, err_msg=name)
