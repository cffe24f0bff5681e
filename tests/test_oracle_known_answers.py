"""Closed-form, known-answer and invariant checks that pin the oracle without
the reference: fp16 rounding, codebook formula, permutation, packing, one
add-compare-select step by brute force, and the encoder invariants of the
reference's own tests. One test plants a mistake in a copy of the oracle's
arithmetic and checks that the known answers catch it.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import c_oracle
from oracle.reference_encoder import ReferenceTrellisEncoder
from oracle.trellis_format_ref import (
    CB_MUL1, MUL1_MULT, codebook_lut, decode_states, pack_trellis, state_index,
    stream_from_words, swap16_storage, tensor_core_perm, tensor_core_perm_inv,
    words_from_storage)

# exl3_quant/xpu_probe.py:221-224: inputs where an fp32 evaluation of
# dh*dh + cost followed by a rounding to fp16 differs from one rounding.
ADV_DH = [0x3C16, 0x3C27, 0x3C32, 0x3C5D, 0x3C71, 0x3C9B, 0x3CC9, 0x3CCE, 0x3CD3, 0x3CE1, 0x3CEA]
ADV_COST = [0x01C1, 0x00EF, 0x03C1, 0x0371, 0x01F1, 0x026F, 0x02EF, 0x03BF, 0x016F, 0x03EF, 0x01BF]


def _exact_half(q: Fraction) -> int:
    """Round a rational to fp16 (nearest, ties to even) from first principles."""
    sign = 0x8000 if q < 0 else 0
    q = abs(q)
    if q == 0:
        return sign
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -14)                                # subnormal range shares 2^-14's scale
    ulp = Fraction(2) ** (e - 10)
    m = q / ulp
    f = m.numerator // m.denominator
    rem = m - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2):
        f += 1
    if f >= 2048:
        f //= 2
        e += 1
    if e > 15:
        return sign | 0x7C00
    if f < 1024:                                   # subnormal
        return sign | f
    return sign | ((e + 15) << 10) | (f - 1024)


def _fr(bits: int) -> Fraction:
    v = np.uint16(bits).view(np.float16)
    return Fraction(float(v))


def test_exact_half_rounding_matches_numpy_on_representables():
    for bits in range(0, 0x7C00, 7):
        assert _exact_half(_fr(bits)) == bits


def test_adversarial_fma_pairs_single_rounding():
    a = np.array(ADV_DH, dtype=np.uint16).view(np.float16)
    c = np.array(ADV_COST, dtype=np.uint16).view(np.float16)
    exact = [_exact_half(_fr(x) * _fr(x) + _fr(y)) for x, y in zip(ADV_DH, ADV_COST)]
    got = c_oracle.fma_f16(a, c).view(np.uint16).tolist()
    assert got == exact
    # numpy restatement's expression (reference_encoder.py:191)
    numpy_expr = (a.astype(np.float64) ** 2 + c.astype(np.float64)).astype(np.float16)
    assert numpy_expr.view(np.uint16).tolist() == exact
    # The pairs discriminate: fp32 evaluation rounds differently on every one.
    fp32 = (a.astype(np.float32) ** 2 + c.astype(np.float32)).astype(np.float16)
    assert np.count_nonzero(fp32.view(np.uint16) != np.array(exact, dtype=np.uint16)) == 11


def test_random_fma_pairs_against_rationals():
    rng = np.random.default_rng(2026)                 # xpu_probe.py:153-183
    dh = rng.normal(0.0, 1.0, size=4096).astype(np.float16)
    cost = (rng.random(4096) * 8.0).astype(np.float16)
    got = c_oracle.fma_f16(dh, cost).view(np.uint16)
    for i in range(0, 4096, 3):
        x, y = int(dh.view(np.uint16)[i]), int(cost.view(np.uint16)[i])
        assert got[i] == _exact_half(_fr(x) * _fr(x) + _fr(y))


def test_planted_double_rounding_is_caught():
    """A copy of the oracle's FMA with the classic mistake (fp32 evaluation,
    then fp16) must fail the known answers."""
    def planted_fma(a, c):
        return (a.astype(np.float32) ** 2 + c.astype(np.float32)).astype(np.float16)
    a = np.array(ADV_DH, dtype=np.uint16).view(np.float16)
    c = np.array(ADV_COST, dtype=np.uint16).view(np.float16)
    assert not np.array_equal(planted_fma(a, c), c_oracle.fma_f16(a, c))


def test_double_to_half_direct_rounding_edge_cases():
    cases = [0.0, -0.0, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -25, 2.0 ** -24,
             65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -14 - 2.0 ** -25, 1.0 + 2.0 ** -11,
             1.0 + 3 * 2.0 ** -11, float("inf"), -float("inf")]
    lib = c_oracle.lib()
    for x in cases:
        assert lib.exl3o_half_from_double(x) == np.float64(x).astype(np.float16).view(np.uint16)
    rng = np.random.default_rng(9)
    xs = np.concatenate([rng.normal(0, 1, 2000), rng.normal(0, 1e-5, 2000),
                         rng.normal(0, 3e4, 1000)])
    for x in xs:
        assert lib.exl3o_half_from_double(float(x)) == np.float64(x).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("state", [0, 1, 2, 12345, 65535])
def test_mul1_closed_form(state):
    """tests/test_trellis_format.py:33-48 of the reference."""
    x = (state * MUL1_MULT) & 0xFFFFFFFF
    bsum = sum((x >> s) & 0xFF for s in (0, 8, 16, 24))
    h = Fraction(1024 + bsum)
    inv, bias = _fr(0x1EEE), _fr(0xC931)
    want = _exact_half(h * inv + bias)
    assert codebook_lut(CB_MUL1).view(np.uint16)[state] == want
    assert c_oracle.codebook_lut(CB_MUL1).view(np.uint16)[state] == want


def test_mul1_level_count_and_extremes():
    """913 distinct levels in [-3.453125, 3.34765625] (algorithm_contract.md:137-147)."""
    lut = codebook_lut(CB_MUL1).astype(np.float64)
    assert np.unique(lut).size == 913
    assert lut.min() == -3.453125 and lut.max() == 3.34765625


def test_tensor_core_perm_known_entries():
    """tests/test_trellis_format.py:110-116 of the reference."""
    perm = tensor_core_perm()
    assert perm[0:8].tolist() == [0, 16, 128, 144, 8, 24, 136, 152]
    assert perm[32:40].tolist() == [1, 17, 129, 145, 9, 25, 137, 153]
    assert sorted(perm.tolist()) == list(range(256))
    np.testing.assert_array_equal(perm[tensor_core_perm_inv()], np.arange(256))


def test_swap16_known_answer():
    """tests/test_trellis_format.py:163-167."""
    s = np.array([0x1111, 0x2222, 0x3333, 0x4444], dtype=np.uint16)
    assert swap16_storage(s).tolist() == [0x2222, 0x1111, 0x4444, 0x3333]


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
def test_pack_decode_round_trip(K):
    """tests/test_trellis_format.py:122-145: decode then re-pack reproduces a
    random bit stream; both pack implementations agree."""
    rng = np.random.default_rng(4242 + K)
    bits = rng.integers(0, 2, size=256 * K)
    nwords = 256 * K // 32
    words = (bits.reshape(nwords, 32) << np.arange(31, -1, -1)).sum(1)
    t16 = np.zeros(256 * K // 16, dtype=np.uint16)
    t16[0::2] = words & 0xFFFF
    t16[1::2] = words >> 16
    states = decode_states(t16, K)
    repacked = swap16_storage(pack_trellis(states, K))
    np.testing.assert_array_equal(stream_from_words(words_from_storage(repacked)), bits)
    np.testing.assert_array_equal(c_oracle.pack_tiles(states[None, :], K)[0], repacked)


def test_state_window_ends_at_bit():
    idx = state_index(4)
    np.testing.assert_array_equal(idx[0], np.arange(4 - 16, 4) % 1024)
    np.testing.assert_array_equal(idx[1], np.arange(8 - 16, 8) % 1024)


def _round_half_scaled(S: int, scale_exp: int) -> int:
    """fp16 bits of the exact value S * 2^scale_exp (S a Python int),
    round to nearest even, by integer arithmetic only."""
    sign = 0x8000 if S < 0 else 0
    S = abs(S)
    if S == 0:
        return sign
    e = max(S.bit_length() - 1 + scale_exp, -14)
    drop = e - 10 - scale_exp                        # low bits below the fp16 ulp
    if drop > 0:
        f, rem = S >> drop, S & ((1 << drop) - 1)
        half = 1 << (drop - 1)
        if rem > half or (rem == half and f & 1):
            f += 1
    else:
        f = S << -drop
    if f >= 2048:
        f >>= 1
        e += 1
    if e > 15:
        return sign | 0x7C00
    return sign | (f if f < 1024 else ((e + 15) << 10) | (f - 1024))


def _half_units(bits: int) -> int:
    """Exact value of a finite fp16 as an integer multiple of 2^-24."""
    mag = bits & 0x7FFF
    exp, man = mag >> 10, mag & 0x3FF
    v = man if exp == 0 else (man | 0x400) << (exp - 1)
    return -v if bits & 0x8000 else v


def _brute_step(lut_bits, w_bits, prev_bits, K):
    """One ACS step in scatter form: every state sigma reaches edge
    sigma & (E-1) from predecessor edge sigma >> K through branch
    sigma >> (16-K); exact integer arithmetic throughout."""
    E = 65536 >> K
    best = [None] * E
    best_k = [0] * E
    wu = _half_units(w_bits)
    for sigma in range(65536):
        e, k, p = sigma & (E - 1), sigma >> (16 - K), sigma >> K
        dh = _round_half_scaled(_half_units(int(lut_bits[sigma])) - wu, -24)
        d = _half_units(dh)
        cost = 0 if prev_bits is None else _half_units(int(prev_bits[p]))
        err = _round_half_scaled(d * d + (cost << 24), -48)   # one rounding (fused)
        if best[e] is None or err < best[e]:                   # non-negative: bits order
            best[e], best_k[e] = err, k                       # sigma ascends in k per edge
    return np.array(best, dtype=np.uint16), np.array(best_k, dtype=np.int64)


@pytest.mark.parametrize("K", [2, 4])
def test_two_acs_steps_by_brute_force(K):
    """The oracle's forward pass (numpy and C) on a 2-element ring against an
    independent scatter-form brute force over all 65536 states."""
    rng = np.random.default_rng(K)
    E = 65536 >> K
    lut_bits = codebook_lut(CB_MUL1).view(np.uint16)
    tile = rng.normal(0, 1, size=2).astype(np.float16)
    w = tile.view(np.uint16)
    c0, k0 = _brute_step(lut_bits, int(w[0]), None, K)
    c1, k1 = _brute_step(lut_bits, int(w[1]), c0, K)
    e = np.arange(E)
    enc = ReferenceTrellisEncoder(K=K, cb=CB_MUL1, tile_len=2)
    edges = np.zeros((2, E), dtype=np.uint16)
    costs = enc.forward(tile, roll=0, pre_state=-1, temp_edges=edges)
    np.testing.assert_array_equal(costs.view(np.uint16), c1)
    np.testing.assert_array_equal(edges[0], (k0 << (16 - 2 * K)) | (e >> K))
    np.testing.assert_array_equal(edges[1], (k1 << (16 - 2 * K)) | (e >> K))
    c_edges, c_costs = c_oracle.forward_pass(tile, K=K, cb=CB_MUL1, roll=0, pre_state=-1)
    np.testing.assert_array_equal(c_costs.view(np.uint16), c1)
    np.testing.assert_array_equal(c_edges, edges)


def test_encoder_invariants_and_mse_ceilings():
    """Ring continuity, tail-biting, recon == lut[idx] and the upstream MSE
    ceilings (tests/test_encoder.py:57-100, tests/test_upstream_encode_oracle.py:56-110)."""
    ceilings = {1: 0.3, 2: 0.1, 3: 0.1, 4: 0.1, 5: 0.1, 6: 0.07, 7: 0.05, 8: 0.04}
    rng = np.random.default_rng(0)
    tiles = rng.standard_normal((4, 256)).astype(np.float32)
    for K in (1, 2, 3, 4, 5, 6, 7, 8):
        ob = c_oracle.encode_tiles(tiles, K=K, cb=CB_MUL1, pre_permute=False)
        idx = ob.output_indices.astype(np.int64)
        mask = (65536 >> K) - 1
        np.testing.assert_array_equal(idx & mask, np.roll(idx, -1, axis=1) >> K)
        np.testing.assert_array_equal(idx[:, 0] >> K, idx[:, 255] & mask)
        np.testing.assert_array_equal(ob.end_state, idx[:, 255] & mask)
        lut = codebook_lut(CB_MUL1)
        np.testing.assert_array_equal(ob.reconstructed_perm.view(np.uint16), lut[idx].view(np.uint16))
        mse = float(np.mean((tiles - ob.reconstructed.astype(np.float32)) ** 2))
        assert mse < ceilings[K]
        for t in range(4):
            np.testing.assert_array_equal(decode_states(ob.packed[t], K), idx[t])


def test_ties_keep_lowest_branch():
    """tests/test_forward_semantics.py:143-163: a constant tile on a constant
    codebook ties every branch; the lowest k must win."""
    enc = ReferenceTrellisEncoder(K=3)
    enc.k_vals = np.zeros((enc.max_q, enc.edges), dtype=np.float16)
    enc.k_preds = np.zeros((enc.max_q, enc.edges), dtype=np.uint16)
    for k in range(enc.max_q):
        enc.k_preds[k] = (k * 7 + 1) % enc.edges
    edges = np.zeros((enc.L, enc.edges), dtype=np.uint16)
    enc.forward(np.full(enc.L, np.float16(0.25)), roll=0, pre_state=-1, temp_edges=edges)
    np.testing.assert_array_equal(edges, np.tile(enc.k_preds[0], (enc.L, 1)))
