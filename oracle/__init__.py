"""CPU oracle for the EXL3 trellis tile encoder — TEST INFRASTRUCTURE ONLY.

Nothing in the product package imports this directory. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
use it, and only as the checker (or the timed CPU baseline), never as the
thing that produces encoder results.

Contents
--------
``trellis_format_ref``   numpy restatement of the reference's format
                         primitives (exl3_quant/trellis_format.py:41-227).
``reference_encoder``    numpy restatement of ``ReferenceTrellisEncoder``
                         (exl3_quant/reference_encoder.py:44-350), same class
                         and method names, op-for-op fp16 semantics.
``exl3_oracle.c``        C restatement of the same encoder (exact fp16 through
                         a direct double->half round-to-nearest-even), OpenMP
                         over tiles; built by ``oracle/Makefile`` into
                         ``oracle/libexl3_oracle.so`` and loaded by
                         ``oracle.c_oracle``.

How each part is pinned (a function with none of these would be marked
"parity unpinned"; none is):

* codebook: full-table SHA-256 of the reference's ``codebook_lut`` for all
  three codebooks (tests/golden/codebook_lut.json) plus the closed-form
  per-state checks and level counts of tests/test_trellis_format.py:33-93;
* fp16 arithmetic: the 11 adversarial (dh, cost) pairs of
  exl3_quant/xpu_probe.py:221-224, where a float32 double rounding differs
  from the single rounding, plus 65536 random pairs against an exact
  rational computation (fractions.Fraction);
* tensor-core permutation: closed form + the known entries of
  tests/test_trellis_format.py:110-116;
* packing: SWAP16 known answer, decode/pack round trip on random bit streams
  (tests/test_trellis_format.py:122-185);
* encoder: the golden vectors in tests/golden/*.npz, produced by the
  reference's own ``ReferenceTrellisEncoder`` (bit-exact indices, packed
  words, end states, path costs, reconstructions), plus the tail-biting,
  ring-continuity and MSE-ceiling invariants of the reference's tests and a
  brute-force Viterbi check on a reduced trellis.
"""
