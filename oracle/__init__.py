"""CPU oracle for the quantized matvec / matmul path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and a C twin under ``oracle/c``), the
reference's weight formats and the arithmetic its kernels perform, so that the
HIP library can be checked against it.  Only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker: nothing in ``qwowl35_amd`` imports, links or executes anything here.

Modules and what pins each one (the pins live in ``tests/test_oracle_*.py``):

* ``gf4``   — e5m2 scale codec and the GF4 packer/decoder
  (reference ``tools/qw35_cook_common.py:48-56,67-80,83-119``).
  Pinned by: the exhaustive 256-entry e5m2 table against the IEEE binary16
  closed form, all 65 536 fp16 patterns through the encoder against a
  round-half-up closed form, the exhaustive (scale byte x code x position)
  decode table against ``-sext3(code) * s / 4``, hand-computed known-answer
  words, repack idempotence and the quantisation error bound.
* ``q8_0``  — ggml q8_0 blocks (reference ``qw35_types.metal:24-36``,
  ``qw35_matvec.metal:136-149,630-683``).  Pinned by the closed form
  ``fp16(d) * int8`` on hand-built blocks and exhaustive int8 sweeps.
* ``q4_k``  — ggml Q4_K super-blocks (reference ``qw35_types.metal:2-7,70-83``,
  ``qw35_matvec.metal:2-38``).  Pinned by two independent restatements (the
  reference's scalar and tile forms) agreeing bit-for-bit on random blocks,
  hand-built blocks with a single non-zero sub-scale / min, and an exhaustive
  sweep of the 6-bit scale packing.
* ``matvec`` — fp64 matvec / matmul on oracle-dequantised weights, bf16/fp16
  rounding helpers, the prefill oracle.  Pinned by brute-force Python loops on
  tiny shapes and by exact-integer cases.

Parity unpinned (no reference test or golden vector covers them, and the
third-party decoder they come from, gguf-py, is not vendored or installed):
the byte-level agreement of ``q8_0``/``q4_k`` decoding with
``gguf.quants.{Q8_0,Q4_K}.dequantize_blocks`` beyond the in-repo Metal
statements cited above.
"""
