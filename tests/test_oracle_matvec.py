"""Pins of the fp64 matvec / prefill oracle (oracle/matvec.py) by brute force."""
from __future__ import annotations

import math

import numpy as np

from oracle import matvec as om


def test_matvec_brute_force_tiny():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((3, 5)).astype(np.float32)
    x = rng.standard_normal((2, 5)).astype(np.float32)
    a = rng.uniform(0.5, 2, 5).astype(np.float32)
    got = om.matvec_f64(w, x, a)
    for b in range(2):
        for r in range(3):
            want = math.fsum(float(w[r, k]) * float(a[k]) * float(x[b, k]) for k in range(5))
            assert abs(got[b, r] - want) <= 1e-12 * max(1.0, abs(want))


def test_matvec_exact_integers():
    w = np.arange(-6, 6, dtype=np.float32).reshape(3, 4)
    x = np.array([1, -2, 3, -4], dtype=np.float32)
    assert om.matvec_f64(w, x).tolist() == [(-6 * 1 + -5 * -2 + -4 * 3 + -3 * -4), (-2 + 2 + 0 - 4),
                                            (2 * 1 + 3 * -2 + 4 * 3 + 5 * -4)]


def test_swiglu_brute_force():
    g = np.array([[1.0, 0.0], [0.0, -2.0]], np.float32)
    u = np.array([[0.5, 0.0], [0.0, 1.0]], np.float32)
    x = np.array([3.0, 1.5], np.float32)
    got = om.swiglu_f64(g, u, x)
    s = lambda v: v / (1 + math.exp(-v))  # noqa: E731
    assert np.allclose(got, [s(3.0) * 1.5, s(-3.0) * 1.5], rtol=0, atol=1e-15)


def test_bf16_rounding_rne():
    # 1 + 2^-8 is halfway between bf16 1.0 and 1 + 2^-7 -> ties to even (1.0);
    # 1 + 3*2^-8 is halfway between 1 + 2^-7 and 1 + 2^-6 -> ties to even (1 + 2^-6)
    v = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, 1 + 2 ** -8 + 2 ** -20, -2.5], np.float32)
    assert om.bf16_round(v).tolist() == [1.0, 1 + 2 ** -6, 1 + 2 ** -7, -2.5]


def test_prefill_oracle_definition():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 8)).astype(np.float32)
    a_bits = om.f32_to_bf16_bits(rng.standard_normal((3, 8)).astype(np.float32))
    awq = rng.uniform(0.5, 2, 8).astype(np.float32)
    got = om.prefill_f64(w, a_bits, awq)
    a32 = om.bf16_bits_to_f32(a_bits)
    for m in range(3):
        for n in range(4):
            terms = [float(om.bf16_round(np.array([a32[m, k] * awq[k]], np.float32))[0]) * float(w[n, k]) for k in range(8)]
            assert abs(got[m, n] - math.fsum(terms)) <= 1e-12


def test_tensor_nbytes_rules():
    # tensor_nbytes (qw35-server/src/loader/tensors.rs:123-172): (8,34) q8_0, (256,144) Q4_K, (8,4) GF4
    assert om.tensor_nbytes(om.TYPE_Q8_0, 4096, 4096) == 4096 * 128 * 34
    assert om.tensor_nbytes(om.TYPE_Q4_K, 248320, 4096) == 572_129_280
    assert om.tensor_nbytes(om.TYPE_GF4, 12288, 4096) == 25_165_824
