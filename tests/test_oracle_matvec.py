"""Pins of the fp64 matvec / prefill oracle (oracle/matvec.py) by brute force."""
from __future__ import annotations

import math
import struct

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
    """prefill_f64 is the fp64 product of the unrounded activations (bf16 bits
    read exactly, or fp32 values) times AWQ: brute force with math.fsum."""
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 8)).astype(np.float32)
    a32 = rng.standard_normal((3, 8)).astype(np.float32)
    a_bits = om.f32_to_bf16_bits(a32)
    awq = rng.uniform(0.5, 2, 8).astype(np.float32)
    for a, vals in ((a_bits, om.bf16_bits_to_f32(a_bits)), (a32, a32)):
        got = om.prefill_f64(w, a, awq)
        for m in range(3):
            for n in range(4):
                want = math.fsum(float(vals[m, k]) * float(awq[k]) * float(w[n, k]) for k in range(8))
                assert abs(got[m, n] - want) <= 1e-12 * max(1.0, abs(want))


def _f16_py(v: float) -> float:
    """fp16 round-to-nearest-even through the struct module (independent of numpy)."""
    return struct.unpack("<e", struct.pack("<e", v))[0]


def _staged_py(row: list[float], a_f32: bool) -> list[float]:
    """The staging restated element by element: 2^e puts max |v| in [2^14, 2^15)."""
    mx = max(abs(v) for v in row)
    e = 0 if mx == 0 else 15 - math.frexp(mx)[1]
    sc = 2.0 ** e
    out = []
    for v in row:
        s = v * sc
        hi = _f16_py(s)
        val = hi
        if a_f32:
            val = hi + _f16_py((s - hi) * 2048.0) / 2048.0
        out.append(val / sc)
    return out


def test_prefill_staged_operand_brute_force():
    """prefill_staged_operand against an element-by-element restatement that
    rounds with the struct module's binary16 packing; rows over a wide range
    of magnitudes, an all-zero row, bf16 and fp32 inputs, with and without AWQ."""
    rng = np.random.default_rng(7)
    a32 = (rng.standard_normal((5, 16)) * np.array([1e-6, 1.0, 3e4, 0.0, 7.5])[:, None]).astype(np.float32)
    awq = rng.uniform(0.5, 2, 16).astype(np.float32)
    for a_f32 in (False, True):
        a = a32 if a_f32 else om.f32_to_bf16_bits(a32)
        vals = a32 if a_f32 else om.bf16_bits_to_f32(a)
        for aw in (None, awq):
            got = om.prefill_staged_operand(a, aw, a_f32)
            for m in range(5):
                row = [float(np.float32(vals[m, k]) * (np.float32(1) if aw is None else aw[k])) for k in range(16)]
                assert got[m].tolist() == _staged_py(row, a_f32)


def test_prefill_staged_operand_precision():
    """What the staging guarantees: bf16 input without AWQ is carried exactly;
    fp32 input (hi/lo) within 2^-21 relative of each element for elements of
    at least 2^-10 of the row maximum; bf16 with AWQ within fp16's 2^-11."""
    rng = np.random.default_rng(8)
    a32 = rng.standard_normal((64, 512)).astype(np.float32)
    awq = rng.uniform(0.5, 2, 512).astype(np.float32)
    bits = om.f32_to_bf16_bits(a32)
    assert np.array_equal(om.prefill_staged_operand(bits, None, False), om.bf16_bits_to_f32(bits).astype(np.float64))
    v = (a32 * awq[None, :]).astype(np.float64)
    big = np.abs(v) >= np.max(np.abs(v), axis=1, keepdims=True) * 2.0 ** -10
    rel = np.abs(om.prefill_staged_operand(a32, awq, True) - v) / np.maximum(np.abs(v), 1e-300)
    assert np.max(rel[big]) <= 2.0 ** -21
    vb = (om.bf16_bits_to_f32(bits) * awq[None, :]).astype(np.float64)
    relb = np.abs(om.prefill_staged_operand(bits, awq, False) - vb) / np.maximum(np.abs(vb), 1e-300)
    assert np.max(relb[np.abs(vb) >= np.max(np.abs(vb), axis=1, keepdims=True) * 2.0 ** -10]) <= 2.0 ** -11


def test_prefill_direct_operand_is_bf16_of_the_product():
    rng = np.random.default_rng(9)
    a32 = rng.standard_normal((3, 8)).astype(np.float32)
    awq = rng.uniform(0.5, 2, 8).astype(np.float32)
    got = om.prefill_direct_operand(a32, awq)
    for m in range(3):
        for k in range(8):
            p = float(np.float32(a32[m, k]) * awq[k])
            b = struct.unpack("<I", struct.pack("<f", p))[0]
            lsb = (b >> 16) & 1
            r = ((b + 0x7FFF + lsb) >> 16) << 16  # round to nearest even on the top 16 bits
            assert got[m, k] == struct.unpack("<f", struct.pack("<I", r & 0xFFFFFFFF))[0]


def test_tensor_nbytes_rules():
    # tensor_nbytes (qw35-server/src/loader/tensors.rs:123-172): (8,34) q8_0, (256,144) Q4_K, (8,4) GF4
    assert om.tensor_nbytes(om.TYPE_Q8_0, 4096, 4096) == 4096 * 128 * 34
    assert om.tensor_nbytes(om.TYPE_Q4_K, 248320, 4096) == 572_129_280
    assert om.tensor_nbytes(om.TYPE_GF4, 12288, 4096) == 25_165_824
