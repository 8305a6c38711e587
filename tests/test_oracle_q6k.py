"""Pins of the Q6_K oracle (oracle/q6_k.py) and of the greedy argmax rule.

The reference ships no Q6_K vectors; these pins are closed forms, hand-built
blocks and independent restatements of the reference's own statements:
the element mapping, the bit extraction of the Q6_K GEMV / argmax-head kernels
(qw35_matvec.metal:458-542, qw35_output.metal:2-80) and the tile dequantiser
(qw35_matvec.metal:65-98)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import c_oracle
from oracle import matvec as om
from oracle import q6_k


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _random_raw(rng, n_blocks):
    raw = rng.integers(0, 256, size=n_blocks * q6_k.Q6_K_BLOCK_BYTES, dtype=np.uint8)
    blk = q6_k.as_blocks(raw)
    blk["d"] = (rng.standard_normal(blk.shape) * 0.01).astype(np.float16)
    return raw


def test_block_layout():
    assert q6_k.BLOCK_DTYPE.itemsize == 210
    assert [q6_k.BLOCK_DTYPE.fields[f][1] for f in ("ql", "qh", "scales", "d")] == [0, 128, 192, 208]


def test_known_answer_block():
    # element e = 128h + 32g + l: code 32 + (e % 7) - 3 in every position, scales s = e // 16 - 8, d = 0.5
    codes = np.array([32 + (e % 7) - 3 for e in range(256)])
    ql = np.zeros(128, np.uint32)
    qh = np.zeros(64, np.uint32)
    for e, q in enumerate(codes):
        h, g, l = e // 128, (e % 128) // 32, e % 32
        ql[64 * h + 32 * (g & 1) + l] |= (q & 15) << (4 * (g >> 1))
        qh[32 * h + l] |= (q >> 4) << (2 * g)
    scales = np.arange(16) - 8
    raw = q6_k.make_block(ql, qh, scales, 0.5)
    w = q6_k.q6_k_dequant(raw, 1, 256)[0]
    want = np.array([0.5 * (e // 16 - 8) * ((e % 7) - 3) for e in range(256)], dtype=np.float32)
    assert np.array_equal(w, want)


@pytest.mark.parametrize("q", range(64))
def test_every_code_closed_form(q):
    # all 256 elements hold code q; scale of sub-block j is 2j - 15; d = -0.375
    ql = np.full(128, (q & 15) | ((q & 15) << 4), np.uint8)
    hb = q >> 4
    qh = np.full(64, hb | (hb << 2) | (hb << 4) | (hb << 6), np.uint8)
    scales = 2 * np.arange(16) - 15
    w = q6_k.q6_k_dequant(q6_k.make_block(ql, qh, scales, -0.375), 1, 256)[0]
    want = np.repeat(np.float32(-0.375) * scales.astype(np.float32), 16) * np.float32(q - 32)
    assert np.array_equal(_bits(w), _bits(want))


def test_gemv_form_agrees_bit_for_bit():
    rng = np.random.default_rng(11)
    raw = _random_raw(rng, 6 * 2)
    a = q6_k.q6_k_dequant(raw, 6, 512)
    b = q6_k.q6_k_dequant_gemv_form(raw, 6, 512)
    assert np.array_equal(_bits(a), _bits(b))


def test_tile_form_agrees_in_value():
    # The tile form rounds (d*sc)*q_unsigned before subtracting 32*d*sc; on
    # these blocks every value agrees (zeros may differ in sign: x - x = +0).
    rng = np.random.default_rng(12)
    raw = _random_raw(rng, 4000)
    a = q6_k.q6_k_dequant(raw, 4000, 256)
    c = q6_k.q6_k_dequant_tile_form(raw, 4000, 256)
    assert np.array_equal(a, c)


def test_c_twin_agrees():
    if not c_oracle.LIB.exists():
        import subprocess

        subprocess.run(["make", "-C", str(c_oracle.LIB.parent.parent)], check=True, capture_output=True)
    rng = np.random.default_rng(13)
    raw = _random_raw(rng, 8 * 4)
    assert np.array_equal(_bits(c_oracle.dequant(om.TYPE_Q6_K, raw, 8, 1024)), _bits(q6_k.q6_k_dequant(raw, 8, 1024)))


def test_encoder_round_trip_bound():
    rng = np.random.default_rng(14)
    x = (rng.standard_normal((12, 1024)) * 0.02).astype(np.float32)
    raw = q6_k.q6_k_quantize(x)
    assert raw.size == 12 * 4 * 210
    deq = q6_k.q6_k_dequant(raw, 12, 1024)
    blk = q6_k.as_blocks(raw).reshape(12, 4)
    step = np.abs(blk["d"].astype(np.float64)[..., None] * blk["scales"].astype(np.float64))
    step = np.repeat(step, 16, axis=-1).reshape(12, 1024)
    # every element within half a step (plus the clip of the largest sub-block
    # magnitude, which the 31-level positive side can cost one step)
    assert np.all(np.abs(deq.astype(np.float64) - x) <= 1.0 * step + 1e-12)
    assert np.linalg.norm(deq - x) / np.linalg.norm(x) < 0.05


def test_argmax_rule_ties_nan_inf():
    lg = np.array([[1.0, 3.0, 3.0, -2.0],
                   [np.nan, 2.0, np.nan, 2.0],
                   [np.nan, np.nan, np.nan, np.nan],
                   [-np.inf, -np.inf, -np.inf, -np.inf],
                   [0.0, -0.0, 0.0, -1.0]], dtype=np.float32)
    ids, best = om.argmax_rule(lg)
    assert ids.tolist() == [1, 1, 0xFFFFFFFF, 0, 0]
    assert best[0] == 3.0 and best[1] == 2.0 and best[2] == -np.inf and best[3] == -np.inf and best[4] == 0.0


def test_argmax_rule_matches_sequential_statement():
    # the reference's sequential scan, restated literally, on random rows with ties
    rng = np.random.default_rng(15)
    lg = rng.integers(-5, 5, size=(6, 300)).astype(np.float32)
    lg[rng.random(lg.shape) < 0.05] = np.nan
    ids, best = om.argmax_rule(lg)
    for b in range(lg.shape[0]):
        bv, bi = -np.inf, 0xFFFFFFFF
        for i, v in enumerate(lg[b]):
            if v > bv or (v == bv and i < bi):
                bv, bi = v, i
        assert ids[b] == bi and best[b] == bv
