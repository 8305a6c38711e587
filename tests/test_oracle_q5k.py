"""Pins of the Q5_K oracle (oracle/q5_k.py).

As for Q4_K, gguf-py is absent, so what is pinned is the block layout and
formulas of qw35-server/src/metal/qw35_types.metal:9-15 and
qw35_matvec.metal:40-62,355-456: hand-built blocks against closed forms in plain
Python arithmetic (the high bit of each byte of qh, the 6-bit scale packing
shared with Q4_K), bit-for-bit agreement of the two independent restatements
(factored GEMV form, tile form) on random bytes, and the encoder's fit.
"""
from __future__ import annotations

import struct

import numpy as np

from oracle import matvec as om
from oracle import q5_k


def _f16(v: float) -> bytes:
    return struct.pack("<e", v)


def _q5k_block(d: float, dmin: float, sc, m, q) -> bytes:
    """Hand-pack one super-block from 8 scales, 8 mins and 256 five-bit codes."""
    scales = bytearray(12)
    for j in range(4):
        scales[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        scales[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        scales[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    qh = bytearray(32)
    for e in range(256):
        if q[e] & 16:
            qh[e % 32] |= 1 << (e // 32)
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = (q[64 * c + l] & 15) | ((q[64 * c + 32 + l] & 15) << 4)
    return _f16(d) + _f16(dmin) + bytes(scales) + bytes(qh) + bytes(qs)


def _closed(d, dmin, sc, m, q):
    d32 = float(np.float16(d))
    dm32 = float(np.float16(dmin))
    return np.array([np.float32(d32 * sc[e // 32] * q[e] - dm32 * m[e // 32]) for e in range(256)], np.float32)


def test_q5_k_layout_constants():
    assert q5_k.Q5_K_BLOCK_BYTES == 176 and om.tensor_nbytes(om.TYPE_Q5_K, 3, 512) == 3 * 2 * 176


def test_q5_k_high_bit_positions():
    # one code of 16 (only the qh bit set) at every position in turn
    for e in range(256):
        q = [0] * 256
        q[e] = 16
        raw = np.frombuffer(_q5k_block(1.0, 0.0, [1] * 8, [0] * 8, q), dtype=np.uint8)[None, :]
        got = q5_k.q5_k_dequant(raw)[0]
        want = np.zeros(256, np.float32)
        want[e] = 16.0
        assert np.array_equal(got, want), e
        assert np.array_equal(q5_k.q5_k_dequant_tiles(raw)[0], want), e


def test_q5_k_closed_form_hand_blocks():
    rng = np.random.default_rng(11)
    for _ in range(50):
        d = float(rng.uniform(-2, 2))
        dmin = float(rng.uniform(0, 1))
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        q = rng.integers(0, 32, 256).tolist()
        raw = np.frombuffer(_q5k_block(d, dmin, sc, m, q), dtype=np.uint8)[None, :]
        want = _closed(d, dmin, sc, m, q)
        assert np.array_equal(q5_k.q5_k_dequant(raw)[0], want)
        assert np.array_equal(q5_k.q5_k_codes(raw)[0, 0].astype(int), np.array(q))


def test_q5_k_factored_and_tile_forms_agree_on_random_bytes():
    rng = np.random.default_rng(12)
    raw = rng.integers(0, 256, (64, 176 * 16), dtype=np.uint8)
    blocks = raw.reshape(64, 16, 176)
    for off in (1, 3):  # finite d and dmin (exponent != 31)
        blocks[..., off] &= np.uint8(0xFB)
    a = q5_k.q5_k_dequant(raw)
    b = q5_k.q5_k_dequant_tiles(raw)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q5_k_encoder_levels_and_roundtrip():
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((6, 512)) * 0.02).astype(np.float32)
    raw = q5_k.q5_k_quantize(w)
    assert raw.shape == (6, 2 * 176)
    codes = q5_k.q5_k_codes(raw)
    assert codes.max() <= 31 and codes.max() >= 16  # the fifth bit is used
    deq = q5_k.q5_k_dequant(raw)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < 0.08  # twice the levels of Q4_K (< 0.15 there)
    # an all-zero row decodes to zeros (scales 0, codes 0)
    zero = q5_k.q5_k_quantize(np.zeros((2, 256), np.float32))
    assert not q5_k.q5_k_dequant(zero).any() and not q5_k.q5_k_codes(zero).any()
