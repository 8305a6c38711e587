"""Pins of the q8_0 and Q4_K oracles (oracle/q8_0.py, oracle/q4_k.py).

gguf-py (the reference's decoder for these types, tools/qw35_cook_common.py:34-35)
is neither vendored nor installed, and no reference test pins its output, so
parity against it is unpinned.  What is pinned here: the block layouts and
formulas the reference states itself in qw35-server/src/metal/qw35_types.metal:2-36,70-83
and qw35_matvec.metal:2-38, through hand-built blocks, closed forms in plain
Python arithmetic and agreement of the two independent Q4_K restatements.
"""
from __future__ import annotations

import struct

import numpy as np

from oracle import q4_k, q8_0


def _f16(v: float) -> bytes:
    return struct.pack("<e", v)


# ---------------------------------------------------------------- q8_0

def test_q8_0_hand_block():
    qs = list(range(-127, 128, 8))[:32]
    raw = np.frombuffer(_f16(0.5) + struct.pack("<32b", *qs), dtype=np.uint8)[None, :]
    got = q8_0.q8_0_dequant(raw)[0]
    assert got.tolist() == [0.5 * q for q in qs]


def test_q8_0_closed_form_random_blocks():
    rng = np.random.default_rng(3)
    blocks = []
    want = []
    for _ in range(200):
        d = float(np.float16(rng.standard_normal() * 10 ** rng.uniform(-6, 2)))
        qs = rng.integers(-128, 128, 32).tolist()
        blocks.append(_f16(d) + struct.pack("<32b", *qs))
        want.extend(d * q for q in qs)  # exact in float64 and in float32
    raw = np.frombuffer(b"".join(blocks), dtype=np.uint8)[None, :]
    got = q8_0.q8_0_dequant(raw)[0]
    assert got.astype(np.float64).tolist() == want


def test_q8_0_layout_and_encoder():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((5, 128)) * 0.02).astype(np.float32)
    raw = q8_0.q8_0_quantize(w)
    assert raw.shape == (5, 4 * 34) and q8_0.q8_0_nbytes(5, 128) == raw.size
    deq = q8_0.q8_0_dequant(raw)
    d = np.abs(w.reshape(5, 4, 32)).max(axis=2) / 127
    d16 = d.astype(np.float16).astype(np.float32)
    # codes are rounded against the fp32 scale while the block stores it in fp16
    bound = 0.5 * d + 127 * np.abs(d16 - d) + 1e-12
    assert np.all(np.abs(deq - w).reshape(5, 4, 32).max(axis=2) <= bound * (1 + 1e-5))


# ---------------------------------------------------------------- Q4_K

def _q4k_block(d: float, dmin: float, sc, m, q) -> bytes:
    """Hand-pack one super-block from 8 scales, 8 mins and 256 nibbles."""
    scales = bytearray(12)
    for j in range(4):
        scales[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        scales[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        scales[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return _f16(d) + _f16(dmin) + bytes(scales) + bytes(qs)


def _q4k_closed(d, dmin, sc, m, q):
    d32 = float(np.float16(d))
    dm32 = float(np.float16(dmin))
    return [np.float32(d32 * sc[e // 32] * q[e] - dm32 * m[e // 32]) for e in range(256)]


def test_q4_k_single_subscale_blocks():
    rng = np.random.default_rng(5)
    for j in range(8):
        sc = [0] * 8
        m = [0] * 8
        sc[j] = 37 if j < 4 else 53  # high sub-blocks exercise the split 6-bit packing
        q = rng.integers(0, 16, 256).tolist()
        raw = np.frombuffer(_q4k_block(0.25, 0.0, sc, m, q), dtype=np.uint8)[None, :]
        got = q4_k.q4_k_dequant(raw)[0]
        want = np.zeros(256, np.float32)
        want[32 * j:32 * j + 32] = [0.25 * sc[j] * v for v in q[32 * j:32 * j + 32]]
        assert np.array_equal(got, want), j


def test_q4_k_dmin_only_blocks():
    for j in range(8):
        m = [0] * 8
        m[j] = 63 - j
        raw = np.frombuffer(_q4k_block(1.0, 0.5, [0] * 8, m, [15] * 256), dtype=np.uint8)[None, :]
        got = q4_k.q4_k_dequant(raw)[0]
        want = np.zeros(256, np.float32)
        want[32 * j:32 * j + 32] = -0.5 * m[j]
        assert np.array_equal(got, want), j


def test_q4_k_closed_form_hand_blocks():
    rng = np.random.default_rng(6)
    for _ in range(50):
        d = float(rng.uniform(-2, 2))
        dmin = float(rng.uniform(0, 1))
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        q = rng.integers(0, 16, 256).tolist()
        raw = np.frombuffer(_q4k_block(d, dmin, sc, m, q), dtype=np.uint8)[None, :]
        assert np.array_equal(q4_k.q4_k_dequant(raw)[0], np.array(_q4k_closed(d, dmin, sc, m, q), np.float32))


def test_q4_k_scalar_and_tile_forms_agree_on_random_bytes():
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 256, (64, 144 * 16), dtype=np.uint8)
    # keep d and dmin finite (exponent != 31) so both forms compare bit-for-bit
    blocks = raw.reshape(64, 16, 144)
    for off in (1, 3):
        blocks[..., off] &= np.uint8(0xFB)
    a = q4_k.q4_k_dequant(raw)
    b = q4_k.q4_k_dequant_tiles(raw)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4_k_scale_packing_exhaustive():
    for j in range(8):
        for v in range(64):
            sc = [0] * 8
            m = [0] * 8
            sc[j] = v
            m[j] = 63 - v
            packed = q4_k.pack_scale_min_k4(np.array([sc]), np.array([m]))
            s_got, m_got = q4_k.get_scale_min_k4(j, packed)
            assert int(s_got[0]) == v and int(m_got[0]) == 63 - v
            for jj in range(8):
                if jj != j:
                    s2, m2 = q4_k.get_scale_min_k4(jj, packed)
                    assert int(s2[0]) == 0 and int(m2[0]) == 0


def test_q4_k_encoder_roundtrip():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((6, 512)) * 0.02).astype(np.float32)
    raw = q4_k.q4_k_quantize(w)
    assert raw.shape == (6, 2 * 144) and q4_k.q4_k_nbytes(6, 512) == raw.size
    deq = q4_k.q4_k_dequant(raw)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < 0.15
