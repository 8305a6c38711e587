"""Pins of the GF2 oracle (oracle/gf2.py) against qw35-server/src/metal/qw35_gf2.metal.

The reference has no GF2 test or packer, so the pins are: the super-block layout
and size rule (qw35_gf2.metal:1-17, loader/tensors.rs:124-135) through
hand-built blocks, the fp32 level arithmetic of qw35_gf2_dot16 /
qw35_dequantize_gf2 (:19-50) in plain Python float32 steps over every scale
byte and code, and properties of this build's encoder (exact recovery of
on-grid groups, idempotence).
"""
from __future__ import annotations

import struct

import numpy as np

from oracle import gf2
from oracle import matvec as om


def _e5m2(b: int) -> float:
    return float(np.frombuffer(struct.pack("<H", b << 8), dtype="<f2")[0])


def _level(q: int) -> np.float32:
    return np.float32(np.float32(q) * np.float32(2.0 / 3.0)) - np.float32(1.0)


def test_levels_follow_the_fp32_arithmetic():
    got = gf2.gf2_levels(np.arange(4))
    assert got.tolist() == [float(_level(q)) for q in range(4)]
    assert got[0] == -1.0 and got[3] == 1.0
    assert got[1] == np.float32(-0.33333331) and got[2] == np.float32(0.33333337)


def test_size_rule():
    # 5 bytes per 16 elements, elements padded to 16 (tensors.rs:124-135)
    assert om.tensor_nbytes(om.TYPE_GF2, 3, 512) == 3 * 2 * 80
    assert gf2.gf2_nbytes(1, 256) == 80


def test_every_scale_byte_and_code():
    # one super-block per scale byte (exponent 31 excluded: not finite); word w
    # holds codes q = (w + i) % 4 at position i, scale byte b for every word
    bytes_ = [b for b in range(256) if (b >> 2) & 0x1F != 0x1F]
    blocks = []
    want = []
    for b in bytes_:
        words = []
        for w in range(16):
            q = [(w + i) % 4 for i in range(16)]
            words.append(sum(v << (2 * i) for i, v in enumerate(q)))
            s = np.float32(_e5m2(b))
            want.extend(np.float32(_level(v) * s) for v in q)
        blocks.append(struct.pack("<16I", *words) + bytes([b] * 16))
    raw = np.frombuffer(b"".join(blocks), dtype=np.uint8)[None, :]
    got = gf2.gf2_dequant(raw, 1, 256 * len(bytes_))[0]
    assert np.array_equal(got.view(np.uint32), np.array(want, np.float32).view(np.uint32))


def test_layout_word_and_scale_positions():
    # word w of super-block c covers columns 256c + 16w ..; its scale is byte 64 + w
    rng = np.random.default_rng(1)
    rows, k = 2, 512
    raw = np.zeros((rows, k // 256 * 80), np.uint8)
    for r in range(rows):
        for c in range(k // 256):
            w = int(rng.integers(16))
            i = int(rng.integers(16))
            word = 3 << (2 * i)  # code 3 (level +1) at position i, code 0 (-1) elsewhere
            raw[r, 80 * c + 4 * w:80 * c + 4 * w + 4] = np.frombuffer(struct.pack("<I", word), np.uint8)
            raw[r, 80 * c + 64 + w] = 0x3C  # 1.0
            got = gf2.gf2_dequant(raw, rows, k)
            col = 256 * c + 16 * w
            assert got[r, col + i] == 1.0
            others = np.delete(got[r, col:col + 16], i)
            assert np.all(others == -1.0)
            raw[r, 80 * c:80 * c + 80] = 0


def test_encoder_recovers_on_grid_groups_and_is_idempotent():
    rng = np.random.default_rng(2)
    rows, k = 4, 512
    q = rng.integers(0, 4, (rows, k))
    q[:, ::16] = 3  # every group holds +1 so max |x| = s
    s = np.float32(0.046875)  # an e5m2 value (0x2A)
    w = (gf2.gf2_levels(q) * s).astype(np.float32)
    raw = gf2.gf2_quantize(w)
    words, scales = gf2.gf2_split(raw, rows, k)
    assert np.all(scales == 0x2A)
    assert np.array_equal(gf2.gf2_codes(words), q)
    assert np.array_equal(gf2.gf2_dequant(raw, rows, k), w)
    x = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
    r1 = gf2.gf2_quantize(x)
    assert np.array_equal(gf2.gf2_quantize(gf2.gf2_dequant(r1, rows, k)), r1)


def test_encoder_zero_and_sign():
    w = np.zeros((1, 256), np.float32)
    w[0, 5] = -0.5
    raw = gf2.gf2_quantize(w)
    d = gf2.gf2_dequant(raw, 1, 256)
    assert d[0, 5] == -0.5  # max |x| = 0.5 exactly representable, code 0
    assert np.all(np.abs(d[0, 16:]) == 0.0)  # all-zero groups: scale byte 0
