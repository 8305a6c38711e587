"""Pins of the GF4 / e5m2 oracle (oracle/gf4.py) against statements that do not
reuse its formulas: IEEE binary16 closed forms, round-to-nearest semantics,
hand-computed known-answer words and packer invariants.

The reference ships no GF4 fixtures or tests (its only kernel test checks
kernel names, qw35-server/src/tests/metal_bridge.rs:1-15), so these checks are
what fixes the oracle's meaning of tools/qw35_cook_common.py:48-119.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import gf4
from oracle import matvec as om
from tests.helpers import random_gf4_words


def e5m2_closed_form(b: int) -> float:
    """IEEE-754 binary16 with the low byte zero: 1 sign, 5 exponent, 2 mantissa bits."""
    sign = -1.0 if b & 0x80 else 1.0
    e = (b >> 2) & 0x1F
    m = b & 3
    if e == 0x1F:
        return sign * math.inf if m == 0 else math.nan
    if e == 0:
        return sign * m * 2.0 ** -16
    return sign * (1.0 + m / 4.0) * 2.0 ** (e - 15)


def sext3(c: int) -> int:
    return c - 8 if c & 4 else c


def test_e5m2_decode_exhaustive():
    got = gf4.e5m2_byte_to_fp32(np.arange(256, dtype=np.uint8))
    for b in range(256):
        want = e5m2_closed_form(b)
        if math.isnan(want):
            assert math.isnan(got[b])
        else:
            assert float(got[b]) == want, b
            assert math.copysign(1.0, float(got[b])) == math.copysign(1.0, want)


def _e5m2_round_nearest_ties_away(v: float) -> int:
    """Nearest e5m2 byte to v (same sign), ties away from zero, >= 61440 -> inf."""
    mags = sorted({abs(e5m2_closed_form(b)) for b in range(128) if not math.isnan(e5m2_closed_form(b))})
    finite = [m for m in mags if not math.isinf(m)]
    a = abs(v)
    if a >= 61440.0:
        mag = math.inf
    else:
        lo = max(m for m in finite if m <= a)
        hi = min([m for m in finite if m >= a] or [math.inf])
        mag = lo if (a - lo) < (hi - a) else hi
    for b in range(128):
        if e5m2_closed_form(b) == mag:
            return b | (0x80 if math.copysign(1.0, v) < 0 else 0)
    raise AssertionError(v)


def test_e5m2_encode_all_fp16_inputs():
    """Every finite binary16 value is encoded to the nearest e5m2 value, ties away from zero."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    enc = gf4.fp32_to_e5m2_byte(vals)
    rng = np.random.default_rng(0)
    idx = np.concatenate([np.arange(0, 65536, 37), rng.integers(0, 65536, 3000)])
    for i in idx:
        v = float(vals[i])
        if math.isnan(v) or math.isinf(v):
            continue
        assert int(enc[i]) == _e5m2_round_nearest_ties_away(v), (hex(int(bits[i])), v)


def test_e5m2_roundtrip_identity():
    b = np.arange(256, dtype=np.uint8)
    vals = gf4.e5m2_byte_to_fp32(b)
    finite = np.isfinite(vals)
    assert np.array_equal(gf4.fp32_to_e5m2_byte(vals[finite]), b[finite])


def test_e5m2_double_rounding_known_answer():
    # 1.125 - 2^-13 first rounds to binary16 1.125 (a tie for e5m2), which then
    # rounds away to 1.25 (0x3D); a direct nearest-e5m2 rounding would give 1.0.
    assert int(gf4.fp32_to_e5m2_byte(np.float32(1.125 - 2.0 ** -13))) == 0x3D
    assert int(gf4.fp32_to_e5m2_byte(np.float32(1.1))) == 0x3C
    assert int(gf4.fp32_to_e5m2_byte(np.float32(-0.5))) == 0xB8


def test_gf4_dequant_exhaustive_scale_code_position():
    """All 256 scale bytes x 8 codes x 8 positions against -sext3(c) * s / 4."""
    for b in range(256):
        s = e5m2_closed_form(b)
        for pos in range(8):
            words = np.array([b | (c << (8 + 3 * pos)) for c in range(8)], dtype=np.uint32)
            got = gf4.gf4_dequant(words[None, :])[0].reshape(8, 8)
            for c in range(8):
                want = -sext3(c) * s / 4.0 if not math.isinf(s) or sext3(c) != 0 else math.nan
                v = float(got[c, pos])
                if math.isnan(want):
                    assert math.isnan(v)
                else:
                    assert v == want, (b, c, pos)
                # every other position holds code 0 -> weight 0 (NaN only for inf/NaN scales)
                others = np.delete(got[c], pos)
                if math.isfinite(s):
                    assert np.all(others == 0.0)


def test_gf4_special_words():
    assert np.all(gf4.gf4_dequant(np.zeros((1, 3), np.uint32)) == 0.0)
    # code 4 (q_raw 0) is +s, code 3 (q_raw 7) is -0.75 s
    w = np.array([[0x3C | (4 << 8) | (3 << 11)]], dtype=np.uint32)  # s = 1.0
    got = gf4.gf4_dequant(w)[0]
    assert got[0] == 1.0 and got[1] == -0.75 and np.all(got[2:] == 0.0)


@pytest.mark.parametrize(
    "group,word",
    [
        # gmax is the first max-|x| element with its sign; -0.5 clips to -0.375 (levels are s*{1..-0.75})
        ([0.5, -0.25, 0.0, 0.125, -0.5, 0.375, 0.25, -0.125], 0x3ABE1438),
        # tie in |x|: the first (negative) element is the scale; +0.5 clips to +0.375
        ([-0.5, 0.5, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0], 0x00001CB8),
        # all-zero group -> zero word
        ([0.0] * 8, 0x00000000),
        # rint ties to even: -4r+4 = 2.5 -> 2, 3.5 -> 4, 0.5 -> 0, 1.5 -> 2, 7.5 -> 8 -> clip 7, 6.5 -> 6, 5.5 -> 6
        ([1.0, 0.375, 0.125, 0.875, 0.625, -0.875, -0.625, -0.375], 0x49E8343C),
    ],
)
def test_gf4_pack_known_answers(group, word):
    got = gf4.gf4_pack(np.array([group], dtype=np.float32))
    assert got.shape == (1, 1) and int(got[0, 0]) == word


def test_gf4_known_answer_dequant():
    w = np.array([[0x3ABE1438, 0x49E8343C]], dtype=np.uint32)
    got = gf4.gf4_dequant(w)[0]
    assert got.tolist() == [0.5, -0.25, 0.0, 0.125, -0.375, 0.375, 0.25, -0.125,
                            1.0, 0.5, 0.0, 1.0, 0.5, -0.75, -0.5, -0.5]


def test_gf4_pack_invariants():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 256)) * np.exp(rng.uniform(-6, 3, (64, 1)))).astype(np.float32)
    words = gf4.gf4_pack(x)
    xh = gf4.gf4_dequant(words)
    # repacking the reconstruction is idempotent (its first max element is exactly s)
    assert np.array_equal(gf4.gf4_pack(xh), words)
    # reconstruction is exact in bf16 and fp16 (<= 5 significant bits)
    assert np.array_equal(xh.astype(np.float16).astype(np.float32), xh)
    b16 = (xh.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    assert np.array_equal(b16, xh)
    # error bound: |x - x_hat| <= 0.25 |s| + |gmax - s| per group (clipping of
    # opposite-sign extremes to -0.75 s and of gmax when s rounds down)
    s = gf4.gf4_scales(words)
    g = x.reshape(64, 32, 8)
    first = np.abs(g).argmax(axis=2)
    gmax = np.take_along_axis(g, first[..., None], axis=2)[..., 0]
    err = np.abs(g - xh.reshape(64, 32, 8)).max(axis=2)
    assert np.all(err <= 0.25 * np.abs(s) + np.abs(gmax - s) + 1e-30)
    # in-range elements (|x/s| <= 0.875 on the negative side) are within half a step
    ratio = g / np.where(s == 0, 1, s)[..., None]
    inner = (ratio >= -0.875) & (ratio <= 1.0)
    e_inner = np.abs(g - xh.reshape(64, 32, 8))
    assert np.all(e_inner[inner] <= (0.125 * np.abs(s)[..., None] * (1 + 1e-6)).repeat(8, axis=2)[inner])


def test_gf4_nbytes_matches_loader_rule():
    # tensor_nbytes(100, n) = ceil(n/8) * 4 (qw35-server/src/loader/tensors.rs:165-167)
    assert gf4.gf4_nbytes(12288, 4096) == 25_165_824
    assert gf4.gf4_nbytes(4096, 12288) == 25_165_824


def test_metal_form_hand_word():
    """Scale byte 0x3C (s = 1.0), codes c0..c7 = 1, 2, 3, 4, 5, 6, 7, 0.  By hand:
    element i = -sext3(c_i) / 4 (c = 4 -> +1.0, c = 5 -> +0.75, c = 7 -> +0.25),
    and the Metal element 4 = 0.75 - (2 | 3 << 3 | 4 << 6) / 8192 / 4 = 0.74139404296875."""
    codes = [1, 2, 3, 4, 5, 6, 7, 0]
    word = 0x3C
    for i, c in enumerate(codes):
        word |= c << (8 + 3 * i)
    w = np.array([[word]], dtype=np.uint32)
    cook = [-0.25, -0.5, -0.75, 1.0, 0.75, 0.5, 0.25, 0.0]
    assert gf4.gf4_dequant(w)[0].tolist() == cook
    metal = gf4.gf4_dequant_metal(w)[0].tolist()
    assert metal == cook[:4] + [0.74139404296875] + cook[5:]


def test_metal_form_differs_only_in_element_4_and_gemv_bound():
    """On arbitrary finite words, the Metal form equals the cook formula except
    element 4, which differs by exactly -s/4 * (c1 | c2 << 3 | c3 << 6) / 8192
    (< 1/16 of a quantisation step; zeros may differ in sign); a GEMV's
    difference is bounded by the sum of those terms times |x_{8g+4}|, and on
    the config-1 weight distribution it is about 0.6% relative L2."""
    rng = np.random.default_rng(17)
    w = random_gf4_words(rng, (64, 512))
    cook = gf4.gf4_dequant(w).reshape(64, 512, 8)
    metal = gf4.gf4_dequant_metal(w).reshape(64, 512, 8)
    others = [0, 1, 2, 3, 5, 6, 7]
    assert np.array_equal(cook[..., others], metal[..., others])  # by value: zeros differ in sign
    s = gf4.e5m2_byte_to_fp32((w & 0xFF).astype(np.uint8)).astype(np.float64)
    e = (((w >> 11) & 7) | (((w >> 14) & 7) << 3) | (((w >> 17) & 7) << 6)).astype(np.float64)
    assert np.array_equal(metal[..., 4].astype(np.float64) - cook[..., 4].astype(np.float64), -s / 4 * e / 8192)
    assert np.all(e <= 511) and np.all(np.abs(s / 4 * e / 8192) <= np.abs(s) / 4 * 0.0624)
    x = rng.standard_normal(4096).astype(np.float64)
    dy = metal.reshape(64, 4096).astype(np.float64) @ x - cook.reshape(64, 4096).astype(np.float64) @ x
    bound = (np.abs(s) / 4 * e / 8192 * np.abs(x[4::8])[None, :]).sum(axis=1)
    assert np.all(np.abs(dy) <= bound * (1 + 1e-12))
    # config-1 distribution (bf16 0.02 N(0,1) rows packed by pack_gf4_prepared): rel-L2 of the difference
    wts = om.bf16_round((rng.standard_normal((256, 4096), dtype=np.float32) * np.float32(0.02)))
    words = gf4.gf4_pack(wts)
    y_cook = gf4.gf4_dequant(words).astype(np.float64) @ x
    y_metal = gf4.gf4_dequant_metal(words).astype(np.float64) @ x
    rel = np.linalg.norm(y_metal - y_cook) / np.linalg.norm(y_cook)
    assert 1e-4 < rel < 5e-2, rel
