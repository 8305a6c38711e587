"""Pins of oracle.matvec.prefill_image: fp16 round-to-nearest-even of the exact
dequantised weight.  Checked against hand-computed binary16 roundings (ties to
even, the largest finite value, overflow to inf, subnormals) and against the
exactness of GF4 weights in fp16 (3 significant bits: the image is exact)."""
from __future__ import annotations

import numpy as np

from oracle import matvec as om
from tests.helpers import make_weight


def test_f16_rounding_known_answers():
    v = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65520.0, 2.0 ** -25, 3 * 2.0 ** -26,
                  -2.5 * 2.0 ** -14, -5 * 2.0 ** -24], dtype=np.float32).reshape(1, -1)
    got = om.quantize(om.TYPE_F16, v).view("<u2").reshape(-1)
    # 1+2^-11 ties to 1.0 (even); 1+3*2^-11 ties up to 1+2^-9; 65520 rounds to inf;
    # 2^-25 ties to 0; 3*2^-26 rounds to 2^-24; -1.25*2^-13 is a normal value;
    # -5*2^-24 is exact as a subnormal
    want = [0x3C00, 0x3C02, 0x7BFF, 0x7C00, 0x0000, 0x0001, 0x8900, 0x8005]
    assert got.tolist() == want


def test_gf4_image_is_exact():
    raw, deq = make_weight(om.TYPE_GF4, 16, 1024, seed=3)
    img = om.prefill_image(om.TYPE_GF4, raw, 16, 1024)
    assert np.array_equal(img.astype(np.float32), deq)


def test_kquant_image_is_nearest():
    for t in (om.TYPE_Q8_0, om.TYPE_Q4_K):
        raw, deq = make_weight(t, 8, 1024, seed=t)
        img = om.prefill_image(t, raw, 8, 1024).astype(np.float64)
        # nearest: no other fp16 value is closer than half an fp16 ulp
        ulp = np.spacing(np.abs(img).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(img - deq) <= ulp / 2)
