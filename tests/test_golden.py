"""The oracle still reproduces the committed golden fixtures bit-for-bit."""
from __future__ import annotations

import os

import numpy as np

from oracle import gf4, q4_k, q8_0
from oracle import matvec as om

FIX = os.path.join(os.path.dirname(__file__), "golden", "gemv_golden.npz")


def _load():
    return np.load(FIX, allow_pickle=False)


def _same(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype.kind == "f":
        a32 = np.ascontiguousarray(a, np.float32)
        b32 = np.ascontiguousarray(b, np.float32)
        return bool(np.all((a32.view(np.uint32) == b32.view(np.uint32)) | (np.isnan(a32) & np.isnan(b32))))
    return np.array_equal(a, b)


def test_golden_gf4():
    g = _load()
    assert _same(gf4.gf4_pack(g["gf4_deq"]), g["gf4_words"])
    assert _same(gf4.gf4_dequant(g["gf4_words"]), g["gf4_deq"])
    assert _same(gf4.gf4_dequant(g["gf4_any_words"]), g["gf4_any_deq"])
    assert np.allclose(om.matvec_f64(g["gf4_deq"], g["x"], g["awq"]), g["gf4_y"], rtol=0, atol=1e-12)
    tab = gf4.e5m2_byte_to_fp32(np.arange(256, dtype=np.uint8))
    assert _same(tab, g["e5m2_table"])


def test_golden_kquants():
    g = _load()
    assert _same(q8_0.q8_0_dequant(g["q8_0_raw"]), g["q8_0_deq"])
    assert _same(q4_k.q4_k_dequant(g["q4_k_raw"]), g["q4_k_deq"])
    assert _same(q4_k.q4_k_dequant_tiles(g["q4_k_raw"]), g["q4_k_deq"])
    assert np.allclose(om.matvec_f64(g["q8_0_deq"], g["x"], g["awq"]), g["q8_0_y"], rtol=0, atol=1e-12)
    assert np.allclose(om.matvec_f64(g["q4_k_deq"], g["x"], g["awq"]), g["q4_k_y"], rtol=0, atol=1e-12)
