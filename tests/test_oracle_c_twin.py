"""The C restatement (oracle/c) and the numpy restatement agree bit-for-bit."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import c_oracle
from oracle import matvec as om
from tests.helpers import make_weight, random_gf4_words


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not c_oracle.LIB.exists():
        import subprocess

        subprocess.run(["make", "-C", str(c_oracle.LIB.parent.parent)], check=True, capture_output=True)


def _same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


@pytest.mark.parametrize("type_id", [om.TYPE_GF4, om.TYPE_GF2, om.TYPE_Q8_0, om.TYPE_Q4_K, om.TYPE_Q5_K])
def test_c_twin_dequant(type_id):
    raw, deq = make_weight(type_id, 24, 1024, seed=type_id)
    assert _same_bits(c_oracle.dequant(type_id, raw, 24, 1024), deq)


def test_c_twin_gf4_arbitrary_words():
    words = random_gf4_words(np.random.default_rng(2), (16, 128))
    assert _same_bits(c_oracle.dequant(om.TYPE_GF4, words, 16, 1024), om.dequant(om.TYPE_GF4, words, 16, 1024))


def test_c_twin_q4_k_random_bytes():
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, (8, 144 * 4), dtype=np.uint8)
    raw.reshape(8, 4, 144)[..., 1] &= np.uint8(0xFB)
    raw.reshape(8, 4, 144)[..., 3] &= np.uint8(0xFB)
    assert _same_bits(c_oracle.dequant(om.TYPE_Q4_K, raw, 8, 1024), om.dequant(om.TYPE_Q4_K, raw, 8, 1024))


def test_c_twin_q5_k_and_gf2_random_bytes():
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, (8, 176 * 4), dtype=np.uint8)
    raw.reshape(8, 4, 176)[..., 1] &= np.uint8(0xFB)  # finite d and dmin
    raw.reshape(8, 4, 176)[..., 3] &= np.uint8(0xFB)
    assert _same_bits(c_oracle.dequant(om.TYPE_Q5_K, raw, 8, 1024), om.dequant(om.TYPE_Q5_K, raw, 8, 1024))
    g = rng.integers(0, 256, (8, 80 * 4), dtype=np.uint8)  # every scale byte, finite or not
    assert _same_bits(c_oracle.dequant(om.TYPE_GF2, g, 8, 1024), om.dequant(om.TYPE_GF2, g, 8, 1024))


def test_c_twin_matvec():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((7, 300)).astype(np.float32)
    x = rng.standard_normal((3, 300)).astype(np.float32)
    assert np.allclose(c_oracle.matvec_f64(w, x), om.matvec_f64(w, x), rtol=1e-13, atol=1e-12)
