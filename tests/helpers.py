"""Seeded synthetic inputs shared by the tests (numpy PCG64, as in the configs)."""
from __future__ import annotations

import numpy as np

from oracle import matvec as om

TYPES = {"gf4": om.TYPE_GF4, "gf2": om.TYPE_GF2, "q8_0": om.TYPE_Q8_0, "q4_k": om.TYPE_Q4_K, "q5_k": om.TYPE_Q5_K,
         "q6_k": om.TYPE_Q6_K}

# rel-L2 bound of a GEMV against the fp64 matvec of the dequantised weights.
GEMV_REL_L2 = 1e-3


def bf16_normal(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    """bf16_RNE(std * N(0,1)) as fp32 (the configs' weight distribution)."""
    return om.bf16_round((rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32))


def make_weight(type_id: int, rows: int, k: int, seed: int, std: float = 0.02):
    """(raw bytes uint8 [rows, row_bytes], dequantised fp32 [rows, k])."""
    rng = np.random.default_rng(seed)
    w = bf16_normal(rng, (rows, k), std)
    raw = om.quantize(type_id, w)
    return raw, om.dequant(type_id, raw, rows, k)


def random_gf4_words(rng: np.random.Generator, shape) -> np.ndarray:
    """Arbitrary 32-bit GF4 words with finite scale bytes (exponent != 31)."""
    w = rng.integers(0, 2**32, size=shape, dtype=np.uint64).astype(np.uint32)
    b = w & np.uint32(0xFF)
    bad = ((b >> np.uint32(2)) & np.uint32(0x1F)) == np.uint32(0x1F)
    return np.where(bad, w & np.uint32(0xFFFFFF83), w).astype(np.uint32)


def activations(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    return rng.standard_normal((n, k), dtype=np.float32)


def awq_scales(rng: np.random.Generator, k: int) -> np.ndarray:
    return rng.uniform(0.5, 2.0, size=k).astype(np.float32)
