"""GF2 codec (GGUF type 101) — numpy restatement.  Test infrastructure only.

Format (``qw35-server/src/metal/qw35_gf2.metal:1-17``; size rule
``loader/tensors.rs:124-135``, 5 bytes per 16 elements): each row is a run of
80-byte super-blocks of 256 columns, 16 little-endian uint32 code words (word
``w`` holds columns ``16*w .. 16*w + 15``, code ``i`` in bits ``2i, 2i+1``)
followed by the 16 e5m2 scale bytes of those words.

Weight (``qw35_gf2_dot16`` / ``qw35_dequantize_gf2``, ``qw35_gf2.metal:19-50``):
``fl32(fl32(fl32(q * fl32(2/3)) - 1) * s)`` with ``s = fp16(b << 8)``, i.e.
``s * {-1, -1/3, +1/3, +1}`` up to the fp32 rounding of the two middle levels
(``-0.33333331``, ``0.33333337``).  ``gf2_dequant`` follows the tile form
(per-weight level times scale, as the prefill dequantiser writes it before its
half conversion); the GEMV form multiplies the scale into the 16-term sum
instead, which the GEMV oracle's fp64 tolerance covers.

The encoder is this build's own (the reference ships none for GF2): per group
of 16, ``b = e5m2(max |x|)`` by the GF4 cook's conversion
(``tools/qw35_cook_common.py:48-52``: fp16 RNE, then the low byte rounded
half-up), ``s = fp16(b << 8)``, ``t = fl(x / s)`` (0 where ``s == 0``) and
``q = clip(rint(fl(fl(t * 1.5) + 1.5)), 0, 3)``.
"""
from __future__ import annotations

import numpy as np

from .gf4 import e5m2_byte_to_fp32, fp32_to_e5m2_byte

GF2_TYPE_ID = 101
GF2_BLOCK_ELEMS = 256
GF2_BLOCK_BYTES = 80

TWO_THIRDS = np.float32(2.0 / 3.0)


def gf2_split(raw: np.ndarray, rows: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Raw bytes -> (code words uint32 [rows, k/16], scale bytes uint8 [rows, k/16])."""
    if k % GF2_BLOCK_ELEMS:
        raise ValueError("GF2 needs columns divisible by 256")
    b = np.ascontiguousarray(raw, dtype=np.uint8).reshape(rows, k // 256, 80)
    words = np.ascontiguousarray(b[..., :64]).view("<u4").reshape(rows, k // 16)
    scales = np.ascontiguousarray(b[..., 64:]).reshape(rows, k // 16)
    return words, scales


def gf2_join(words: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Inverse of ``gf2_split``: -> raw bytes uint8 [rows, k/256*80]."""
    rows, groups = words.shape
    out = np.empty((rows, groups // 16, 80), dtype=np.uint8)
    out[..., :64] = np.ascontiguousarray(words, dtype="<u4").reshape(rows, groups // 16, 16).view(np.uint8)
    out[..., 64:] = scales.reshape(rows, groups // 16, 16)
    return out.reshape(rows, -1)


def gf2_levels(q: np.ndarray) -> np.ndarray:
    """fp32 level of code q: fl(fl(q * fl(2/3)) - 1)."""
    return (np.asarray(q, dtype=np.float32) * TWO_THIRDS - np.float32(1.0)).astype(np.float32)


def gf2_codes(words: np.ndarray) -> np.ndarray:
    """uint32 [..., G] -> codes uint8 [..., G*16] in column order."""
    shifts = (2 * np.arange(16, dtype=np.uint32))
    q = (words[..., None] >> shifts) & np.uint32(3)
    return q.reshape(words.shape[:-1] + (-1,)).astype(np.uint8)


def gf2_dequant(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Raw GF2 bytes -> fp32 [rows, k], ``fl(level(q) * s)`` per weight."""
    words, scales = gf2_split(raw, rows, k)
    lev = gf2_levels(gf2_codes(words)).reshape(rows, k // 16, 16)
    s = e5m2_byte_to_fp32(scales)[..., None]
    return (lev * s).astype(np.float32).reshape(rows, k)


def gf2_quantize(w: np.ndarray) -> np.ndarray:
    """fp32 [R, K] (K % 256 == 0) -> raw GF2 bytes [R, K/256*80]."""
    w = np.asarray(w, dtype=np.float32)
    rows, k = w.shape
    if k % GF2_BLOCK_ELEMS:
        raise ValueError("GF2 needs columns divisible by 256")
    g = w.reshape(rows, k // 16, 16)
    amax = np.abs(g).max(axis=2)
    b = fp32_to_e5m2_byte(amax)
    s = e5m2_byte_to_fp32(b)[..., None]
    t = np.zeros_like(g)
    np.divide(g, s, out=t, where=s != 0)
    v = (t * np.float32(1.5)).astype(np.float32) + np.float32(1.5)
    q = np.clip(np.rint(v.astype(np.float32)), 0, 3).astype(np.uint32)
    shifts = 2 * np.arange(16, dtype=np.uint32)
    words = np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)
    return gf2_join(words, b)


def gf2_nbytes(rows: int, k: int) -> int:
    return rows * ((k + 15) // 16) * 5
