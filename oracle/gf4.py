"""GF4 weight codec — numpy restatement of the reference packer/decoder.

Test infrastructure only (see ``oracle/__init__.py``).

GF4 (GGUF type-id 100, 8 elements / 4 bytes, ``tools/gguf_custom_types.py:26-30``,
``qw35-server/src/loader/tensors.rs:165-167``) stores each group of eight
consecutive weights of a row in one little-endian uint32:

* bits 0..7    — e5m2 scale byte ``b`` (the top byte of an IEEE binary16),
* bits 8+3i..  — 3-bit code ``c_i = q_raw_i ^ 4`` for column ``8g + i``.

Dequantisation (``tools/qw35_cook_common.py:79``):
``w_i = (4 - (c_i ^ 4)) * 0.25 * s`` with ``s = fp16(b << 8)``.  Every value is
exact in fp32, fp16 and bf16.  The reference's Metal helper
(``qw35_gf4.metal:8-20``) deviates from this for element 4; this oracle follows
the Python formula, which is the format's definition.
"""
from __future__ import annotations

import numpy as np

GF4_TYPE_ID = 100
GF4_BLOCK_ELEMS = 8
GF4_BLOCK_BYTES = 4

_F32 = np.float32


def fp32_to_e5m2_byte(values: np.ndarray) -> np.ndarray:
    """fp32 -> e5m2 byte: RNE to binary16, then round the low byte half-up.

    Follows ``tools/qw35_cook_common.py:48-51``.
    """
    half = np.asarray(values, dtype=np.float32).astype(np.float16)
    bits = half.view(np.uint16).astype(np.uint32)
    return (((bits + np.uint32(0x80)) >> np.uint32(8)) & np.uint32(0xFF)).astype(np.uint8)


def e5m2_byte_to_fp32(values: np.ndarray) -> np.ndarray:
    """e5m2 byte -> fp32 (exact): the byte is the high half of a binary16.

    Follows ``tools/qw35_cook_common.py:54-56``.
    """
    bits = np.asarray(values, dtype=np.uint8).astype(np.uint16) << np.uint16(8)
    return bits.view(np.float16).astype(np.float32)


def _quantize_with_scale(groups: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """q_raw in [0, 7] for (R, G, 8) fp32 groups and a signed per-group scale.

    Follows ``tools/qw35_cook_common.py:67-80``: an IEEE fp32 divide (0 where the
    scale is 0), ``* -4`` (exact), ``+ 4`` (rounded), rint half-to-even, clip.
    """
    ratio = np.zeros(groups.shape, dtype=np.float32)
    sc = scale[..., None].astype(np.float32)
    np.divide(groups, sc, out=ratio, where=sc != 0.0)
    t = ratio * _F32(-4.0) + _F32(4.0)
    return np.clip(np.rint(t), _F32(0.0), _F32(7.0)).astype(np.uint32)


def gf4_pack(rows: np.ndarray) -> np.ndarray:
    """Pack an fp32 [R, K] matrix into GF4 words [R, K/8] (uint32, little-endian).

    Restates ``pack_gf4_prepared(rows, scale_search=False)``
    (``tools/qw35_cook_common.py:83-119``): the group scale is the first
    max-|x| element *with its sign*, rounded to e5m2.
    """
    rows = np.asarray(rows, dtype=np.float32)
    if rows.ndim != 2 or rows.shape[1] % 8 != 0:
        raise ValueError(f"GF4 needs a 2-D matrix with columns divisible by 8, got {rows.shape}")
    groups = rows.reshape(rows.shape[0], rows.shape[1] // 8, 8)
    first_max = np.abs(groups).argmax(axis=2)
    gmax = np.take_along_axis(groups, first_max[..., None], axis=2)[..., 0]
    scale_byte = fp32_to_e5m2_byte(gmax)
    q_raw = _quantize_with_scale(groups, e5m2_byte_to_fp32(scale_byte))
    codes = q_raw ^ np.uint32(4)
    words = scale_byte.astype(np.uint32)
    for i in range(8):
        words = words | (codes[:, :, i] << np.uint32(8 + 3 * i))
    return words.astype("<u4")


def gf4_codes(words: np.ndarray) -> np.ndarray:
    """Stored 3-bit codes c_i, shape words.shape + (8,)."""
    w = np.asarray(words, dtype=np.uint32)
    shifts = np.arange(8, dtype=np.uint32) * np.uint32(3) + np.uint32(8)
    return (w[..., None] >> shifts) & np.uint32(7)


def gf4_scales(words: np.ndarray) -> np.ndarray:
    """Signed group scales s (fp32) of each word."""
    return e5m2_byte_to_fp32((np.asarray(words, dtype=np.uint32) & np.uint32(0xFF)).astype(np.uint8))


def gf4_dequant(words: np.ndarray) -> np.ndarray:
    """GF4 words [R, G] -> fp32 weights [R, 8G].

    ``x_hat = (4 - q_raw) * 0.25 * s`` (``tools/qw35_cook_common.py:79``), with
    ``q_raw = c ^ 4`` undoing the prepared packing (``:115``).
    """
    w = np.asarray(words, dtype=np.uint32)
    q_raw = (gf4_codes(w) ^ np.uint32(4)).astype(np.float32)
    s = gf4_scales(w)
    vals = (_F32(4.0) - q_raw) * _F32(0.25) * s[..., None]
    return vals.reshape(*w.shape[:-1], w.shape[-1] * 8).astype(np.float32)


def gf4_dequant_metal(words: np.ndarray) -> np.ndarray:
    """GF4 words [R, G] -> fp32 [R, 8G] as the reference's Metal decoder computes them.

    ``qw35_gf4_dot8_vec_f32`` / ``qw35_dequantize_gf4`` (``qw35_gf4.metal:8-20,41-58``)
    repack the codes as ``packed = (w & 0xfff00000) | ((w >> 4) & 0x0000fff0)``,
    shift by ``9 - 3i`` and read the two 16-bit halves as signed shorts, masking
    with ``0xe000e000`` for ``i != 0`` only, and scale by
    ``fp16(b << 8) * -0.25 * 2^-13``.  Elements 0..3 and 5..7 equal
    ``gf4_dequant``; element 4's high short keeps, below its code, the bits of
    codes 1..3, so it is ``gf4_dequant``'s value minus
    ``s/4 * (c1 | c2 << 3 | c3 << 6) / 8192``.  Test infrastructure: this build
    follows the cook formula (``gf4_dequant``); this form measures the
    difference to the reference server's kernels.
    """
    w = np.asarray(words, dtype=np.uint32)
    packed = ((w & np.uint32(0xFFF00000)) | ((w >> np.uint32(4)) & np.uint32(0x0000FFF0))).astype(np.uint32)
    scale = (e5m2_byte_to_fp32((w & np.uint32(0xFF)).astype(np.uint8)) * _F32(-0.25) * _F32(2.0 ** -13))
    out = np.empty(w.shape + (8,), dtype=np.float32)
    for i in range(4):
        shifted = (packed << np.uint32(9 - 3 * i)) & np.uint32(0xFFFFFFFF)
        if i != 0:
            shifted &= np.uint32(0xE000E000)
        lo = (shifted & np.uint32(0xFFFF)).astype(np.uint16).view(np.int16).astype(np.float32)
        hi = (shifted >> np.uint32(16)).astype(np.uint16).view(np.int16).astype(np.float32)
        out[..., i] = lo * scale
        out[..., i + 4] = hi * scale
    return out.reshape(*w.shape[:-1], w.shape[-1] * 8)


def gf4_nbytes(rows: int, k: int) -> int:
    """Tensor byte size, ``tensor_nbytes(100, n)`` (``loader/tensors.rs:165-167``)."""
    return rows * ((k + 7) // 8) * 4
