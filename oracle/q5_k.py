"""ggml Q5_K codec — numpy restatement.  Test infrastructure only.

Super-block of 256 weights = 176 bytes (``qw35_types.metal:9-15``;
``tensor_nbytes(13, n)`` = ``(256, 176)`` at ``loader/tensors.rs:145``):

* ``d``, ``dmin``  — little-endian binary16 super-scales,
* ``scales[12]``   — eight (6-bit scale, 6-bit min) pairs, packed as for Q4_K
  (``qw35_get_scale_min_k4``, ``qw35_types.metal:70-83``),
* ``qh[32]``       — bit ``j`` of byte ``l`` is bit 4 of element ``32*j + l``,
* ``qs[128]``      — low nibbles, laid out as Q4_K's: byte ``32*c + l`` holds
  element ``64*c + l`` (low) and ``64*c + 32 + l`` (high).

Weight ``e`` of sub-block ``j = e // 32`` is ``fl32(d*sc_j*q_e - dmin*m_j)``
with the 5-bit ``q_e = nibble + 16*bit``; both products are exact in fp32
(at most 22 significant bits), so there is exactly one rounding.

Two restatements are kept and must agree bit-for-bit: ``q5_k_dequant``
follows the factored decode GEMV ``qw35_decode_matmul_q5_k_2row_f32``
(``qw35_matvec.metal:355-456``: ``q & 0x0F`` / ``(q & 0xF0) / 16`` plus
``16 *`` the ``qh`` bit, times ``d*sc``, minus ``dmin*m``), and
``q5_k_dequant_tiles`` follows the tile form ``qw35_dequantize_q5_k``
(``qw35_matvec.metal:40-62``: ``d/16`` for high nibbles, high value 16 or 256).

The encoder is this build's own, the Q4_K fit with 31 levels: per 32-element
sub-block ``scale = (max - min(min, 0)) / 31`` and ``mins = -min(min, 0)``;
``d = fp16(max scale / 63)``, ``dmin = fp16(max mins / 63)``; 6-bit ``sc``,
``m`` by rint against them; ``q = clip(rint((x + dmin*m) / (d*sc)), 0, 31)``.
"""
from __future__ import annotations

import numpy as np

from .q4_k import _get_scale_min_k4_pair, get_scale_min_k4, pack_scale_min_k4

Q5_K_TYPE_ID = 13
Q5_K_BLOCK_ELEMS = 256
Q5_K_BLOCK_BYTES = 176

BLOCK_DTYPE = np.dtype([("d", "<f2"), ("dmin", "<f2"), ("scales", "u1", (12,)), ("qh", "u1", (32,)),
                        ("qs", "u1", (128,))])
assert BLOCK_DTYPE.itemsize == Q5_K_BLOCK_BYTES


def q5_k_blocks(raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    return raw.reshape(raw.shape[0], -1).view(BLOCK_DTYPE)


def q5_k_codes(raw: np.ndarray) -> np.ndarray:
    """5-bit codes uint8 [R, K/256, 256] (nibble from qs, bit 4 from qh)."""
    b = q5_k_blocks(raw)
    qs = b["qs"].astype(np.uint32)
    qh = b["qh"].astype(np.uint32)
    out = np.empty(b.shape + (256,), dtype=np.uint8)
    for j in range(8):
        base = (j // 2) * 32
        nib = qs[..., base:base + 32]
        nib = (nib & 0x0F) if j % 2 == 0 else (nib >> 4)
        out[..., 32 * j:32 * j + 32] = nib | (((qh >> j) & 1) << 4)
    return out


def q5_k_dequant(raw: np.ndarray) -> np.ndarray:
    """Raw bytes [R, K/256*176] -> fp32 [R, K], the decode GEMV's factored form
    (``qw35_matvec.metal:355-456``)."""
    b = q5_k_blocks(raw)
    d = b["d"].astype(np.float32)
    dmin = b["dmin"].astype(np.float32)
    qs = b["qs"].astype(np.uint32)
    qh = b["qh"].astype(np.uint32)
    out = np.empty(b.shape + (256,), dtype=np.float32)
    for j in range(8):
        sc, m = get_scale_min_k4(j, b["scales"])
        base = (j // 2) * 32
        nib = qs[..., base:base + 32]
        if j % 2 == 0:
            lo = (nib & 0x0F).astype(np.float32)
        else:
            lo = (nib & 0xF0).astype(np.float32) / np.float32(16.0)
        hi = np.where(((qh >> j) & 1) != 0, np.float32(16.0), np.float32(0.0))
        q = (lo + hi).astype(np.float32)
        dsc = d * sc.astype(np.float32)
        mm = dmin * m.astype(np.float32)
        out[..., 32 * j:32 * (j + 1)] = dsc[..., None] * q - mm[..., None]
    return out.reshape(b.shape[0], -1)


def q5_k_dequant_tiles(raw: np.ndarray) -> np.ndarray:
    """Same as ``q5_k_dequant`` through the 16-element tile form (``qw35_matvec.metal:40-62``)."""
    b = q5_k_blocks(raw)
    qs = b["qs"].astype(np.uint32)
    qh_all = b["qh"].astype(np.uint32)
    d0 = b["d"].astype(np.float32)
    dmin = b["dmin"].astype(np.float32)
    out = np.empty(b.shape + (256,), dtype=np.float32)
    for il_full in range(16):
        is_ = (il_full // 4) * 2
        off = 32 * (il_full // 4) + 16 * (il_full & 1)
        hoff = 16 * (il_full & 1)
        high_mask = np.uint32(1 << (il_full // 2))
        il = il_full & 3
        sc, m = _get_scale_min_k4_pair(is_, il // 2, b["scales"])
        d = d0 * (np.float32(1.0) if il < 2 else np.float32(1.0 / 16.0))
        dl = d * sc.astype(np.float32)
        ml = dmin * m.astype(np.float32)
        low_mask = np.uint32(0x0F) if il < 2 else np.uint32(0xF0)
        high_value = np.float32(16.0) if il < 2 else np.float32(256.0)
        q = qs[..., off:off + 16]
        qh = qh_all[..., hoff:hoff + 16]
        qv = (q & low_mask).astype(np.float32) + np.where((qh & high_mask) != 0, high_value, np.float32(0.0))
        out[..., il_full * 16:(il_full + 1) * 16] = dl[..., None] * qv.astype(np.float32) - ml[..., None]
    return out.reshape(b.shape[0], -1)


def q5_k_quantize(rows: np.ndarray) -> np.ndarray:
    """fp32 [R, K] (K % 256 == 0) -> raw Q5_K bytes [R, K/256*176]."""
    rows = np.asarray(rows, dtype=np.float32)
    r, k = rows.shape
    if k % 256:
        raise ValueError("Q5_K needs columns divisible by 256")
    nb = k // 256
    sub = rows.reshape(r, nb, 8, 32)
    lo = np.minimum(sub.min(axis=3), 0.0).astype(np.float32)
    hi = sub.max(axis=3).astype(np.float32)
    scale = ((hi - lo) / np.float32(31.0)).astype(np.float32)
    mins = (-lo).astype(np.float32)
    d = (scale.max(axis=2) / np.float32(63.0)).astype(np.float16)
    dmin = (mins.max(axis=2) / np.float32(63.0)).astype(np.float16)
    df = d.astype(np.float32)[..., None]
    dminf = dmin.astype(np.float32)[..., None]
    sc = np.zeros_like(scale)
    np.divide(scale, df, out=sc, where=df != 0)
    sc = np.clip(np.rint(sc), 0, 63).astype(np.uint32)
    mq = np.zeros_like(mins)
    np.divide(mins, dminf, out=mq, where=dminf != 0)
    mq = np.clip(np.rint(mq), 0, 63).astype(np.uint32)
    step = df * sc.astype(np.float32)
    offs = dminf * mq.astype(np.float32)
    qf = np.zeros_like(sub)
    np.divide(sub + offs[..., None], step[..., None], out=qf, where=step[..., None] != 0)
    q = np.clip(np.rint(qf), 0, 31).astype(np.uint8)  # [r, nb, 8, 32]
    out = np.zeros((r, nb), dtype=BLOCK_DTYPE)
    out["d"] = d
    out["dmin"] = dmin
    out["scales"] = pack_scale_min_k4(sc, mq)
    qh = np.zeros((r, nb, 32), dtype=np.uint8)
    for j in range(8):
        qh |= ((q[:, :, j, :] >> 4) & 1) << j
    out["qh"] = qh
    qs = np.zeros((r, nb, 128), dtype=np.uint8)
    for c in range(4):
        qs[..., 32 * c:32 * c + 32] = (q[:, :, 2 * c, :] & 0x0F) | ((q[:, :, 2 * c + 1, :] & 0x0F) << 4)
    out["qs"] = qs
    return out.view(np.uint8).reshape(r, nb * 176)


def q5_k_nbytes(rows: int, k: int) -> int:
    return rows * ((k + 255) // 256) * 176
