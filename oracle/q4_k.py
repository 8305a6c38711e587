"""ggml Q4_K codec — numpy restatement.  Test infrastructure only.

Super-block of 256 weights = 144 bytes (``qw35_types.metal:2-7``;
``tensor_nbytes(12, n)`` = ``(256, 144)`` at ``loader/tensors.rs:146``):

* ``d``, ``dmin``  — little-endian binary16 super-scales,
* ``scales[12]``   — eight (6-bit scale, 6-bit min) pairs, packed as
  ``qw35_get_scale_min_k4`` unpacks them (``qw35_types.metal:70-83``),
* ``qs[128]``      — nibbles: byte ``32*c + l`` holds element ``64*c + l`` in
  its low nibble and element ``64*c + 32 + l`` in its high nibble.

Weight ``e`` of sub-block ``j = e // 32`` is ``fl32(d*sc_j*q_e - dmin*m_j)``;
both products are exact in fp32 so there is exactly one rounding.

Two independent restatements are kept on purpose and must agree bit-for-bit:
``q4_k_dequant`` follows the scalar form ``qw35_dequant_q4_k_at``
(``qw35_matvec.metal:2-12``) and ``q4_k_dequant_tiles`` follows the tile form
``qw35_dequantize_q4_k`` + ``qw35_get_scale_min_k4_pair``
(``qw35_matvec.metal:14-38``).

The encoder is this build's own (the reference reads K-quants only through the
external gguf-py): per 32-element sub-block an affine min/max fit, then 6-bit
quantisation of the sub-scales and mins against ``d``/``dmin``.
"""
from __future__ import annotations

import numpy as np

Q4_K_TYPE_ID = 12
Q4_K_BLOCK_ELEMS = 256
Q4_K_BLOCK_BYTES = 144

BLOCK_DTYPE = np.dtype([("d", "<f2"), ("dmin", "<f2"), ("scales", "u1", (12,)), ("qs", "u1", (128,))])
assert BLOCK_DTYPE.itemsize == Q4_K_BLOCK_BYTES


def get_scale_min_k4(j: int, q: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(sc, m) of sub-block j from scales bytes ``q[..., 12]`` (``qw35_types.metal:70-83``)."""
    q = q.astype(np.uint32)
    if j < 4:
        sc = q[..., j] & 63
        m = q[..., j + 4] & 63
    else:
        sc = (q[..., j + 4] & 0x0F) | ((q[..., j - 4] >> 6) << 4)
        m = (q[..., j + 4] >> 4) | ((q[..., j] >> 6) << 4)
    return sc, m


def pack_scale_min_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of ``get_scale_min_k4``: (…, 8) 6-bit scales and mins -> (…, 12) bytes."""
    sc = np.asarray(sc, dtype=np.uint32)
    m = np.asarray(m, dtype=np.uint32)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint32)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (m[..., j] & 63) | ((m[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 0x0F) | ((m[..., j + 4] & 0x0F) << 4)
    return out.astype(np.uint8)


def q4_k_blocks(raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    return raw.reshape(raw.shape[0], -1).view(BLOCK_DTYPE)


def q4_k_dequant(raw: np.ndarray) -> np.ndarray:
    """Raw bytes [R, K/256*144] -> fp32 [R, K] — scalar form (``qw35_matvec.metal:2-12``)."""
    b = q4_k_blocks(raw)
    d = b["d"].astype(np.float32)
    dmin = b["dmin"].astype(np.float32)
    qs = b["qs"].astype(np.uint32)
    out = np.empty(b.shape + (256,), dtype=np.float32)
    for group in range(8):
        sc, m = get_scale_min_k4(group, b["scales"])
        base = (group // 2) * 32
        nib = qs[..., base:base + 32]
        q = (nib & 0x0F) if group % 2 == 0 else (nib >> 4)
        dsc = d * sc.astype(np.float32)
        mm = dmin * m.astype(np.float32)
        out[..., group * 32:(group + 1) * 32] = dsc[..., None] * q.astype(np.float32) - mm[..., None]
    return out.reshape(b.shape[0], -1)


def _get_scale_min_k4_pair(j: int, k: int, q: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``qw35_get_scale_min_k4_pair`` (``qw35_matvec.metal:14-18``)."""
    q = q.astype(np.uint32)
    if j < 4:
        return q[..., j + k] & 63, q[..., j + 4 + k] & 63
    return ((q[..., j + 4 + k] & 0x0F) | ((q[..., j - 4 + k] & 0xC0) >> 2),
            (q[..., j + 4 + k] >> 4) | ((q[..., j + k] & 0xC0) >> 2))


def q4_k_dequant_tiles(raw: np.ndarray) -> np.ndarray:
    """Same as ``q4_k_dequant`` through the 16-element tile form (``qw35_matvec.metal:20-38``)."""
    b = q4_k_blocks(raw)
    qs = b["qs"].astype(np.uint32)
    d0 = b["d"].astype(np.float32)
    dmin = b["dmin"].astype(np.float32)
    out = np.empty(b.shape + (256,), dtype=np.float32)
    for il_full in range(16):
        is_ = (il_full // 4) * 2
        off = (il_full // 4) * 32 + 16 * (il_full & 1)
        il = il_full & 3
        sc, m = _get_scale_min_k4_pair(is_, il // 2, b["scales"])
        d = d0 * (np.float32(1.0) if il < 2 else np.float32(1.0 / 16.0))
        dl = d * sc.astype(np.float32)
        ml = dmin * m.astype(np.float32)
        mask = np.uint32(0x0F) if il < 2 else np.uint32(0xF0)
        q = (qs[..., off:off + 16] & mask).astype(np.float32)
        out[..., il_full * 16:(il_full + 1) * 16] = dl[..., None] * q - ml[..., None]
    return out.reshape(b.shape[0], -1)


def q4_k_quantize(rows: np.ndarray) -> np.ndarray:
    """fp32 [R, K] (K % 256 == 0) -> raw Q4_K bytes [R, K/256*144]."""
    rows = np.asarray(rows, dtype=np.float32)
    r, k = rows.shape
    if k % 256:
        raise ValueError("Q4_K needs columns divisible by 256")
    nb = k // 256
    sub = rows.reshape(r, nb, 8, 32)
    lo = np.minimum(sub.min(axis=3), 0.0).astype(np.float32)
    hi = sub.max(axis=3).astype(np.float32)
    scale = ((hi - lo) / np.float32(15.0)).astype(np.float32)
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
    q = np.clip(np.rint(qf), 0, 15).astype(np.uint8)
    out = np.zeros((r, nb), dtype=BLOCK_DTYPE)
    out["d"] = d
    out["dmin"] = dmin
    out["scales"] = pack_scale_min_k4(sc, mq)
    qs = np.zeros((r, nb, 128), dtype=np.uint8)
    for c in range(4):
        qs[..., 32 * c:32 * c + 32] = q[:, :, 2 * c, :] | (q[:, :, 2 * c + 1, :] << 4)
    out["qs"] = qs
    return out.view(np.uint8).reshape(r, nb * 144)


def q4_k_nbytes(rows: int, k: int) -> int:
    return rows * ((k + 255) // 256) * 144
