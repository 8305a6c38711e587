"""ggml Q6_K codec — numpy restatement.  Test infrastructure only.

Super-block of 256 weights = 210 bytes (``qw35_block_q6_k``,
``qw35-server/src/metal/qw35_types.metal:17-22``):

* ``ql[128]``     — low 4 bits of each 6-bit code,
* ``qh[64]``      — high 2 bits of each code,
* ``scales[16]``  — signed 8-bit scale of each 16-weight sub-block,
* ``d``           — little-endian binary16 super-scale.

Element ``e = 128*h + 32*g + l`` (``h`` in 0..1, ``g`` in 0..3, ``l`` in 0..31)
takes its low nibble from ``ql[64*h + 32*(g & 1) + l]`` (low nibble for
``g < 2``, high nibble otherwise) and its high bits from bits ``2g..2g+1`` of
``qh[32*h + l]``; its sub-block is ``e // 16`` and its weight is
``d * scales[e // 16] * (q - 32)``.  ``d * sc`` (11 x 8 significant bits) and
its product with ``q - 32`` (6 bits) are exact in fp32, so the weight is the
exact value — what ggml's C ``dequantize_row_q6_K`` and gguf-py compute.

Three restatements are kept on purpose:

* ``q6_k_dequant`` — the element mapping above, vectorised;
* ``q6_k_dequant_gemv_form`` — the bit extraction of the reference's Q6_K
  GEMV and argmax-head kernels (``qw35_matvec.metal:458-542``,
  ``qw35_output.metal:2-80``: ``y_offset``/``q_offset_l``/``q_offset_h``
  indexing, ``kmask1..4``), which must agree bit-for-bit with the first;
* ``q6_k_dequant_tile_form`` — the reference's tile dequantiser
  ``qw35_dequantize_q6_k`` (``qw35_matvec.metal:65-98``), which rounds
  ``(d*sc) * q_unsigned`` before subtracting ``32*d*sc``: it equals the exact
  value whenever that product is exact and is otherwise within one rounding.

The encoder is this build's own (the reference only reads Q6_K through gguf-py
and the Metal kernels): per 16-weight sub-block a symmetric scale, then 8-bit
quantisation of the sub-scales against ``d``.
"""
from __future__ import annotations

import numpy as np

Q6_K_TYPE_ID = 14
Q6_K_BLOCK_ELEMS = 256
Q6_K_BLOCK_BYTES = 210

BLOCK_DTYPE = np.dtype([("ql", "u1", (128,)), ("qh", "u1", (64,)), ("scales", "i1", (16,)), ("d", "<f2")])
assert BLOCK_DTYPE.itemsize == Q6_K_BLOCK_BYTES


def _element_index() -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """For element e of a super-block: (ql byte, nibble shift, qh byte, qh shift)."""
    e = np.arange(256)
    h, g, l = e // 128, (e % 128) // 32, e % 32
    ql_idx = 64 * h + 32 * (g & 1) + l
    ql_shift = 4 * (g >> 1)
    qh_idx = 32 * h + l
    qh_shift = 2 * g
    return ql_idx, ql_shift, qh_idx, qh_shift


_QL_IDX, _QL_SHIFT, _QH_IDX, _QH_SHIFT = _element_index()


def as_blocks(raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    assert raw.size % Q6_K_BLOCK_BYTES == 0
    return raw.view(BLOCK_DTYPE)


def q6_k_codes(blocks: np.ndarray) -> np.ndarray:
    """Unsigned 6-bit codes (…, 256) of the super-blocks."""
    ql = blocks["ql"].astype(np.uint32)
    qh = blocks["qh"].astype(np.uint32)
    lo = (ql[..., _QL_IDX] >> _QL_SHIFT) & 0x0F
    hi = (qh[..., _QH_IDX] >> _QH_SHIFT) & 0x03
    return (lo | (hi << 4)).astype(np.int32)


def q6_k_dequant(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """fp32 [rows][k] from raw tensor bytes (exact: d * sc * (q - 32))."""
    assert k % Q6_K_BLOCK_ELEMS == 0
    blocks = as_blocks(raw).reshape(rows, k // Q6_K_BLOCK_ELEMS)
    q = q6_k_codes(blocks) - 32                                   # (rows, nb, 256)
    dsc = blocks["d"].astype(np.float32)[..., None] * blocks["scales"].astype(np.float32)  # exact
    w = np.repeat(dsc, 16, axis=-1) * q.astype(np.float32)         # exact
    return w.reshape(rows, k).astype(np.float32)


def q6_k_dequant_gemv_form(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Scalar statement following the reference GEMV's byte/bit extraction
    (qw35_matvec.metal:458-542): lane ``tid`` (ip = tid // 8, il = tid % 8,
    l0 = 4*il) covers elements y_offset + {l, l+32, l+64, l+96}, l in l0..l0+3,
    with scales sc[is + {0, 2, 4, 6}], is = 8*ip + l0 // 16."""
    blocks = as_blocks(raw).reshape(rows, k // Q6_K_BLOCK_ELEMS)
    out = np.zeros((rows, k), dtype=np.float32)
    for r in range(rows):
        for b in range(k // Q6_K_BLOCK_ELEMS):
            blk = blocks[r, b]
            ql = blk["ql"].astype(np.int64)
            qh = blk["qh"].astype(np.int64)
            sc = blk["scales"].astype(np.int64)
            d = np.float32(blk["d"])
            for tid in range(16):
                ip, il = tid // 8, tid % 8
                l0 = 4 * il
                is_ = 8 * ip + l0 // 16
                y_off = 128 * ip + l0
                ql_off = 64 * ip + l0
                qh_off = 32 * ip + l0
                for l in range(4):
                    q1 = ql[ql_off + l]
                    q2 = ql[ql_off + 32 + l]
                    h = qh[qh_off + l]
                    vals = (
                        ((q1 & 0x0F) | ((h & 0x03) << 4)) - 32,
                        ((q2 & 0x0F) | ((h & 0x0C) << 2)) - 32,
                        ((q1 >> 4) | (h & 0x30)) - 32,
                        ((q2 >> 4) | ((h & 0xC0) >> 2)) - 32,
                    )
                    for j, v in enumerate(vals):
                        dsc = np.float32(d * np.float32(sc[is_ + 2 * j]))
                        out[r, b * 256 + y_off + 32 * j + l] = np.float32(dsc * np.float32(v))
    return out


def q6_k_dequant_tile_form(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """The reference tile dequantiser qw35_dequantize_q6_k (qw35_matvec.metal:65-98):
    sub-block il (16 weights) -> fl(fl(dl0 * q_unsigned) - ml), dl0 = d * sc[il],
    ml = 32 * dl0."""
    blocks = as_blocks(raw).reshape(rows, k // Q6_K_BLOCK_ELEMS)
    qu = q6_k_codes(blocks).astype(np.float32)                    # (rows, nb, 256)
    dl0 = blocks["d"].astype(np.float32)[..., None] * blocks["scales"].astype(np.float32)
    dl0 = np.repeat(dl0, 16, axis=-1).astype(np.float32)
    ml = (dl0 * np.float32(32.0)).astype(np.float32)
    return ((dl0 * qu).astype(np.float32) - ml).astype(np.float32).reshape(rows, k)


def q6_k_quantize(x: np.ndarray) -> np.ndarray:
    """fp32 [rows][k] -> raw bytes (this build's encoder; any valid block works).

    Every step is one IEEE fp32 (or binary16) operation, so the library's GPU
    encoder reproduces it bit for bit:
      amax_s = max |x| over sub-block s (16 weights),  sub_s = amax_s / 31
      d      = fp16_rne(max_s sub_s / 127)
      sc_s   = clip(rint(sub_s / d), 0, 127)             (0 when d == 0)
      q      = clip(rint(x / (d * sc_s)), -32, 31) + 32   (32 when d * sc_s == 0)
    """
    x = np.asarray(x, dtype=np.float32)
    rows, k = x.shape
    assert k % Q6_K_BLOCK_ELEMS == 0
    nb = k // Q6_K_BLOCK_ELEMS
    xb = x.reshape(rows, nb, 16, 16)
    amax = np.abs(xb).max(axis=-1)                                            # (rows, nb, 16)
    sub = (amax / np.float32(31.0)).astype(np.float32)
    d16 = (sub.max(axis=-1) / np.float32(127.0)).astype(np.float32).astype(np.float16)
    d = d16.astype(np.float32)[..., None]
    sc = np.zeros_like(sub)
    np.divide(sub, d, out=sc, where=d != 0)
    sc = np.clip(np.rint(sc), 0, 127).astype(np.int8)
    step = (d * sc.astype(np.float32)).astype(np.float32)                     # exact
    qf = np.zeros_like(xb)
    np.divide(xb, step[..., None], out=qf, where=step[..., None] != 0)
    q = (np.clip(np.rint(qf), -32, 31) + 32).astype(np.uint32).reshape(rows, nb, 256)
    blocks = np.zeros((rows, nb), dtype=BLOCK_DTYPE)
    ql = np.zeros((rows, nb, 128), dtype=np.uint32)
    qh = np.zeros((rows, nb, 64), dtype=np.uint32)
    np.bitwise_or.at(ql, (slice(None), slice(None), _QL_IDX), (q & 0x0F) << _QL_SHIFT)
    np.bitwise_or.at(qh, (slice(None), slice(None), _QH_IDX), (q >> 4) << _QH_SHIFT)
    blocks["ql"] = ql.astype(np.uint8)
    blocks["qh"] = qh.astype(np.uint8)
    blocks["scales"] = sc
    blocks["d"] = d16
    return blocks.reshape(-1).view(np.uint8)


def make_block(ql: np.ndarray, qh: np.ndarray, scales: np.ndarray, d: float) -> np.ndarray:
    """One raw super-block from its fields (tests build known-answer blocks with it)."""
    b = np.zeros(1, dtype=BLOCK_DTYPE)
    b["ql"] = np.asarray(ql, dtype=np.uint8)
    b["qh"] = np.asarray(qh, dtype=np.uint8)
    b["scales"] = np.asarray(scales, dtype=np.int8)
    b["d"] = np.float16(d)
    return b.view(np.uint8)
