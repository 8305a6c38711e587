"""ggml q8_0 codec — numpy restatement.  Test infrastructure only.

Block of 32 weights = 34 bytes: little-endian binary16 ``d`` followed by 32
int8 ``qs`` (``qw35_types.metal:24-27``; ``tensor_nbytes(8, n)`` =
``(32, 34)`` at ``qw35-server/src/loader/tensors.rs:142``).  A row of ``k``
columns is ``k/32`` consecutive blocks.  Dequantisation is ``fp32(d) * qs[j]``
(``qw35_matvec.metal:136-149``, ``:630-654``) — exact in fp32.

The encoder is this build's own (the reference only reads q8_0 through the
external gguf-py); it follows ggml's reference quantiser: ``d = max|x| / 127``,
``q = round_half_away(x / d)``.  Any valid encoding serves the parity tests,
which check decoding and matvec, not the encoder.
"""
from __future__ import annotations

import numpy as np

Q8_0_TYPE_ID = 8
Q8_0_BLOCK_ELEMS = 32
Q8_0_BLOCK_BYTES = 34

BLOCK_DTYPE = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])
assert BLOCK_DTYPE.itemsize == Q8_0_BLOCK_BYTES


def q8_0_quantize(rows: np.ndarray) -> np.ndarray:
    """fp32 [R, K] (K % 32 == 0) -> raw bytes [R, K/32*34] (uint8)."""
    rows = np.asarray(rows, dtype=np.float32)
    r, k = rows.shape
    if k % 32:
        raise ValueError("q8_0 needs columns divisible by 32")
    blocks = rows.reshape(r, k // 32, 32)
    amax = np.abs(blocks).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.zeros_like(d)
    np.divide(np.float32(1.0), d, out=inv, where=d != 0)
    scaled = blocks * inv[..., None]
    q = np.clip(np.trunc(scaled + np.copysign(np.float32(0.5), scaled)), -127, 127).astype(np.int8)
    out = np.empty((r, k // 32), dtype=BLOCK_DTYPE)
    out["d"] = d.astype(np.float16)
    out["qs"] = q
    return out.view(np.uint8).reshape(r, (k // 32) * 34)


def q8_0_blocks(raw: np.ndarray) -> np.ndarray:
    """Raw row bytes [R, nbytes] -> structured blocks [R, K/32]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    return raw.reshape(raw.shape[0], -1).view(BLOCK_DTYPE)


def q8_0_dequant(raw: np.ndarray) -> np.ndarray:
    """Raw bytes [R, K/32*34] -> fp32 weights [R, K]: ``fp32(d) * qs``."""
    b = q8_0_blocks(raw)
    d = b["d"].astype(np.float32)
    w = d[..., None] * b["qs"].astype(np.float32)
    return w.reshape(b.shape[0], -1)


def q8_0_nbytes(rows: int, k: int) -> int:
    return rows * ((k + 31) // 32) * 34
