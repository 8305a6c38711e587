"""fp64 matvec / matmul oracle on dequantised weights.  Test infrastructure only.

The quantity every kernel is checked against is the fp64 product of the
oracle-dequantised weights with the activations the kernel was given:

* decode GEMV (``qw35_gf4.metal:99-136``, ``qw35_matvec.metal:171-261,630-654``):
  ``y[b, r] = sum_k W[r, k] * (a[k] * x[b, k])`` (``a`` = 1 when no AWQ vector),
  ``y += ...`` for the residual variants (``qw35_gf4.metal:209-246``);
* fused gate/up/SwiGLU (``qw35_gf4.metal:62-96``):
  ``silu(gate . x) * (up . x)`` with ``silu(v) = v / (1 + exp(-v))``
  (``qw35_types.metal:40-42``);
* prefill dequant-matmul (``qw35_tiled_mm.metal:36-198``; output layout
  ``dst[token * rows + row]`` at ``:157-165``): ``C[m, n] = sum_k W[n, k] *
  (a[k] * A[m, k])`` in fp64 on the unrounded activations, which the
  reference's tiled matmul keeps in fp32 (src1 staged as float,
  ``qw35_tiled_mm.metal:200-224``).  ``prefill_f64`` is that reference.  Two
  more functions restate the activation rounding of this library's two
  prefill paths (not the reference's arithmetic), so that tests can bound the
  kernel's own accumulation error tightly: ``prefill_staged_operand`` (fp16
  staging with a per-token power of two; an fp16 hi/lo pair for fp32 input)
  and ``prefill_direct_operand`` (bf16 operands of the path without a
  workspace).
"""
from __future__ import annotations

import numpy as np

from . import gf2, gf4, q4_k, q5_k, q6_k, q8_0

TYPE_GF4 = gf4.GF4_TYPE_ID
TYPE_GF2 = gf2.GF2_TYPE_ID
TYPE_Q8_0 = q8_0.Q8_0_TYPE_ID
TYPE_Q4_K = q4_k.Q4_K_TYPE_ID
TYPE_Q5_K = q5_k.Q5_K_TYPE_ID
TYPE_Q6_K = q6_k.Q6_K_TYPE_ID
TYPE_F16 = 1


def tensor_nbytes(type_id: int, rows: int, k: int) -> int:
    """Byte size of a rows x k tensor (``qw35-server/src/loader/tensors.rs:123-172``)."""
    if type_id == TYPE_GF4:
        return gf4.gf4_nbytes(rows, k)
    if type_id == TYPE_GF2:
        return gf2.gf2_nbytes(rows, k)
    if type_id == TYPE_Q8_0:
        return q8_0.q8_0_nbytes(rows, k)
    if type_id == TYPE_Q4_K:
        return q4_k.q4_k_nbytes(rows, k)
    if type_id == TYPE_Q5_K:
        return q5_k.q5_k_nbytes(rows, k)
    if type_id == TYPE_Q6_K:
        assert k % q6_k.Q6_K_BLOCK_ELEMS == 0
        return rows * (k // q6_k.Q6_K_BLOCK_ELEMS) * q6_k.Q6_K_BLOCK_BYTES
    if type_id == TYPE_F16:
        return rows * k * 2
    raise ValueError(f"unsupported type id {type_id}")


def quantize(type_id: int, w: np.ndarray) -> np.ndarray:
    """fp32 [R, K] -> raw tensor bytes as uint8 [R, row_bytes]."""
    if type_id == TYPE_GF4:
        return gf4.gf4_pack(w).view(np.uint8).reshape(w.shape[0], -1)
    if type_id == TYPE_GF2:
        return gf2.gf2_quantize(w)
    if type_id == TYPE_Q8_0:
        return q8_0.q8_0_quantize(w)
    if type_id == TYPE_Q4_K:
        return q4_k.q4_k_quantize(w)
    if type_id == TYPE_Q5_K:
        return q5_k.q5_k_quantize(w)
    if type_id == TYPE_Q6_K:
        return q6_k.q6_k_quantize(w).reshape(w.shape[0], -1)
    if type_id == TYPE_F16:
        return np.asarray(w, dtype=np.float32).astype(np.float16).view(np.uint8).reshape(w.shape[0], -1)
    raise ValueError(f"unsupported type id {type_id}")


def dequant(type_id: int, raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Raw tensor bytes (any shape, rows*row_bytes total) -> fp32 [rows, k]."""
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(rows, -1)
    if type_id == TYPE_GF4:
        return gf4.gf4_dequant(raw.view("<u4"))
    if type_id == TYPE_GF2:
        return gf2.gf2_dequant(raw, rows, raw.size // rows // gf2.GF2_BLOCK_BYTES * gf2.GF2_BLOCK_ELEMS)
    if type_id == TYPE_Q8_0:
        return q8_0.q8_0_dequant(raw)
    if type_id == TYPE_Q4_K:
        return q4_k.q4_k_dequant(raw)
    if type_id == TYPE_Q5_K:
        return q5_k.q5_k_dequant(raw)
    if type_id == TYPE_Q6_K:
        return q6_k.q6_k_dequant(raw, rows, raw.size // rows // q6_k.Q6_K_BLOCK_BYTES * q6_k.Q6_K_BLOCK_ELEMS)
    if type_id == TYPE_F16:
        return raw.view("<f2").astype(np.float32)
    raise ValueError(f"unsupported type id {type_id}")


def matvec_f64(w: np.ndarray, x: np.ndarray, awq: np.ndarray | None = None) -> np.ndarray:
    """fp64 ``y[b] = W @ (a * x[b])`` for x of shape [K] or [B, K]."""
    w64 = np.asarray(w, dtype=np.float64)
    x64 = np.atleast_2d(np.asarray(x, dtype=np.float64))
    if awq is not None:
        x64 = x64 * np.asarray(awq, dtype=np.float64)[None, :]
    y = x64 @ w64.T
    return y if np.ndim(x) == 2 else y[0]


def silu_f64(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def swiglu_f64(w_gate, w_up, x, awq=None):
    return silu_f64(matvec_f64(w_gate, x, awq)) * matvec_f64(w_up, x, awq)


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


# -- bf16 helpers -----------------------------------------------------------

def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round-to-nearest-even (NaN kept quiet)."""
    bits = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    lsb = (bits >> np.uint32(16)) & np.uint32(1)
    rounded = (bits + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    nan = np.isnan(np.asarray(v, dtype=np.float32))
    rounded = np.where(nan, (bits >> np.uint32(16)) | np.uint32(0x40), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(v: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(v))


def prefill_input(a: np.ndarray, awq: np.ndarray | None = None) -> np.ndarray:
    """fp64 ``awq * A`` of prefill activations ``a``: bf16 bit patterns (uint16)
    or fp32 values, taken exactly."""
    a = np.asarray(a)
    a64 = (bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)).astype(np.float64)
    if awq is not None:
        a64 = a64 * np.asarray(awq, dtype=np.float32).astype(np.float64)[None, :]
    return a64


def prefill_f64(w: np.ndarray, a: np.ndarray, awq: np.ndarray | None = None) -> np.ndarray:
    """fp64 ``C[M, rows] = (awq * A) @ W^T`` on the unrounded activations (bf16
    bits or fp32 values), the reference product the prefill paths are measured against."""
    return prefill_input(a, awq) @ np.asarray(w, dtype=np.float64).T


def _f16(v: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 round-to-nearest-even (numpy's cast), back to fp32."""
    return np.asarray(v, dtype=np.float32).astype(np.float16).astype(np.float32)


def _pow2_scale(max_abs: np.ndarray) -> np.ndarray:
    """2^e with max_abs * 2^e in [2^14, 2^15), e clamped to [-124, 126]; 1 for a
    zero or non-finite maximum (the staging's power-of-two factor)."""
    out = np.ones(max_abs.shape, dtype=np.float64)
    ok = (max_abs > 0) & np.isfinite(max_abs)
    _, e = np.frexp(max_abs[ok].astype(np.float64))  # max in [2^(e-1), 2^e)
    out[ok] = np.exp2(np.clip(15 - e, -124, 126).astype(np.float64))
    return out


def prefill_staged_operand(a: np.ndarray, awq: np.ndarray | None, a_f32: bool) -> np.ndarray:
    """The activations the staged prefill path (a workspace given) contracts, in
    fp64: v = fp32(awq * A), one power of two 2^e per token row putting max |v|
    in [2^14, 2^15), hi = fp16_rne(2^e v); fp32 input adds lo =
    fp16_rne((2^e v - hi) 2^11) and contracts hi + 2^-11 lo.  The operand is
    that sum times 2^-e.  This library's own staging, restated so a test can
    separate the staging's rounding from the kernel's accumulation."""
    a = np.asarray(a)
    v = bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)
    if awq is not None:
        v = (v * np.asarray(awq, dtype=np.float32)[None, :]).astype(np.float32)
    sc = _pow2_scale(np.max(np.abs(v), axis=1))[:, None]
    s = (v.astype(np.float64) * sc).astype(np.float32)  # exact: a power of two
    hi = _f16(s).astype(np.float64)
    op = hi
    if a_f32:
        lo = _f16(((s.astype(np.float64) - hi) * 2048.0).astype(np.float32)).astype(np.float64)
        op = hi + lo / 2048.0
    return op / sc


def prefill_direct_operand(a: np.ndarray, awq: np.ndarray | None) -> np.ndarray:
    """The activations the prefill path without a workspace contracts on bf16
    MFMA: bf16_rne(fp32(awq * A)), in fp64 (this library's direct path)."""
    a = np.asarray(a)
    v = bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)
    if awq is not None:
        v = (v * np.asarray(awq, dtype=np.float32)[None, :]).astype(np.float32)
    return bf16_round(v).astype(np.float64)


def argmax_rule(logits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Greedy head reduction of the reference (``qw35_output.metal:120-182``):
    starting from (-inf, 0xFFFFFFFF), a value replaces the best when it is
    larger, or equal with a smaller row id.  So per batch row: the largest
    logit, ties to the smaller id, NaN never selected (an all-NaN row gives
    0xFFFFFFFF and -inf).  Returns (ids uint32, logits fp32) over ``logits[b, r]``."""
    lg = np.atleast_2d(np.asarray(logits, dtype=np.float32))
    ids = np.full(lg.shape[0], 0xFFFFFFFF, dtype=np.uint32)
    best = np.full(lg.shape[0], -np.inf, dtype=np.float32)
    for b in range(lg.shape[0]):
        row = lg[b]
        ok = ~np.isnan(row)
        if ok.any():
            m = row[ok].max()
            ids[b] = np.flatnonzero(ok & (row == m))[0]
            best[b] = m
    return ids, best


def prefill_image(type_id: int, raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """The fp16 prefill image of a weight: fp16_rne of the exact dequantised
    value (numpy's float32 -> float16 cast rounds to nearest even), the half
    dequantisation of the reference's tiled matmul (qw35_tiled_mm.metal:199-255)."""
    return dequant(type_id, raw, rows, k).astype(np.float16)
