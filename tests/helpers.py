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


def random_kq_bytes(rng: np.random.Generator, type_id: int, rows: int, k: int) -> np.ndarray:
    """Arbitrary Q4_K / Q5_K bytes (every nibble, high bit and 6-bit scale/min
    pattern) with d and dmin drawn from fp16 values, negative and subnormal ones
    included, that keep every dequantised weight inside fp16's range
    (|d| * 63 * 31 < 65504).  Mixed magnitudes of d * sc * q and dmin * m make
    the fp32 rounding of the weight inexact, which separates fp16(fl32(w))
    from a single rounding of w straight to fp16."""
    bb = {om.TYPE_Q4_K: 144, om.TYPE_Q5_K: 176}[type_id]
    raw = rng.integers(0, 256, size=(rows, k // 256, bb), dtype=np.uint8)
    pick = np.array([2.0 ** -24, 2.0 ** -14, 2.0 ** -10, 0.013, -0.5, 1.0, 3.5, -30.0], np.float16)
    for off in (0, 2):
        raw[:, :, off:off + 2] = rng.choice(pick, size=(rows, k // 256)).view(np.uint8).reshape(rows, k // 256, 2)
    return raw.reshape(-1)


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


def prefill_rel_l2_bar(a_f32: bool, awq_on: bool) -> float:
    """rel-L2 bar of a prefill's fp32 output against oracle.matvec.prefill_f64
    (unrounded activations) on the weights the kernel contracts: 1e-5 where the
    staged operand carries the activations exactly (bf16 without AWQ) or to
    ~22 bits (fp32 as an fp16 hi/lo pair); 4e-4 for bf16 with AWQ (the product
    rounded once to fp16)."""
    return 4e-4 if (awq_on and not a_f32) else 1e-5


def bf16_out_ok(got_bf16_bits: np.ndarray, want: np.ndarray, a_eff: np.ndarray, w: np.ndarray) -> tuple[bool, str]:
    """bf16 output within one bf16 ulp of the fp64 value plus the
    fp32-accumulation allowance 2^-16 * sum_k |A'_k W_k|, per element."""
    got = om.bf16_bits_to_f32(got_bf16_bits).astype(np.float64)
    mag = np.abs(want)
    ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 2.0 ** -126))) - 7)
    abs_sum = np.abs(a_eff.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = ulp + abs_sum * 2.0 ** -16
    err = np.abs(got - want)
    worst = float(np.max(err / bound))
    return bool(np.all(err <= bound)), f"worst err/bound {worst:.3f}"


def check_prefill(out, a_host: np.ndarray, awq: np.ndarray | None, w_op: np.ndarray, staged: bool = True,
                  w_exact: np.ndarray | None = None) -> float:
    """Bars on a prefill result.  ``out``: the device result (token rows
    matching ``a_host``); ``a_host``: bf16 bit patterns (uint16) or fp32
    activations; ``w_op``: the weights the kernel contracts (exact GF4
    dequantisation, or the fp16 image of a q8_0 / k-quant weight);
    ``w_exact``: the exact dequantisation when ``w_op`` is an fp16 image.

    * accumulation: against the fp64 product of the operand the path contracts
      (prefill_staged_operand / prefill_direct_operand): fp32 output within
      2^-16 * sum_k |A'_k W_k| per element, bf16 output within one ulp more;
    * fp32 output: rel-L2 against prefill_f64 on the unrounded activations
      within prefill_rel_l2_bar, and against the exact weights within 1e-3.

    Returns the rel-L2 against prefill_f64 on ``w_exact`` (else ``w_op``), or 0
    for bf16 output."""
    import torch

    a_f32 = a_host.dtype == np.float32
    w64 = np.asarray(w_op).astype(np.float64)
    op = om.prefill_staged_operand(a_host, awq, a_f32) if staged else om.prefill_direct_operand(a_host, awq)
    want_op = op @ w64.T
    if out.dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        bound = (np.abs(op) @ np.abs(w64).T) * 2.0 ** -16 + 1e-30
        worst = float(np.max(np.abs(got - want_op) / bound))
        assert worst <= 1.0, f"accumulation: worst err/bound {worst:.3f}"
        err = om.rel_l2(got, om.prefill_f64(w64, a_host, awq))
        assert err <= prefill_rel_l2_bar(a_f32, awq is not None), f"rel-L2 {err:.3e} against the unrounded product"
        if w_exact is not None:
            err = om.rel_l2(got, om.prefill_f64(w_exact, a_host, awq))
            assert err <= GEMV_REL_L2, f"rel-L2 {err:.3e} against the exact weights"
        return err
    got_bits = out.view(torch.int16).cpu().numpy().view(np.uint16)
    ok, msg = bf16_out_ok(got_bits, want_op, op, w64)
    assert ok, msg
    return 0.0


def pinned_rows(rows: int, edge: int = 1024, stride: int = 61) -> np.ndarray:
    """Rows of a large weight whose dequantisation is pinned to the oracle: the
    first and last ``edge`` rows and every ``stride``-th row."""
    return np.unique(np.concatenate([np.arange(min(edge, rows)), np.arange(max(0, rows - edge), rows),
                                     np.arange(0, rows, stride)])).astype(np.int64)


def assert_dequant_pinned(w, rows: np.ndarray) -> None:
    """The library's dequantisation of rows ``rows`` of the device weight ``w``
    (qw35_hip_dequantize with a row gather) equals, bit for bit, the oracle's
    dequantisation of the same rows' bytes."""
    import torch

    from qwowl35_amd import runtime as rt

    dev = w.storage.device
    ids = torch.from_numpy(rows.astype(np.int32)).to(dev)
    got = rt.dequantize(w, ids).cpu().numpy()
    rb = rt.row_bytes(w.type_id, w.k)
    raw = w.storage[: w.rows * rb].view(w.rows, rb)[ids.long()].cpu().numpy().reshape(-1)
    want = om.dequant(w.type_id, raw, len(rows), w.k)
    bad = np.flatnonzero(np.any(got.view(np.uint32) != want.view(np.uint32), axis=1))
    assert bad.size == 0, f"rows {rows[bad[:8]].tolist()} differ from the oracle"
