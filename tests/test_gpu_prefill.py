"""GPU parity of the GF4 prefill dequant-matmul (qw35_hip_matmul_prefill).

The oracle is oracle/matvec.py:prefill_f64: an fp64 product of the exact bf16
operands the kernel contracts, A' = bf16_rne(awq * A) and the GF4 weights
(exact in bf16).  Bars: fp32 output within 1e-3 relative L2; bf16 output
within one bf16 ulp of the fp64 value per element, plus the fp32-accumulation
allowance 2^-16 * sum_k |A'_k W_k| (a few percent of an ulp at these shapes).
Full config-4 shapes are checked on a seeded sample of output rows.  Both
paths are covered: staged (workspace: fp16 activations with per-token
power-of-two scales, fp16 MFMA) and direct (bf16 MFMA).  The small shapes
take the staged path's K split (fp32 partial sums in the workspace, then an
ordered reduction), including a row count that is not a multiple of 4.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import gf4 as ogf4
from oracle import matvec as om
from tests.helpers import awq_scales, bf16_normal

pytestmark = pytest.mark.gpu

F32_REL_L2 = 1e-3


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _bf16_tensor(bits: np.ndarray, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _bf16_out_ok(got_bf16_bits: np.ndarray, want: np.ndarray, a_eff: np.ndarray, w: np.ndarray) -> tuple[bool, str]:
    got = om.bf16_bits_to_f32(got_bf16_bits).astype(np.float64)
    mag = np.abs(want)
    ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 2.0 ** -126))) - 7)
    abs_sum = np.abs(a_eff.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = ulp + abs_sum * 2.0 ** -16
    err = np.abs(got - want)
    worst = float(np.max(err / bound))
    return bool(np.all(err <= bound)), f"worst err/bound {worst:.3f}"


def _case(cuda, m, n, k, seed, awq_on, out_f32, a_f32=False, staged=True):
    import torch

    rng = np.random.default_rng(seed)
    w = bf16_normal(rng, (n, k), 0.02)
    words = ogf4.gf4_pack(w)
    wdq = ogf4.gf4_dequant(words)
    a32 = rng.standard_normal((m, k), dtype=np.float32)
    awq = awq_scales(rng, k) if awq_on else None
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    if a_f32:
        a_dev = _t(a32, cuda)
        # the kernel rounds fp32 input to bf16 after the AWQ multiply
        a_eff = om.bf16_round(a32 * (awq[None, :] if awq is not None else np.float32(1.0)))
    else:
        bits = om.f32_to_bf16_bits(a32)
        a_dev = _bf16_tensor(bits, cuda)
        a_eff = om.prefill_operand(bits, awq)
    out = _rt().matmul_prefill(hw, a_dev, awq=_t(awq, cuda) if awq is not None else None,
                               out_dtype=torch.float32 if out_f32 else torch.bfloat16, workspace=staged)
    want = a_eff.astype(np.float64) @ wdq.astype(np.float64).T
    if out_f32:
        got = out.cpu().numpy()
        assert om.rel_l2(got, want) <= F32_REL_L2
    else:
        got_bits = out.view(torch.int16).cpu().numpy().view(np.uint16)
        ok, msg = _bf16_out_ok(got_bits, want, a_eff, wdq)
        assert ok, msg


@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (9, 64, 256), (37, 100, 512), (130, 272, 1024),
                                   (50, 302, 2048), (64, 4096, 4096), (300, 520, 12288)])
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("staged", [True, False])
def test_prefill_parity(cuda, m, n, k, awq_on, out_f32, staged):
    _case(cuda, m, n, k, seed=m * 7 + n + k, awq_on=awq_on, out_f32=out_f32, staged=staged)


@pytest.mark.parametrize("m,n,k", [(5, 48, 256), (200, 384, 4096)])
def test_prefill_fp32_activations(cuda, m, n, k):
    for staged in (True, False):
        _case(cuda, m, n, k, seed=3 + m, awq_on=True, out_f32=True, a_f32=True, staged=staged)
        _case(cuda, m, n, k, seed=4 + m, awq_on=False, out_f32=False, a_f32=True, staged=staged)


def test_prefill_staged_extreme_token_scales(cuda):
    """Staging scales each token row by its own power of two: rows of very
    different magnitude (and an all-zero row) keep their relative accuracy."""
    import torch

    rng = np.random.default_rng(31)
    n, k, m = 96, 1024, 6
    words = ogf4.gf4_pack(bf16_normal(rng, (n, k), 0.02))
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    a32 = rng.standard_normal((m, k), dtype=np.float32) * np.array([1e-6, 1.0, 3e4, 0.0, 1e-3, 2.5e8],
                                                                    np.float32)[:, None]
    bits = om.f32_to_bf16_bits(a32)
    out = _rt().matmul_prefill(hw, _bf16_tensor(bits, cuda), out_dtype=torch.float32).cpu().numpy()
    want = om.prefill_f64(ogf4.gf4_dequant(words), bits)
    for r in range(m):
        if r == 3:
            assert np.all(out[r] == 0.0)
        else:
            assert om.rel_l2(out[r], want[r]) <= 1e-6, r


def test_prefill_workspace_validation(cuda):
    import torch

    rng = np.random.default_rng(2)
    words = ogf4.gf4_pack(bf16_normal(rng, (32, 256), 0.02))
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, 32, 256)
    a = torch.zeros((4, 256), dtype=torch.bfloat16, device=cuda)
    small = torch.empty(64, dtype=torch.uint8, device=cuda)
    with pytest.raises(_rt().Qw35Error, match="workspace"):
        _rt().matmul_prefill(hw, a, workspace=small)


def test_prefill_prefix_equals_shorter_chunk(cuda):
    """Rows of C depend only on their own token: a chunk's first rows equal a
    shorter chunk's.  Bit for bit on the direct path (every tile shape sums k
    in the same order); the staged path may split K differently for the two
    token counts, which only changes fp32 rounding of the partial sums."""
    import torch

    rng = np.random.default_rng(12)
    n, k = 1024, 4096
    words = ogf4.gf4_pack(bf16_normal(rng, (n, k), 0.02))
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    a = _bf16_tensor(om.f32_to_bf16_bits(rng.standard_normal((700, k), dtype=np.float32)), cuda)
    long = _rt().matmul_prefill(hw, a, out_dtype=torch.float32, workspace=None)
    short = _rt().matmul_prefill(hw, a[:33].contiguous(), out_dtype=torch.float32, workspace=None)
    assert torch.equal(long[:33], short)
    long = _rt().matmul_prefill(hw, a, out_dtype=torch.float32).cpu().numpy()
    short = _rt().matmul_prefill(hw, a[:33].contiguous(), out_dtype=torch.float32).cpu().numpy()
    assert om.rel_l2(long[:33], short) <= 1e-6


@pytest.mark.parametrize("m", [128, 512, 2048])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_prefill_config4_shapes(cuda, m, n, k):
    """Config 4: W = GF4(bf16 N(0,0.02)) made by the GPU packer, A bf16 N(0,1),
    AWQ U(0.5,2), bf16 out; 48 sampled token rows against the oracle."""
    import torch

    rt = _rt()
    g = torch.Generator(device=cuda)
    g.manual_seed(m + n)
    w32 = (torch.randn((n, k), generator=g, device=cuda) * 0.02).to(torch.bfloat16).float()
    hw = rt.quantize_weight(w32, om.TYPE_GF4)
    del w32
    a = torch.randn((m, k), generator=g, device=cuda).to(torch.bfloat16)
    awq = torch.rand((k,), generator=g, device=cuda) * 1.5 + 0.5
    out = rt.matmul_prefill(hw, a, awq=awq)
    direct = rt.matmul_prefill(hw, a, awq=awq, workspace=None)
    rows = np.sort(np.random.default_rng(m).choice(m, size=min(48, m), replace=False))
    words = hw.storage.cpu().numpy().view("<u4").reshape(n, k // 8)
    wdq = ogf4.gf4_dequant(words)
    a_bits = a.view(torch.int16).cpu().numpy().view(np.uint16)[rows]
    a_eff = om.prefill_operand(a_bits, awq.cpu().numpy())
    want = a_eff.astype(np.float64) @ wdq.astype(np.float64).T
    for res in (out, direct):
        got_bits = res.view(torch.int16).cpu().numpy().view(np.uint16)[rows]
        ok, msg = _bf16_out_ok(got_bits, want, a_eff, wdq)
        assert ok, msg


@pytest.mark.parametrize("m,n,k", [(128, 8192, 4096), (100, 4096, 4096), (128, 6000, 4096), (64, 12288, 4096),
                                   (128, 12288, 4096), (128, 8192, 1024)])
@pytest.mark.parametrize("out_f32", [False, True])
def test_prefill_k_quarters(cuda, m, n, k, out_f32):
    """Shapes the planner gives four in-block K parts (64-token tiles, k <= 4096,
    one block per CU or fewer): 8 waves over 64 rows, or 16 over 128 rows
    (12288 rows at M = 128); ragged tokens (100) and rows (6000); quarters of
    256 columns (k = 1024).  GPU-packed GF4 weights, AWQ; 32 sampled token rows
    against the oracle, to the same bars as every prefill output."""
    import torch

    rt = _rt()
    g = torch.Generator(device=cuda)
    g.manual_seed(m + n + k)
    w32 = (torch.randn((n, k), generator=g, device=cuda) * 0.02).to(torch.bfloat16).float()
    hw = rt.quantize_weight(w32, om.TYPE_GF4)
    del w32
    a = torch.randn((m, k), generator=g, device=cuda).to(torch.bfloat16)
    awq = torch.rand((k,), generator=g, device=cuda) * 1.5 + 0.5
    out = rt.matmul_prefill(hw, a, awq=awq, out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    rows = np.sort(np.random.default_rng(n + m).choice(m, size=32, replace=False))
    words = hw.storage.cpu().numpy().view("<u4").reshape(n, k // 8)
    wdq = ogf4.gf4_dequant(words)
    a_eff = om.prefill_operand(a.view(torch.int16).cpu().numpy().view(np.uint16)[rows], awq.cpu().numpy())
    want = a_eff.astype(np.float64) @ wdq.astype(np.float64).T
    if out_f32:
        got = out.cpu().numpy()[rows].astype(np.float64)
        assert om.rel_l2(got, want) <= F32_REL_L2
        assert np.all(np.abs(got - want) <= (np.abs(a_eff) @ np.abs(wdq).T) * 2.0 ** -16 + 1e-30)
    else:
        got_bits = out.view(torch.int16).cpu().numpy().view(np.uint16)[rows]
        ok, msg = _bf16_out_ok(got_bits, want, a_eff, wdq)
        assert ok, msg


@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_prefill_workspace_without_room_for_a_split(cuda, n, k):
    """A workspace of only the staging bytes (room for no K split) runs the
    planned tiles unsplit, the two in-block K halves included; the result
    matches the planned call within fp32 rounding and the oracle on sampled
    rows."""
    import torch

    rt = _rt()
    m = 128
    g = torch.Generator(device=cuda)
    g.manual_seed(n + 3)
    w32 = (torch.randn((n, k), generator=g, device=cuda) * 0.02).to(torch.bfloat16).float()
    hw = rt.quantize_weight(w32, om.TYPE_GF4)
    del w32
    a = torch.randn((m, k), generator=g, device=cuda).to(torch.bfloat16)
    staged_only = (m * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256
    small = torch.empty(staged_only, dtype=torch.uint8, device=cuda)
    out = rt.matmul_prefill(hw, a, out_dtype=torch.float32, workspace=small).cpu().numpy().astype(np.float64)
    planned = rt.matmul_prefill(hw, a, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    assert om.rel_l2(out, planned) <= 1e-6
    rows = np.sort(np.random.default_rng(n).choice(m, size=32, replace=False))
    words = hw.storage.cpu().numpy().view("<u4").reshape(n, k // 8)
    wdq = ogf4.gf4_dequant(words).astype(np.float64)
    a_eff = om.prefill_operand(a.view(torch.int16).cpu().numpy().view(np.uint16)[rows], None).astype(np.float64)
    want = a_eff @ wdq.T
    assert om.rel_l2(out[rows], want) <= F32_REL_L2
    assert np.all(np.abs(out[rows] - want) <= (np.abs(a_eff) @ np.abs(wdq).T) * 2.0 ** -16 + 1e-30)


def test_matvec_batch_long_chunk_uses_prefill(cuda):
    """encodeMatvecBatch semantics: > 8 fp32 tokens on a GF4 weight -> fp32 [tokens, rows]."""
    rng = np.random.default_rng(2)
    n, k, m = 256, 4096, 12
    words = ogf4.gf4_pack(bf16_normal(rng, (n, k), 0.02))
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    y = _rt().matvec_batch(hw, _t(x, cuda)).cpu().numpy()
    want = om.bf16_round(x).astype(np.float64) @ ogf4.gf4_dequant(words).astype(np.float64).T
    assert y.shape == (m, n) and om.rel_l2(y, want) <= F32_REL_L2
