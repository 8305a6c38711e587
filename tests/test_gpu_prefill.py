"""GPU parity of the GF4 prefill dequant-matmul (qw35_hip_matmul_prefill).

Two bars on every output:

* against the reference product, oracle/matvec.py:prefill_f64: fp64
  (awq * A) @ W^T on the unrounded activations, which the reference's tiled
  matmul keeps in fp32 (qw35-server/src/metal/qw35_tiled_mm.metal:200-224).
  fp32 output within REL_L2[case] relative L2: 1e-5 where the staged operand
  carries the activations exactly or to ~22 bits (bf16 input without AWQ;
  fp32 input as an fp16 hi/lo pair), 4e-4 for bf16 input with AWQ (the
  product rounded once to fp16), all under the 1e-3 bar;
* the kernel's own accumulation: against the fp64 product of the operand the
  path contracts (prefill_staged_operand / prefill_direct_operand), fp32
  output within the fp32-accumulation allowance 2^-16 * sum_k |A'_k W_k| per
  element; bf16 output within one bf16 ulp plus that allowance.

Both paths are covered: staged (workspace: fp16 activations with per-token
power-of-two scales, fp16 MFMA) and direct (no workspace, bf16 MFMA, bf16
activations without AWQ only).  The small shapes take the staged path's K
split (fp32 partial sums in the workspace, then an ordered reduction),
including a row count that is not a multiple of 4.  Full config-4 shapes are
checked on a seeded sample of token rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import gf4 as ogf4
from oracle import matvec as om
from tests.helpers import awq_scales, bf16_normal, check_prefill

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _bf16_tensor(bits: np.ndarray, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _case(cuda, m, n, k, seed, awq_on, out_f32, a_f32=False, staged=True):
    import torch

    rng = np.random.default_rng(seed)
    w = bf16_normal(rng, (n, k), 0.02)
    words = ogf4.gf4_pack(w)
    wdq = ogf4.gf4_dequant(words)
    a32 = rng.standard_normal((m, k), dtype=np.float32)
    awq = awq_scales(rng, k) if awq_on else None
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    a_host = a32 if a_f32 else om.f32_to_bf16_bits(a32)
    a_dev = _t(a32, cuda) if a_f32 else _bf16_tensor(a_host, cuda)
    out = _rt().matmul_prefill(hw, a_dev, awq=_t(awq, cuda) if awq is not None else None,
                               out_dtype=torch.float32 if out_f32 else torch.bfloat16, workspace=staged)
    check_prefill(out, a_host, awq, wdq, staged)


SHAPES = [(1, 16, 256), (9, 64, 256), (37, 100, 512), (130, 272, 1024), (50, 302, 2048), (64, 4096, 4096),
          (300, 520, 12288)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [False, True])
def test_prefill_parity_staged(cuda, m, n, k, awq_on, out_f32):
    _case(cuda, m, n, k, seed=m * 7 + n + k, awq_on=awq_on, out_f32=out_f32, staged=True)


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("out_f32", [False, True])
def test_prefill_parity_direct(cuda, m, n, k, out_f32):
    _case(cuda, m, n, k, seed=m * 7 + n + k, awq_on=False, out_f32=out_f32, staged=False)


@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (5, 48, 256), (9, 64, 256), (37, 100, 512), (130, 272, 1024),
                                   (200, 384, 4096), (300, 520, 12288)])
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [False, True])
def test_prefill_fp32_activations(cuda, m, n, k, awq_on, out_f32):
    """fp32 activations keep fp32 precision (staged as an fp16 hi/lo pair):
    within 1e-5 of the fp64 product of the unrounded activations."""
    _case(cuda, m, n, k, seed=3 + m + k, awq_on=awq_on, out_f32=out_f32, a_f32=True, staged=True)


def test_prefill_direct_refuses_rounded_operands(cuda):
    """The path without a workspace contracts bf16 operands: fp32 activations or
    an AWQ product would be rounded to 8 bits, so it takes neither."""
    import torch

    rng = np.random.default_rng(5)
    words = ogf4.gf4_pack(bf16_normal(rng, (32, 256), 0.02))
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, 32, 256)
    with pytest.raises(_rt().Qw35Error, match="workspace"):
        _rt().matmul_prefill(hw, torch.zeros((4, 256), dtype=torch.float32, device=cuda), workspace=None)
    with pytest.raises(_rt().Qw35Error, match="workspace"):
        _rt().matmul_prefill(hw, torch.zeros((4, 256), dtype=torch.bfloat16, device=cuda),
                             awq=torch.ones(256, device=cuda), workspace=None)


def test_prefill_staged_extreme_token_scales(cuda):
    """Staging scales each token row by its own power of two: rows of very
    different magnitude (and an all-zero row) keep their relative accuracy,
    for bf16 and fp32 activations."""
    import torch

    rng = np.random.default_rng(31)
    n, k, m = 96, 1024, 6
    words = ogf4.gf4_pack(bf16_normal(rng, (n, k), 0.02))
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    a32 = rng.standard_normal((m, k), dtype=np.float32) * np.array([1e-6, 1.0, 3e4, 0.0, 1e-3, 2.5e8],
                                                                    np.float32)[:, None]
    bits = om.f32_to_bf16_bits(a32)
    wdq = ogf4.gf4_dequant(words)
    for a_host, a_dev in ((bits, _bf16_tensor(bits, cuda)), (a32, _t(a32, cuda))):
        out = _rt().matmul_prefill(hw, a_dev, out_dtype=torch.float32).cpu().numpy()
        want = om.prefill_f64(wdq, a_host)
        for r in range(m):
            if r == 3:
                assert np.all(out[r] == 0.0)
            else:
                assert om.rel_l2(out[r], want[r]) <= 1e-5, r


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


def _gpu_gf4(rt, cuda, n, k, seed):
    """GF4(bf16 N(0, 0.02)) packed by the GPU packer, and its oracle dequantisation."""
    import torch

    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    w32 = (torch.randn((n, k), generator=g, device=cuda) * 0.02).to(torch.bfloat16).float()
    hw = rt.quantize_weight(w32, om.TYPE_GF4)
    del w32
    words = hw.storage.cpu().numpy().view("<u4").reshape(n, k // 8)
    return hw, ogf4.gf4_dequant(words), g


@pytest.mark.parametrize("m", [128, 512, 2048])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_prefill_config4_shapes(cuda, m, n, k):
    """Config 4: W = GF4(bf16 N(0,0.02)) made by the GPU packer, A bf16 N(0,1),
    AWQ U(0.5,2), bf16 out (staged) and fp32 out; the direct path on the same
    activations without AWQ; 48 sampled token rows against the oracle."""
    import torch

    rt = _rt()
    hw, wdq, g = _gpu_gf4(rt, cuda, n, k, m + n)
    a = torch.randn((m, k), generator=g, device=cuda).to(torch.bfloat16)
    awq = torch.rand((k,), generator=g, device=cuda) * 1.5 + 0.5
    rows = np.sort(np.random.default_rng(m).choice(m, size=min(48, m), replace=False))
    a_bits = a.view(torch.int16).cpu().numpy().view(np.uint16)[rows]
    awq_h = awq.cpu().numpy()
    check_prefill(rt.matmul_prefill(hw, a, awq=awq)[rows], a_bits, awq_h, wdq)
    check_prefill(rt.matmul_prefill(hw, a, awq=awq, out_dtype=torch.float32)[rows], a_bits, awq_h, wdq)
    check_prefill(rt.matmul_prefill(hw, a, workspace=None)[rows], a_bits, None, wdq, staged=False)


@pytest.mark.parametrize("m", [9, 128, 512, 2048])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_prefill_fp32_activations_full_shapes(cuda, m, n, k):
    """fp32 activations N(0,1) with AWQ U(0.5,2) at the 9B projection shapes,
    fp32 out: sampled token rows within 1e-5 relative L2 of the fp64 product
    of the unrounded activations (the reference keeps src1 in fp32,
    qw35_tiled_mm.metal:200-224), and within the accumulation bound of the
    staged hi/lo operand."""
    import torch

    rt = _rt()
    hw, wdq, g = _gpu_gf4(rt, cuda, n, k, 7 * m + n)
    a = torch.randn((m, k), generator=g, device=cuda)
    awq = torch.rand((k,), generator=g, device=cuda) * 1.5 + 0.5
    out = rt.matmul_prefill(hw, a, awq=awq, out_dtype=torch.float32)
    rows = np.sort(np.random.default_rng(m + 1).choice(m, size=min(32, m), replace=False))
    err = check_prefill(out[rows], a.cpu().numpy()[rows], awq.cpu().numpy(), wdq)
    print(f"fp32 activations {n}x{k} M={m}: rel-L2 {err:.2e}")


@pytest.mark.parametrize("m,n,k,waves", [(128, 8192, 4096, 8), (100, 4096, 4096, 8), (128, 6000, 4096, 8),
                                         (64, 12288, 4096, 8), (128, 12288, 4096, 12), (100, 11900, 4096, 12),
                                         (128, 16384, 4096, 16), (128, 8192, 1024, 8)])
@pytest.mark.parametrize("out_f32", [False, True])
def test_prefill_k_quarters(cuda, m, n, k, waves, out_f32):
    """Shapes the planner gives four in-block K parts (64-token tiles, k <= 4096,
    one block per CU or fewer): 8 waves over 64 rows, 12 over 96 (12288 rows at
    M = 128; 11900 rows end in a partial tile) or 16 over 128 (16384 rows);
    ragged tokens (100) and rows (6000); quarters of 256 columns (k = 1024).
    GPU-packed GF4 weights, AWQ; 32 sampled token rows against the oracle, to
    the same bars as every prefill output.  fp32 activations of half the
    tokens stage two rows per token and take the same quarters."""
    import torch

    rt = _rt()
    hw, wdq, g = _gpu_gf4(rt, cuda, n, k, m + n + k)
    c_dt = torch.float32 if out_f32 else torch.bfloat16
    for tokens, a_dt in ((m, torch.bfloat16), (m // 2, torch.float32)):
        desc = rt.prefill_kernel(hw, tokens, a_dt, awq=True, out_dtype=c_dt)
        assert desc["name"].startswith(f"gf4_prefill_f16_kernel<64, {waves}, 1, 4,"), (tokens, a_dt, desc)
    a = torch.randn((m, k), generator=g, device=cuda).to(torch.bfloat16)
    awq = torch.rand((k,), generator=g, device=cuda) * 1.5 + 0.5
    out = rt.matmul_prefill(hw, a, awq=awq, out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    rows = np.sort(np.random.default_rng(n + m).choice(m, size=32, replace=False))
    check_prefill(out[rows], a.view(torch.int16).cpu().numpy().view(np.uint16)[rows], awq.cpu().numpy(), wdq)
    a32 = torch.randn((m // 2, k), generator=g, device=cuda)
    out = rt.matmul_prefill(hw, a32, awq=awq, out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    check_prefill(out, a32.cpu().numpy(), awq.cpu().numpy(), wdq)


@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
@pytest.mark.parametrize("a_f32", [False, True])
def test_prefill_workspace_without_room_for_a_split(cuda, n, k, a_f32):
    """A workspace of only the staging bytes (room for no K split) runs the
    planned tiles unsplit, the two in-block K halves included; the result
    matches the planned call within fp32 rounding and the oracle on sampled
    rows.  fp32 activations stage two rows per token, 32-token groups."""
    import torch

    rt = _rt()
    m = 128
    hw, wdq, g = _gpu_gf4(rt, cuda, n, k, n + 3)
    a = torch.randn((m, k), generator=g, device=cuda)
    if not a_f32:
        a = a.to(torch.bfloat16)
    staged_rows = 64 * ((m + 31) // 32) if a_f32 else m
    staged_only = (staged_rows * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256
    small = torch.empty(staged_only, dtype=torch.uint8, device=cuda)
    out = rt.matmul_prefill(hw, a, out_dtype=torch.float32, workspace=small)
    planned = rt.matmul_prefill(hw, a, out_dtype=torch.float32)
    assert om.rel_l2(out.cpu().numpy(), planned.cpu().numpy()) <= 1e-6
    with pytest.raises(rt.Qw35Error, match="workspace"):
        rt.matmul_prefill(hw, a, out_dtype=torch.float32, workspace=small[:staged_only - 256])
    rows = np.sort(np.random.default_rng(n).choice(m, size=32, replace=False))
    a_host = a.cpu().numpy() if a_f32 else a.view(torch.int16).cpu().numpy().view(np.uint16)
    check_prefill(out[rows], a_host[rows], None, wdq)


@pytest.mark.parametrize("m", [9, 12, 40, 100])
def test_matvec_batch_long_chunk_uses_prefill(cuda, m):
    """encodeMatvecBatch semantics: > 8 fp32 tokens on a GF4 weight -> fp32
    [tokens, rows] at fp32 activation precision, so the step from 8 tokens
    (decode GEMV) to 9 (prefill matmul) keeps the same accuracy."""
    rng = np.random.default_rng(2 + m)
    n, k = 256, 4096
    words = ogf4.gf4_pack(bf16_normal(rng, (n, k), 0.02))
    wdq = ogf4.gf4_dequant(words)
    hw = _rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    y = _rt().matvec_batch(hw, _t(x, cuda))
    assert tuple(y.shape) == (m, n)
    check_prefill(y, x, None, wdq)
    y8 = _rt().matvec_batch(hw, _t(x[:8], cuda)).cpu().numpy()
    assert om.rel_l2(y8, om.prefill_f64(wdq, x[:8])) <= 1e-4
