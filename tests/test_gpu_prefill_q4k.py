"""GPU parity of the Q4_K prefill matmul with the super-blocks dequantised
inside the staged kernel (qw35_hip_matmul_prefill with a type-12 weight, no
fp16 image).

The kernel's weight operand is fp16 of the exact Q4_K value
fl32(d * sc * q - dmin * m) (the half dequantisation of the reference's tiled
matmul, qw35_mul_mm_q4_k_f32, qw35_tiled_mm.metal:199-255), the value the fp16
prefill image holds (oracle.matvec.prefill_image).  Two kinds of check:

* one-hot activations (token t = e_t, optionally times a power-of-two AWQ
  entry): every product is a power of two times an fp16 weight and every sum
  adds zeros, so the fp32 output is the image's value bit for bit; over all
  columns of two super-blocks of arbitrary bytes this pins the nibble order,
  the 6-bit scale and min unpacking, the AWQ column of every sub-block and
  the two roundings fp16(fl32(w)) where fl32 is inexact (a fused rounding
  straight to fp16 differs there);
* random activations: tests/helpers.py:check_prefill's bars against the fp64
  product of the unrounded activations and the image (and the exact weights),
  at ragged shapes and, at the 9B's shapes, against the F16-image path on the
  GPU and the oracle on sampled rows."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import activations, awq_scales, check_prefill, make_weight, random_kq_bytes

pytestmark = pytest.mark.gpu

T = om.TYPE_Q4_K


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _bf16_tensor(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


@pytest.mark.parametrize("a_f32", [False, True])
@pytest.mark.parametrize("awq_on", [False, True])
def test_q4k_prefill_one_hot_gives_the_image_bits(cuda, a_f32, awq_on):
    import torch

    n, k = 300, 512
    m = k
    print(f"q4_k prefill one-hot {n}x{k} f32={a_f32} awq={awq_on}", flush=True)
    rng = np.random.default_rng(40 + 2 * a_f32 + awq_on)
    raw = random_kq_bytes(rng, T, n, k)
    w = _rt().HipWeight.upload(raw, T, n, k)
    assert w.prefill is w  # Q4_K takes no image
    awq = np.exp2(rng.integers(-3, 4, size=k)).astype(np.float32) if awq_on else None
    a32 = np.eye(m, k, dtype=np.float32)
    a = _t(a32, cuda) if a_f32 else _bf16_tensor(om.f32_to_bf16_bits(a32), cuda)
    out = _rt().matmul_prefill(w, a, awq=_t(awq, cuda) if awq is not None else None, out_dtype=torch.float32)
    img = om.prefill_image(T, raw, n, k).astype(np.float32)
    # + 0: a weight of -0 sums with the +0 products of the other columns to +0
    want = (img.T * (awq[:, None] if awq is not None else np.float32(1)) + np.float32(0)).astype(np.float32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    if not a_f32 and not awq_on:
        out16 = _rt().matmul_prefill(w, a, out_dtype=torch.bfloat16)
        got = out16.cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, om.f32_to_bf16_bits(want))


# ragged token and row counts, k from one super-block to 12288
@pytest.mark.parametrize("m,n,k", [(1, 256, 256), (37, 1000, 4096), (128, 4096, 4096), (300, 640, 12288),
                                   (64, 33, 2048), (513, 300, 1024), (130, 520, 768)])
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [True, False])
def test_q4k_prefill_matches_oracle(cuda, m, n, k, awq_on, out_f32):
    import torch

    print(f"q4_k prefill m={m} n={n} k={k} awq={awq_on} f32={out_f32}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k + awq_on)
    raw, deq = make_weight(T, n, k, seed=m + n + k)
    w = _rt().HipWeight.upload(raw, T, n, k)
    a32 = activations(rng, m, k)
    awq = awq_scales(rng, k) if awq_on else None
    bits = om.f32_to_bf16_bits(a32)
    img = om.prefill_image(T, raw, n, k).astype(np.float32)
    for a_host, a in ((bits, _bf16_tensor(bits, cuda)), (a32, _t(a32, cuda))):
        out = _rt().matmul_prefill(w, a, awq=_t(awq, cuda) if awq is not None else None,
                                   out_dtype=torch.float32 if out_f32 else torch.bfloat16)
        check_prefill(out, a_host, awq, img, w_exact=deq)


@pytest.mark.parametrize("rows,k,m", [(12288, 4096, 128), (4096, 12288, 512), (8192, 4096, 2048),
                                      (4096, 4096, 300)])
def test_q4k_prefill_full_shapes(cuda, rows, k, m):
    """Q4_K projections at the 9B's FFN / mixer sizes: against the F16-image
    path on the GPU (the same fp16 weights; another tile plan may split K
    differently) and against the oracle on 48 sampled weight rows."""
    import torch

    print(f"q4_k prefill full {rows}x{k} m={m}", flush=True)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(rows + k + m + 1)
    from qwowl35_amd import qwen35

    w = qwen35.synthetic_weight(gen, T, rows, k)
    a = torch.randn((m, k), generator=gen, device=cuda).to(torch.bfloat16)
    out = _rt().matmul_prefill(w, a, out_dtype=torch.float32)
    img = _rt().prefill_image(w)
    ref = _rt().matmul_prefill(img, a, out_dtype=torch.float32)
    assert om.rel_l2(out.cpu().numpy().astype(np.float64), ref.cpu().numpy().astype(np.float64)) <= 1e-5
    rows_s = np.random.default_rng(rows + m).choice(rows, 48, replace=False)
    raw = w.storage.cpu().numpy()
    rb = k // 256 * 144
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows_s])
    w_s = om.prefill_image(T, sub, 48, k).astype(np.float32)
    a_bits = a.cpu().view(torch.int16).numpy().view(np.uint16)
    check_prefill(out[:, rows_s], a_bits, None, w_s, w_exact=om.dequant(T, sub, 48, k))


def test_q4k_matvec_batch_long_chunk(cuda):
    """matvec_batch over more than 8 fp32 tokens sends a Q4_K weight to the
    in-kernel prefill path: fp32 activation precision, fp16 weights."""
    rows, k, m = 700, 4096, 40
    raw, deq = make_weight(T, rows, k, seed=19)
    x = activations(np.random.default_rng(20), m, k)
    w = _rt().HipWeight.upload(raw, T, rows, k)
    got = _rt().matvec_batch(w, _t(x, cuda))
    check_prefill(got, x, None, om.prefill_image(T, raw, rows, k).astype(np.float32), w_exact=deq)


def test_q4k_prefill_needs_workspace(cuda):
    import torch

    raw, _ = make_weight(T, 64, 2048, seed=3)
    w = _rt().HipWeight.upload(raw, T, 64, 2048)
    a = torch.zeros((4, 2048), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(_rt().Qw35Error, match="q4_k weights need a 256-byte aligned workspace"):
        _rt().matmul_prefill(w, a, workspace=False)
