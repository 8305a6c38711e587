"""GPU parity of the q8_0 prefill matmul with the weights dequantised inside
the staged kernel (qw35_hip_matmul_prefill with a type-8 weight, no fp16
image).

The kernel's weight operand is fp16(d * q), the same value the fp16 prefill
image holds (oracle.matvec.prefill_image: fp16_rne of the exact dequantised
weight, the half dequantisation of the reference's tiled matmul,
qw35_tiled_mm.metal:199-255), so the oracle is the fp64 product of
the unrounded activations (oracle.matvec.prefill_f64) and that image, with the
bars of tests/helpers.py:check_prefill: fp32 output within prefill_rel_l2_bar
of it, within 1e-3 of the product with the exact weights, and per element
within the fp32-accumulation allowance 2^-16 * sum_k |A'_k W_k| of the staged
operand; bf16 output within one bf16 ulp plus that allowance.  At the 9B's full shapes the in-kernel path is
checked against the F16-image path on the GPU (same products, possibly another
K split) and against the oracle on sampled rows."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import activations, awq_scales, check_prefill, make_weight

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _bf16_tensor(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


# ragged token and row counts, k from one 256-column chunk (four 64-column
# steps: the last step's span sits at the end of its loads) to 12288
@pytest.mark.parametrize("m,n,k", [(1, 256, 256), (37, 1000, 4096), (128, 4096, 4096), (300, 640, 12288),
                                   (64, 33, 2048), (513, 300, 1024)])
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [True, False])
def test_q8_prefill_matches_oracle(cuda, m, n, k, awq_on, out_f32):
    import torch

    print(f"q8_0 prefill m={m} n={n} k={k} awq={awq_on} f32={out_f32}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k + awq_on)
    raw, _ = make_weight(om.TYPE_Q8_0, n, k, seed=m + n + k)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q8_0, n, k)
    assert w.prefill is w  # q8_0 takes no image
    a32 = activations(rng, m, k)
    awq = awq_scales(rng, k) if awq_on else None
    bits = om.f32_to_bf16_bits(a32)
    out = _rt().matmul_prefill(w, _bf16_tensor(bits, cuda), awq=_t(awq, cuda) if awq is not None else None,
                               out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    img = om.prefill_image(om.TYPE_Q8_0, raw, n, k).astype(np.float32)
    check_prefill(out, bits, awq, img, w_exact=om.dequant(om.TYPE_Q8_0, raw, n, k))
    out = _rt().matmul_prefill(w, _t(a32, cuda), awq=_t(awq, cuda) if awq is not None else None,
                               out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    check_prefill(out, a32, awq, img, w_exact=om.dequant(om.TYPE_Q8_0, raw, n, k))


def test_q8_prefill_fp32_input_and_extreme_scales(cuda):
    """fp32 activations over a wide range (the staging pass scales each token
    row by a power of two) and q8_0 blocks whose d spans fp16's range."""
    import torch

    rng = np.random.default_rng(11)
    m, n, k = 96, 512, 4096
    raw, _ = make_weight(om.TYPE_Q8_0, n, k, seed=12)
    blocks = np.asarray(raw).reshape(n, k // 32, 34).copy()
    # fp16(d * q) stays finite: |q| <= 128, d <= 64
    d = rng.choice(np.array([2.0 ** -14, 2.0 ** -8, 1.0, 64.0], np.float16), size=(n, k // 32))
    blocks[:, :, :2] = d.view(np.uint8).reshape(n, k // 32, 2)
    raw = blocks.reshape(-1)
    a32 = activations(rng, m, k) * np.exp2(rng.integers(-20, 20, size=(m, 1))).astype(np.float32)
    awq = awq_scales(rng, k)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q8_0, n, k)
    out = _rt().matmul_prefill(w, _t(a32, cuda), awq=_t(awq, cuda), out_dtype=torch.float32)
    assert np.all(np.isfinite(out.cpu().numpy()))
    check_prefill(out, a32, awq, om.prefill_image(om.TYPE_Q8_0, raw, n, k).astype(np.float32))


@pytest.mark.parametrize("rows,k,m", [(8192, 4096, 2048), (8192, 4096, 512), (8192, 4096, 128), (4096, 4096, 128),
                                      (12352, 4096, 512), (4096, 12288, 512), (4096, 4096, 1200)])
def test_q8_prefill_full_shapes(cuda, rows, k, m):
    """The 9B's q8_0 projections at full size: against the F16-image path on
    the GPU and against the oracle on 48 sampled weight rows."""
    import torch

    print(f"q8_0 prefill full {rows}x{k} m={m}", flush=True)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(rows + k + m)
    from qwowl35_amd import qwen35

    w = qwen35.synthetic_weight(gen, om.TYPE_Q8_0, rows, k)
    a = torch.randn((m, k), generator=gen, device=cuda).to(torch.bfloat16)
    out = _rt().matmul_prefill(w, a, out_dtype=torch.float32)
    img = _rt().prefill_image(w)
    ref = _rt().matmul_prefill(img, a, out_dtype=torch.float32)
    assert om.rel_l2(out.cpu().numpy().astype(np.float64), ref.cpu().numpy().astype(np.float64)) <= 1e-5
    rows_s = np.random.default_rng(rows).choice(rows, 48, replace=False)
    raw = w.storage.cpu().numpy()
    rb = k // 32 * 34
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows_s])
    w_s = om.prefill_image(om.TYPE_Q8_0, sub, 48, k).astype(np.float32)
    a_bits = a.cpu().view(torch.int16).numpy().view(np.uint16)
    for res in (out, ref):  # the in-kernel path and the F16-image path (256-token tiles at M = 2048)
        check_prefill(res[:, rows_s], a_bits, None, w_s, w_exact=om.dequant(om.TYPE_Q8_0, sub, 48, k))


def test_q8_prefill_needs_workspace(cuda):
    import torch

    raw, _ = make_weight(om.TYPE_Q8_0, 64, 2048, seed=3)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q8_0, 64, 2048)
    a = torch.zeros((4, 2048), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(_rt().Qw35Error, match="q8_0 weights need a 256-byte aligned workspace"):
        _rt().matmul_prefill(w, a, workspace=False)
