"""GPU parity of the k-quant prefill path: the fp16 prefill image
(qw35_hip_dequantize_f16) and the F16-weight prefill matmul
(qw35_hip_matmul_prefill with a type-1 weight).

Oracle: oracle.matvec.prefill_image (fp16_rne of the exact dequantised weight,
the half dequantisation of the reference's tiled matmul,
qw35_tiled_mm.metal:199-255) and oracle.matvec.prefill_f64, the fp64 product
of the unrounded activations (the reference keeps them fp32,
qw35_tiled_mm.metal:200-224).  Bars: the image bit-exact; the bars of
tests/helpers.py:check_prefill (the GF4 prefill bars): fp32 output within
prefill_rel_l2_bar of the product with the image and within 1e-3 of the
product with the exact weights, per element within the fp32-accumulation
allowance of the staged operand; bf16 output within one bf16 ulp plus that
allowance."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from oracle import q6_k as oq6
from tests.helpers import activations, awq_scales, bf16_normal, check_prefill, make_weight, random_kq_bytes

pytestmark = pytest.mark.gpu

NAMES = {"gf4": om.TYPE_GF4, "gf2": om.TYPE_GF2, "q8_0": om.TYPE_Q8_0, "q4_k": om.TYPE_Q4_K, "q5_k": om.TYPE_Q5_K,
         "q6_k": om.TYPE_Q6_K}


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _weight(name, rows, k, seed):
    if name == "q6_k":
        rng = np.random.default_rng(seed)
        raw = oq6.q6_k_quantize(bf16_normal(rng, (rows, k), 0.02))
        return raw, oq6.q6_k_dequant(raw, rows, k)
    return make_weight(NAMES[name], rows, k, seed=seed)


@pytest.mark.parametrize("name", list(NAMES))
@pytest.mark.parametrize("rows,k", [(37, 2048), (96, 4096)])
def test_prefill_image_bit_exact(cuda, name, rows, k):
    raw, _ = _weight(name, rows, k, seed=rows + k)
    w = _rt().HipWeight.upload(raw, NAMES[name], rows, k)
    img = _rt().prefill_image(w)
    assert img.type_id == om.TYPE_F16 and img.rows == rows and img.k == k
    got = img.storage.cpu().numpy().view(np.uint16).reshape(rows, k)
    want = om.prefill_image(NAMES[name], raw, rows, k).view(np.uint16)
    assert np.array_equal(got, want)
    # the F16 weight dequantises back to exactly the fp16 values
    back = _rt().dequantize(img).cpu().numpy()
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


@pytest.mark.parametrize("name", ["q4_k", "q5_k"])
def test_prefill_image_bit_exact_random_bytes(cuda, name):
    """Arbitrary super-block bytes: the image is fp16 of the fp32 weight (two
    roundings), also where the fp32 rounding is inexact."""
    rows, k = 64, 1024
    raw = random_kq_bytes(np.random.default_rng(31), NAMES[name], rows, k)
    w = _rt().HipWeight.upload(raw, NAMES[name], rows, k)
    got = _rt().prefill_image(w).storage.cpu().numpy().view(np.uint16).reshape(rows, k)
    assert np.array_equal(got, om.prefill_image(NAMES[name], raw, rows, k).view(np.uint16))


def _bf16_tensor(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


@pytest.mark.parametrize("m,n,k", [(1, 256, 2048), (37, 1000, 4096), (128, 4096, 4096), (300, 640, 12288)])
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [True, False])
@pytest.mark.parametrize("a_f32", [False, True])
def test_f16_prefill_matches_oracle(cuda, m, n, k, awq_on, out_f32, a_f32):
    import torch

    rng = np.random.default_rng(m * 7 + n + k + awq_on)
    w16 = bf16_normal(rng, (n, k), 0.02).astype(np.float16)
    a32 = activations(rng, m, k)
    awq = awq_scales(rng, k) if awq_on else None
    a_host = a32 if a_f32 else om.f32_to_bf16_bits(a32)
    a_dev = _t(a32, cuda) if a_f32 else _bf16_tensor(a_host, cuda)
    hw = _rt().HipWeight.upload(w16.view(np.uint8), om.TYPE_F16, n, k)
    out = _rt().matmul_prefill(hw, a_dev, awq=_t(awq, cuda) if awq is not None else None,
                               out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    check_prefill(out, a_host, awq, w16.astype(np.float32))


def test_f16_prefill_fp32_input(cuda):
    """fp32 activations of larger magnitude with AWQ: fp32 precision (hi/lo staging)."""
    import torch

    rng = np.random.default_rng(5)
    m, n, k = 64, 512, 4096
    w16 = bf16_normal(rng, (n, k), 0.02).astype(np.float16)
    a32 = activations(rng, m, k) * np.float32(100.0)
    awq = awq_scales(rng, k)
    hw = _rt().HipWeight.upload(w16.view(np.uint8), om.TYPE_F16, n, k)
    out = _rt().matmul_prefill(hw, _t(a32, cuda), awq=_t(awq, cuda), out_dtype=torch.float32)
    check_prefill(out, a32, awq, w16.astype(np.float32))


@pytest.mark.parametrize("name", ["gf2", "q8_0", "q4_k", "q5_k", "q6_k"])
def test_matvec_batch_long_kquant_chunk(cuda, name):
    """More than 8 fp32 tokens on a k-quant weight: the prefill matmul on its
    fp16 image (q8_0, Q4_K: decoded in the kernel to the same values) with fp32
    activation precision; against the exact weights the fp16 weights cost
    ~2^-12 per weight, under the 1e-3 bar."""
    rows, k, m = 700, 4096, 64
    raw, deq = _weight(name, rows, k, seed=9)
    rng = np.random.default_rng(10)
    x = activations(rng, m, k)
    w = _rt().HipWeight.upload(raw, NAMES[name], rows, k)
    got = _rt().matvec_batch(w, _t(x, cuda))
    img = om.prefill_image(NAMES[name], raw, rows, k)
    check_prefill(got, x, None, img.astype(np.float32), w_exact=deq)
    assert w.prefill is w.prefill  # the image is made once and kept


def test_f16_weight_is_prefill_only(cuda):
    import torch

    w16 = np.zeros((16, 2048), np.float16)
    hw = _rt().HipWeight.upload(w16.view(np.uint8), om.TYPE_F16, 16, 2048)
    x = torch.zeros(2048, dtype=torch.float32, device=cuda)
    with pytest.raises(_rt().Qw35Error, match="prefill matmul only"):
        _rt().decode_matvec(hw, x)
    a = torch.zeros((4, 2048), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(_rt().Qw35Error, match="need a 256-byte aligned workspace"):
        _rt().matmul_prefill(hw, a, workspace=False)
