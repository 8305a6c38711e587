"""GPU parity of the k-quant prefill path: the fp16 prefill image
(qw35_hip_dequantize_f16) and the F16-weight prefill matmul
(qw35_hip_matmul_prefill with a type-1 weight).

Oracle: oracle.matvec.prefill_image (fp16_rne of the exact dequantised weight,
the half dequantisation of the reference's tiled matmul,
qw35_tiled_mm.metal:199-255) and an fp64 product of the exact operands the
kernel contracts, A' = bf16_rne(awq * A) and the fp16 weights.  Bars: the image
bit-exact; fp32 output within 1e-3 relative L2 and, per element, within the
fp32-accumulation allowance 2^-16 * sum_k |A'_k W_k|; bf16 output within one
bf16 ulp plus that allowance (the GF4 prefill bars of test_gpu_prefill.py)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from oracle import q6_k as oq6
from tests.helpers import activations, awq_scales, bf16_normal, make_weight

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


def _bf16_tensor(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


@pytest.mark.parametrize("m,n,k", [(1, 256, 2048), (37, 1000, 4096), (128, 4096, 4096), (300, 640, 12288)])
@pytest.mark.parametrize("awq_on", [False, True])
@pytest.mark.parametrize("out_f32", [True, False])
def test_f16_prefill_matches_oracle(cuda, m, n, k, awq_on, out_f32):
    import torch

    rng = np.random.default_rng(m * 7 + n + k + awq_on)
    w16 = bf16_normal(rng, (n, k), 0.02).astype(np.float16)
    a32 = activations(rng, m, k)
    awq = awq_scales(rng, k) if awq_on else None
    bits = om.f32_to_bf16_bits(a32)
    a_eff = om.prefill_operand(bits, awq)
    hw = _rt().HipWeight.upload(w16.view(np.uint8), om.TYPE_F16, n, k)
    out = _rt().matmul_prefill(hw, _bf16_tensor(bits, cuda), awq=_t(awq, cuda) if awq is not None else None,
                               out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    w64 = w16.astype(np.float64)
    want = a_eff.astype(np.float64) @ w64.T
    allow = (np.abs(a_eff.astype(np.float64)) @ np.abs(w64).T) * 2.0 ** -16
    if out_f32:
        got = out.cpu().numpy().astype(np.float64)
        assert om.rel_l2(got, want) <= 1e-3
        assert np.all(np.abs(got - want) <= allow + 1e-30)
    else:
        got = om.bf16_bits_to_f32(out.cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
        assert np.all(np.abs(got - want) <= ulp + allow)


def test_f16_prefill_fp32_input(cuda):
    import torch

    rng = np.random.default_rng(5)
    m, n, k = 64, 512, 4096
    w16 = bf16_normal(rng, (n, k), 0.02).astype(np.float16)
    a32 = activations(rng, m, k) * np.float32(100.0)
    awq = awq_scales(rng, k)
    hw = _rt().HipWeight.upload(w16.view(np.uint8), om.TYPE_F16, n, k)
    out = _rt().matmul_prefill(hw, _t(a32, cuda), awq=_t(awq, cuda), out_dtype=torch.float32).cpu().numpy()
    a_eff = om.bf16_round(a32 * awq[None, :]).astype(np.float64)
    want = a_eff @ w16.astype(np.float64).T
    assert om.rel_l2(out, want) <= 1e-3


@pytest.mark.parametrize("name", ["gf2", "q8_0", "q4_k", "q5_k", "q6_k"])
def test_matvec_batch_long_kquant_chunk(cuda, name):
    rows, k, m = 700, 4096, 64
    raw, deq = _weight(name, rows, k, seed=9)
    rng = np.random.default_rng(10)
    x = activations(rng, m, k)
    w = _rt().HipWeight.upload(raw, NAMES[name], rows, k)
    got = _rt().matvec_batch(w, _t(x, cuda)).cpu().numpy()
    img = om.prefill_image(NAMES[name], raw, rows, k).astype(np.float64)
    assert om.rel_l2(got, om.bf16_round(x).astype(np.float64) @ img.T) <= 1e-3
    # against the exact weights and fp32 activations: fp16 weights and bf16
    # activations (the reference tiled matmul's half weights) cost ~2^-9
    assert om.rel_l2(got, om.matvec_f64(deq, x)) <= 5e-3
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
