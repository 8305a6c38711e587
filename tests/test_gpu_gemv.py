"""GPU parity of the decode GEMVs and the dequantiser, through the C ABI.

Bars: dequantisation bit-exact against the oracle; GEMV outputs within
GEMV_REL_L2 (1e-3) relative L2 of the fp64 matvec on the oracle-dequantised
weights.  Shapes run from tiny/ragged cases to the Qwen3.5-9B projections.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import gf4 as ogf4
from oracle import matvec as om
from tests.helpers import GEMV_REL_L2, TYPES, activations, awq_scales, make_weight, random_gf4_words

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _upload(raw, type_id, rows, k):
    return _rt().HipWeight.upload(raw, type_id, rows, k)


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    same = a.view(np.uint32) == b.view(np.uint32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(same | both_nan))


@pytest.mark.parametrize("name", ["gf4", "gf2", "q8_0", "q4_k", "q5_k"])
@pytest.mark.parametrize("rows,k", [(3, 256), (64, 4096), (37, 12288)])
def test_dequant_bit_exact(cuda, name, rows, k):
    type_id = TYPES[name]
    raw, deq = make_weight(type_id, rows, k, seed=rows * 7 + k)
    w = _upload(raw, type_id, rows, k)
    got = _rt().dequantize(w).cpu().numpy()
    assert _bits_equal(got, deq)


def test_dequant_gf4_arbitrary_words(cuda):
    rng = np.random.default_rng(11)
    words = random_gf4_words(rng, (256, 512))
    w = _upload(words.view(np.uint8), om.TYPE_GF4, 256, 4096)
    got = _rt().dequantize(w).cpu().numpy()
    assert _bits_equal(got, ogf4.gf4_dequant(words))


def test_dequant_row_gather(cuda):
    import torch

    raw, deq = make_weight(om.TYPE_Q8_0, 50, 512, seed=3)
    w = _upload(raw, om.TYPE_Q8_0, 50, 512)
    ids = np.array([7, 0, 49, 7, 1000], dtype=np.int32)  # 1000 is out of range -> zeros
    got = _rt().dequantize(w, torch.from_numpy(ids).to(cuda)).cpu().numpy()
    want = np.concatenate([deq[[7, 0, 49, 7]], np.zeros((1, 512), np.float32)])
    assert _bits_equal(got, want)


@pytest.mark.parametrize("name", ["gf4", "gf2", "q8_0", "q4_k", "q5_k"])
@pytest.mark.parametrize("rows,k", [(1, 256), (37, 4096), (130, 12288), (5, 8192), (64, 1024)])
@pytest.mark.parametrize("nb", [1, 2, 3, 8])
def test_gemv_parity(cuda, name, rows, k, nb):
    type_id = TYPES[name]
    rng = np.random.default_rng(rows + k + nb)
    raw, deq = make_weight(type_id, rows, k, seed=rows * 31 + k)
    x = activations(rng, nb, k)
    w = _upload(raw, type_id, rows, k)
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    want = om.matvec_f64(deq, x)
    assert om.rel_l2(y, want) <= GEMV_REL_L2


@pytest.mark.parametrize("name", ["gf4", "gf2", "q8_0", "q4_k", "q5_k"])
def test_gemv_awq_and_residual(cuda, name):
    import torch

    type_id = TYPES[name]
    rows, k, nb = 96, 4096, 2
    rng = np.random.default_rng(5)
    raw, deq = make_weight(type_id, rows, k, seed=9)
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    base = rng.standard_normal((nb, rows)).astype(np.float32)
    w = _upload(raw, type_id, rows, k)
    dst = torch.from_numpy(base.copy()).to(cuda)
    _rt().decode_matvec(w, _t(x, cuda), dst=dst, residual=True, awq=_t(a, cuda))
    want = base.astype(np.float64) + om.matvec_f64(deq, x, a)
    assert om.rel_l2(dst.cpu().numpy(), want) <= GEMV_REL_L2


@pytest.mark.parametrize("name", ["gf4", "gf2", "q8_0", "q4_k", "q5_k"])
@pytest.mark.parametrize("nb", [1, 4])
def test_swiglu_parity(cuda, name, nb):
    type_id = TYPES[name]
    rows, k = 200, 4096
    rng = np.random.default_rng(21 + nb)
    rg, dg = make_weight(type_id, rows, k, seed=1, std=0.05)
    ru, du = make_weight(type_id, rows, k, seed=2, std=0.05)
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    g = _upload(rg, type_id, rows, k)
    u = _upload(ru, type_id, rows, k)
    y = _rt().ffn_gate_up_swiglu(g, u, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy()
    want = om.swiglu_f64(dg, du, x, a)
    assert om.rel_l2(y, want) <= GEMV_REL_L2


def test_gemv_extreme_activation_scale(cuda):
    """fp16 staging of GF4 activations must not overflow or flush: |x| ~ 1e6 and ~ 1e-6."""
    rows, k = 64, 4096
    raw, deq = make_weight(om.TYPE_GF4, rows, k, seed=4)
    w = _upload(raw, om.TYPE_GF4, rows, k)
    rng = np.random.default_rng(8)
    for mag in (1e6, 1e-6):
        x = activations(rng, 2, k) * np.float32(mag)
        y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
        assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


def test_gemv_config1_full_size(cuda):
    """Config 1: GF4 12288x4096, batch 1, W = bf16(0.02 N(0,1)), x = N(0,1)."""
    raw, deq = make_weight(om.TYPE_GF4, 12288, 4096, seed=1)
    w = _upload(raw, om.TYPE_GF4, 12288, 4096)
    x = activations(np.random.default_rng(2), 1, 4096)
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


def test_golden_fixtures(cuda):
    """The library reproduces the committed fixtures (tests/golden/gemv_golden.npz)."""
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemv_golden.npz"), allow_pickle=False)
    x = _t(g["x"], cuda)
    a = _t(g["awq"], cuda)
    for name, raw_key, rows in (("gf4", "gf4_words", 32), ("q8_0", "q8_0_raw", 16), ("q4_k", "q4_k_raw", 16)):
        type_id = TYPES[name]
        w = _upload(np.ascontiguousarray(g[raw_key]).view(np.uint8), type_id, rows, 512)
        assert _bits_equal(_rt().dequantize(w).cpu().numpy(), g[f"{name}_deq"]), name
        y = _rt().decode_matvec(w, x, awq=a).cpu().numpy()
        assert om.rel_l2(y, g[f"{name}_y"]) <= GEMV_REL_L2, name
    w = _upload(g["gf4_any_words"].view(np.uint8), om.TYPE_GF4, 8, 512)
    assert _bits_equal(_rt().dequantize(w).cpu().numpy(), g["gf4_any_deq"])


@pytest.mark.parametrize("name", ["gf2", "q4_k", "q5_k"])
@pytest.mark.parametrize("nb", [1, 8])
def test_gemv_large_ragged_kquant(cuda, name, nb):
    """65549 x 4096 k-quant weights made on the GPU (the >= 4096-tile plans of
    an LM-head-sized matrix, with a ragged last tile): the GEMV against the fp64
    product of the library's dequantised weight, which the tests above pin
    bit-for-bit to the oracle at smaller shapes."""
    import torch

    rt = _rt()
    type_id = TYPES[name]
    rows, k = 65549, 4096
    g = torch.Generator(device=cuda)
    g.manual_seed(5 + nb)
    src = torch.randn((rows, k), generator=g, device=cuda) * 0.02
    w = rt.quantize_weight(src, type_id)
    del src
    x = torch.randn((nb, k), generator=g, device=cuda)
    y = rt.decode_matvec(w, x).double()
    want = rt.dequantize(w).double() @ x.double().T
    assert om.rel_l2(y.cpu().numpy(), want.T.cpu().numpy()) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [8, 4])
@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q5_k", "gf2", "gf4"])
def test_swiglu_tall_batch8(cuda, name, nb):
    """Fused gate/up at batch 4 and 8 on 8208 rows (the tall-matrix launch
    shapes: three row tiles per workgroup, ragged last tile), weights made on
    the GPU, against fp64 on the library's dequantised weights."""
    import torch

    rt = _rt()
    type_id = TYPES[name]
    rows, k = 8208, 4096
    g = torch.Generator(device=cuda)
    g.manual_seed(3)
    wg = rt.quantize_weight(torch.randn((rows, k), generator=g, device=cuda) * 0.02, type_id)
    wu = rt.quantize_weight(torch.randn((rows, k), generator=g, device=cuda) * 0.02, type_id)
    x = torch.randn((nb, k), generator=g, device=cuda)
    y = rt.ffn_gate_up_swiglu(wg, wu, x).double()
    gate = rt.dequantize(wg).double() @ x.double().T
    up = rt.dequantize(wu).double() @ x.double().T
    want = (gate / (1 + torch.exp(-gate)) * up).T
    assert om.rel_l2(y.cpu().numpy(), want.cpu().numpy()) <= GEMV_REL_L2


def test_entry_points_validate_buffers(cuda):
    """The Python entry points reject, before any launch, an output that does
    not hold n_batch x rows fp32 values, an AWQ vector that is not k fp32
    values, and weight bytes outside their storage (the C ABI sees only raw
    pointers, so these would otherwise be out-of-bounds device accesses)."""
    import torch

    rt = _rt()
    raw, _ = make_weight(om.TYPE_Q8_0, 64, 512, seed=1)
    w = _upload(raw, om.TYPE_Q8_0, 64, 512)
    x = torch.zeros((2, 512), dtype=torch.float32, device=cuda)
    bad_dst = [torch.zeros((2, 63), dtype=torch.float32, device=cuda),
               torch.zeros((2, 64), dtype=torch.float16, device=cuda),
               torch.zeros((2, 128), dtype=torch.float32, device=cuda)[:, ::2]]
    for d in bad_dst:
        with pytest.raises(rt.Qw35Error, match="dst"):
            rt.decode_matvec(w, x, dst=d)
        with pytest.raises(rt.Qw35Error, match="dst"):
            rt.DecodePlan().matvec(w, x, d)
        with pytest.raises(rt.Qw35Error, match="dst"):
            rt.ffn_gate_up_swiglu(w, w, x, dst=d)
    for a in (torch.ones(511, device=cuda), torch.ones(512, dtype=torch.float16, device=cuda)):
        with pytest.raises(rt.Qw35Error, match="awq"):
            rt.decode_matvec(w, x, awq=a)
        with pytest.raises(rt.Qw35Error, match="awq"):
            rt.output_argmax(w, x, awq=a)
    with pytest.raises(rt.Qw35Error, match="n_batch"):
        rt.decode_matvec(w, torch.zeros((9, 512), dtype=torch.float32, device=cuda))
    with pytest.raises(rt.Qw35Error, match="exceed"):
        rt.HipWeight.from_device(w.storage, om.TYPE_Q8_0, 64, 512, offset=16)
    with pytest.raises(rt.Qw35Error, match="bytes"):
        rt.HipWeight.upload(raw[:-1], om.TYPE_Q8_0, 64, 512)
