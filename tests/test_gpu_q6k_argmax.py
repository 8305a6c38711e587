"""GPU parity of the Q6_K codec (dequantiser, encoder, GEMV) and of the greedy
LM head (qw35_hip_output_argmax), through the C ABI.

Bars: Q6_K dequantisation and encoding bit-exact against oracle/q6_k.py; GEMV
within GEMV_REL_L2 (1e-3) relative L2 of the fp64 matvec; the greedy head
returns exactly the reference rule (largest, ties to the smaller row, NaN never
chosen: oracle.matvec.argmax_rule) applied to the logits qw35_hip_decode_matvec
computes for the same weight and input (q8_0 / Q4_K / Q6_K share the GEMV
kernel and plan, so the logits are bit-identical); for GF4 the chosen row's
fp64 logit is within the GEMV tolerance of the fp64 maximum."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from oracle import q6_k as oq6
from tests.helpers import GEMV_REL_L2, activations, awq_scales, bf16_normal, make_weight

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _q6k(rows, k, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = bf16_normal(rng, (rows, k), std)
    raw = oq6.q6_k_quantize(w)
    return raw, oq6.q6_k_dequant(raw, rows, k)


def _random_q6k_raw(rng, rows, k):
    raw = rng.integers(0, 256, size=rows * (k // 256) * 210, dtype=np.uint8)
    blk = oq6.as_blocks(raw)
    blk["d"] = (rng.standard_normal(blk.shape) * np.exp(rng.uniform(-8, 2, blk.shape))).astype(np.float16)
    return raw


@pytest.mark.parametrize("rows,k", [(3, 2048), (64, 4096), (37, 12288)])
def test_q6k_dequant_bit_exact(cuda, rows, k):
    raw, deq = _q6k(rows, k, seed=rows + k)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, rows, k)
    assert np.array_equal(_bits(_rt().dequantize(w).cpu().numpy()), _bits(deq))


def test_q6k_dequant_random_blocks_and_gather(cuda):
    import torch

    rng = np.random.default_rng(21)
    raw = _random_q6k_raw(rng, 40, 4096)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, 40, 4096)
    deq = oq6.q6_k_dequant(raw, 40, 4096)
    assert np.array_equal(_bits(_rt().dequantize(w).cpu().numpy()), _bits(deq))
    ids = torch.tensor([39, 0, 7, 1000], dtype=torch.int32, device=cuda)
    got = _rt().dequantize(w, row_ids=ids).cpu().numpy()
    assert np.array_equal(_bits(got[:3]), _bits(deq[[39, 0, 7]]))
    assert np.all(got[3] == 0)


@pytest.mark.parametrize("rows,k", [(5, 2048), (48, 4096), (17, 12288)])
def test_q6k_encoder_bit_exact(cuda, rows, k):
    rng = np.random.default_rng(rows * 3 + k)
    src = bf16_normal(rng, (rows, k), 0.02)
    src[0, :16] = 0.0                      # an all-zero sub-block
    src[1, 256:512] *= 1000.0              # a wide-range super-block
    got = _rt().quantize(_t(src, cuda), om.TYPE_Q6_K).cpu().numpy()
    assert np.array_equal(got, oq6.q6_k_quantize(src))


def test_q6k_encoder_with_awq_columns(cuda):
    rng = np.random.default_rng(22)
    src = bf16_normal(rng, (9, 4096), 0.02)
    cs = awq_scales(rng, 4096)
    got = _rt().quantize(_t(src, cuda), om.TYPE_Q6_K, col_scale=_t(cs, cuda)).cpu().numpy()
    assert np.array_equal(got, oq6.q6_k_quantize((src * cs).astype(np.float32)))


@pytest.mark.parametrize("nb", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("rows,k", [(64, 4096), (37, 12288), (1000, 2048)])
def test_q6k_gemv(cuda, nb, rows, k):
    raw, deq = _q6k(rows, k, seed=nb * 100 + rows)
    rng = np.random.default_rng(nb + rows)
    x = activations(rng, nb, k)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, rows, k)
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


# Rows of k % 2048 != 0 start 4, 8 or 12 bytes past a 16-byte boundary:
# 2560 -> 2100-byte rows (4 mod 16), 5120 -> 4200 (8), 9728 -> 7980 (12).
@pytest.mark.parametrize("rows,k", [(100, 2560), (102, 5120), (36, 9728), (2, 5120), (4, 2560)])
@pytest.mark.parametrize("nb", [1, 3, 8])
def test_q6k_gemv_unaligned_rows(cuda, rows, k, nb):
    import torch

    print(f"q6_k gemv {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(rows + k + nb)
    raw = _random_q6k_raw(rng, rows, k)
    deq = oq6.q6_k_dequant(raw, rows, k)
    x = activations(rng, nb, k)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, rows, k)
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2
    a = awq_scales(rng, k)
    y0 = rng.standard_normal((nb, rows)).astype(np.float32)
    dst = torch.from_numpy(y0.copy()).to(cuda)
    _rt().decode_matvec(w, _t(x, cuda), dst=dst, residual=True, awq=_t(a, cuda))
    assert om.rel_l2(dst.cpu().numpy(), y0.astype(np.float64) + om.matvec_f64(deq, x, a)) <= GEMV_REL_L2
    # every row within the bar relative to its batch row's RMS output: a misread row (the last
    # one's final 16-byte segment ends the matrix) fails here even where rel-L2 over all would not
    ref = om.matvec_f64(deq, x)
    scale = np.linalg.norm(ref, axis=1, keepdims=True) / np.sqrt(rows)
    assert np.all(np.abs(y - ref) <= GEMV_REL_L2 * scale + 1e-6)


@pytest.mark.parametrize("nb", [1, 5])
def test_q6k_head_unaligned_rows(cuda, nb):
    """The fused greedy head on a 5120-column Q6_K head (4200-byte rows) equals
    the rule on the same launch shape's logits, and its logits match fp64."""
    rows, k = 4000, 5120
    rng = np.random.default_rng(nb)
    raw, deq = _q6k(rows, k, seed=nb)
    x = activations(rng, nb, k)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, rows, k)
    xt = _t(x, cuda)
    logits = _rt().decode_matvec(w, xt).cpu().numpy()
    assert om.rel_l2(logits, om.matvec_f64(deq, x)) <= GEMV_REL_L2
    tok, lg = _rt().output_argmax(w, xt)
    ids, best = om.argmax_rule(logits)
    assert np.array_equal(tok.cpu().numpy().view(np.uint32), ids)
    assert np.array_equal(_bits(lg.cpu().numpy()), _bits(best))


def test_q6k_gemv_awq_residual_and_random_blocks(cuda):
    import torch

    rng = np.random.default_rng(23)
    rows, k, nb = 300, 4096, 4
    raw = _random_q6k_raw(rng, rows, k)
    deq = oq6.q6_k_dequant(raw, rows, k)
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    y0 = rng.standard_normal((nb, rows)).astype(np.float32)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, rows, k)
    dst = torch.from_numpy(y0.copy()).to(cuda)
    _rt().decode_matvec(w, _t(x, cuda), dst=dst, residual=True, awq=_t(a, cuda))
    ref = y0.astype(np.float64) + om.matvec_f64(deq, x, a)
    assert om.rel_l2(dst.cpu().numpy(), ref) <= GEMV_REL_L2


def test_q6k_rejects_unaligned_rows_and_swiglu(cuda):
    raw, _ = _q6k(4, 2048, seed=1)
    with pytest.raises(_rt().Qw35Error, match="k % 512"):
        _rt().HipWeight.upload(np.zeros(4 * 5 * 210, np.uint8), om.TYPE_Q6_K, 4, 1280)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, 4, 2048)
    import torch

    x = torch.zeros(2048, dtype=torch.float32, device=cuda)
    with pytest.raises(_rt().Qw35Error, match="no fused gate/up"):
        _rt().ffn_gate_up_swiglu(w, w, x)


def _weight(name, rows, k, seed):
    if name == "q6_k":
        return _q6k(rows, k, seed)
    return make_weight(_TYPE[name], rows, k, seed=seed)


_TYPE = {"q8_0": om.TYPE_Q8_0, "q4_k": om.TYPE_Q4_K, "q5_k": om.TYPE_Q5_K, "q6_k": om.TYPE_Q6_K,
         "gf4": om.TYPE_GF4, "gf2": om.TYPE_GF2}


@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q5_k", "q6_k", "gf2"])
@pytest.mark.parametrize("nb", [1, 2, 5, 8])
@pytest.mark.parametrize("rows", [1000, 4133])
def test_argmax_equals_rule_on_matvec_logits(cuda, name, nb, rows):
    k = 4096
    raw, _ = _weight(name, rows, k, seed=rows + nb)
    rng = np.random.default_rng(rows * nb)
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    w = _rt().HipWeight.upload(raw, _TYPE[name], rows, k)
    xt, at = _t(x, cuda), _t(a, cuda)
    logits = _rt().decode_matvec(w, xt, awq=at).cpu().numpy()
    tok, lg = _rt().output_argmax(w, xt, awq=at)
    ids, best = om.argmax_rule(logits)
    assert np.array_equal(tok.cpu().numpy().view(np.uint32), ids)
    assert np.array_equal(_bits(lg.cpu().numpy()), _bits(best))


def test_argmax_ties_go_to_smaller_row(cuda):
    rows, k = 2000, 4096
    raw, _ = _q6k(1, k, seed=5)
    rb = raw.size
    full = np.tile(raw.reshape(1, rb), (rows, 1))       # every row identical: all logits tie
    rng = np.random.default_rng(6)
    x = activations(rng, 3, k)
    w = _rt().HipWeight.upload(full, om.TYPE_Q6_K, rows, k)
    tok, _ = _rt().output_argmax(w, _t(x, cuda))
    assert tok.cpu().numpy().tolist() == [0, 0, 0]
    # the maximum row repeated at rows 1500, 700 and 1999: the smallest wins
    raw2, deq2 = _q6k(rows, k, seed=7)
    x1 = activations(rng, 1, k)
    r_best = int(np.argmax(om.matvec_f64(deq2, x1)[0]))
    rows2 = raw2.reshape(rows, rb).copy()
    for r in (1500, 700, 1999):
        rows2[r] = rows2[r_best]
    w2 = _rt().HipWeight.upload(rows2, om.TYPE_Q6_K, rows, k)
    tok2, _ = _rt().output_argmax(w2, _t(x1, cuda))
    assert int(tok2.cpu()[0]) == min(r_best, 700)


def test_argmax_nan_input_never_chosen(cuda):
    raw, _ = _q6k(300, 4096, seed=8)
    x = np.full((2, 4096), np.nan, dtype=np.float32)
    w = _rt().HipWeight.upload(raw, om.TYPE_Q6_K, 300, 4096)
    tok, lg = _rt().output_argmax(w, _t(x, cuda))
    assert tok.cpu().numpy().view(np.uint32).tolist() == [0xFFFFFFFF, 0xFFFFFFFF]
    assert np.all(np.isneginf(lg.cpu().numpy()))


@pytest.mark.parametrize("nb", [1, 4])
def test_argmax_gf4_against_fp64(cuda, nb):
    rows, k = 3000, 4096
    raw, deq = _weight("gf4", rows, k, seed=9)
    rng = np.random.default_rng(10)
    x = activations(rng, nb, k)
    w = _rt().HipWeight.upload(raw, om.TYPE_GF4, rows, k)
    tok, lg = _rt().output_argmax(w, _t(x, cuda))
    ref = om.matvec_f64(deq, x)
    scale = np.linalg.norm(ref, axis=1) / np.sqrt(rows)
    for b in range(nb):
        t = int(tok.cpu()[b])
        assert ref[b, t] >= ref[b].max() - GEMV_REL_L2 * scale[b]
        assert abs(float(lg.cpu()[b]) - ref[b, t]) <= GEMV_REL_L2 * scale[b]


def test_argmax_large_ragged_head(cuda):
    """A 65549 x 4096 Q6_K head made on the GPU: the fused head equals the rule
    on the full logits (size-independent property)."""
    import torch

    rt = _rt()
    rows, k = 65549, 4096
    g = torch.Generator(device=cuda)
    g.manual_seed(3)
    src = torch.randn((rows, k), generator=g, device=cuda) * 0.02
    w = rt.quantize_weight(src, om.TYPE_Q6_K)
    del src
    x = torch.randn((2, k), generator=g, device=cuda)
    logits = rt.decode_matvec(w, x).cpu().numpy()
    tok, lg = rt.output_argmax(w, x)
    ids, best = om.argmax_rule(logits)
    assert np.array_equal(tok.cpu().numpy().view(np.uint32), ids)
    assert np.array_equal(_bits(lg.cpu().numpy()), _bits(best))
