"""Parity at the Qwen3.5-9B shapes, one test per launch plan the decode stack
and the benchmark use (the planners pick the kernel shape from rows, k and
batch, so small matrices do not reach them):

* q8_0 at 8192 x 4096, 12288 x 4096, 4096 x 12288 and the 12352-row merged
  DeltaNet mixer (qkv + gate + beta + alpha), batch 1, 2 and 8;
* GF4 fused gate/up/SwiGLU at 12288 x 4096 and GF4 down at 4096 x 12288,
  with AWQ, batch 1, 2, 4 and 8;
* Q6_K / Q4_K / Q5_K / GF2 / q8_0 LM-head-sized matrices (65549 rows) at batch
  1, 4 and 8, and the fused greedy head on each (token and logit bit for bit
  equal to the reference's rule applied to the GEMV's logits);
* the block-diagonal GF4 form (batch 1-2) with outlier activation channels,
  and every kernel family with activation magnitudes from 1e-12 to 1e12.

Weights are encoded on the GPU by the library's encoders (bit-identical to
the oracle's, tests/test_gpu_encode.py); the reference values are the oracle's
dequantisation of those bytes (checked bit for bit against the library's) and
an fp64 matvec on the host, within GEMV_REL_L2.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import gf4 as ogf4
from oracle import matvec as om
from tests.helpers import GEMV_REL_L2, TYPES

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _gpu_weight(cuda, type_id, rows, k, seed, std=0.02):
    """(HipWeight, raw bytes on the host) encoded on the GPU from N(0, std)."""
    from qwowl35_amd import qwen35

    import torch

    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    w = qwen35.synthetic_weight(g, type_id, rows, k, std=std)
    return w, w.storage.cpu().numpy()


def _oracle_deq(cuda, w, raw):
    """The oracle's dequantisation of the weight's bytes, checked bit for bit
    against the library's."""
    deq = om.dequant(w.type_id, raw, w.rows, w.k)
    got = _rt().dequantize(w).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))
    return deq


def _x(seed, nb, k):
    return np.random.default_rng(seed).standard_normal((nb, k), dtype=np.float32)


@pytest.mark.parametrize("nb", [1, 2, 8])
@pytest.mark.parametrize("rows,k", [(8192, 4096), (12288, 4096), (4096, 12288)])
def test_q8_0_projection_shapes(cuda, rows, k, nb):
    print(f"q8_0 {rows}x{k} b{nb}", flush=True)
    w, raw = _gpu_weight(cuda, om.TYPE_Q8_0, rows, k, seed=rows + k)
    deq = _oracle_deq(cuda, w, raw)
    x = _x(nb, nb, k)
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [1, 8])
def test_q8_0_merged_delta_mixer(cuda, nb):
    """The 9B DeltaNet mixer's four input projections (8192 + 4096 + 32 + 32 =
    12352 rows over one input) as one merged plan launch (planned for 12352
    rows, so not necessarily the launch shape of each single call), each
    output against the oracle."""
    import torch

    rt = _rt()
    shapes = [8192, 4096, 32, 32]
    ws = [_gpu_weight(cuda, om.TYPE_Q8_0, r, 4096, seed=50 + i) for i, r in enumerate(shapes)]
    x = _x(7 + nb, nb, 4096)
    xt = _t(x, cuda)
    outs = [torch.full((nb, r), float("nan"), dtype=torch.float32, device=cuda) for r in shapes]
    plan = rt.DecodePlan()
    for (w, _), o in zip(ws, outs):
        plan.matvec(w, xt, o)
    plan.record()
    plan.launch()
    torch.cuda.synchronize()
    for (w, raw), o in zip(ws, outs):
        deq = _oracle_deq(cuda, w, raw)
        assert om.rel_l2(o.cpu().numpy(), om.matvec_f64(deq, x)) <= GEMV_REL_L2
    plan.close()


@pytest.fixture(scope="module")
def gf4_ffn(cuda):
    """GF4 gate / up 12288 x 4096 and down 4096 x 12288 packed by the oracle's
    packer (pack_gf4_prepared) from bf16 N(0, 0.02), AWQ columns U(0.5, 2)."""
    rng = np.random.default_rng(77)
    out = {}
    for name, rows, k in (("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)):
        w = om.bf16_round((rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02)))
        words = ogf4.gf4_pack(w)
        out[name] = (_rt().HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, rows, k, device=cuda),
                     ogf4.gf4_dequant(words))
    return out


@pytest.mark.parametrize("nb", [1, 2, 4, 8])
def test_gf4_gate_up_swiglu_12288(cuda, gf4_ffn, nb):
    print(f"gf4 gate/up 12288x4096 b{nb}", flush=True)
    rng = np.random.default_rng(300 + nb)
    x = rng.standard_normal((nb, 4096), dtype=np.float32)
    a = rng.uniform(0.5, 2.0, 4096).astype(np.float32)
    (g, dg), (u, du) = gf4_ffn["gate"], gf4_ffn["up"]
    y = _rt().ffn_gate_up_swiglu(g, u, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.swiglu_f64(dg, du, x, a)) <= GEMV_REL_L2


@pytest.mark.parametrize("awq", [True, False])
@pytest.mark.parametrize("nb", [1, 2, 4, 8])
def test_gf4_down_residual_4096x12288(cuda, gf4_ffn, nb, awq):
    import torch

    rng = np.random.default_rng(400 + nb)
    x = rng.standard_normal((nb, 12288), dtype=np.float32)
    a = rng.uniform(0.5, 2.0, 12288).astype(np.float32) if awq else None
    base = rng.standard_normal((nb, 4096)).astype(np.float32)
    w, deq = gf4_ffn["down"]
    dst = torch.from_numpy(base.copy()).to(cuda)
    _rt().decode_matvec(w, _t(x, cuda), dst=dst, residual=True, awq=_t(a, cuda) if awq else None)
    want = base.astype(np.float64) + om.matvec_f64(deq, x, a)
    assert om.rel_l2(dst.cpu().numpy(), want) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [1, 2, 4, 8])
def test_gf4_plain_12288x4096(cuda, gf4_ffn, nb):
    """The GF4 12288 x 4096 GEMV without SwiGLU or AWQ (config 1 and its batches)."""
    rng = np.random.default_rng(450 + nb)
    x = rng.standard_normal((nb, 4096), dtype=np.float32)
    w, deq = gf4_ffn["gate"]
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


def _outlier_x(rng, nb, k, frac=0.01, gain=100.0):
    x = rng.standard_normal((nb, k), dtype=np.float32)
    ch = rng.choice(k, size=max(1, int(frac * k)), replace=False)
    x[:, ch] *= np.float32(gain)
    return x


@pytest.mark.parametrize("nb", [1, 2])
@pytest.mark.parametrize("which", ["gate", "down"])
def test_gf4_block_diagonal_outlier_channels(cuda, gf4_ffn, which, nb):
    """The block-diagonal GF4 form (batch 1-2) subtracts the MFMA's biased
    partials from per-word bias sums ~1028 |x|; 1% of the channels at 100x
    the others (post-norm outliers, what AWQ exists for) must stay within the
    bar overall and, per row, within 1e-3 of the Cauchy-Schwarz size
    ||W_r|| ||awq * x||."""
    w, deq = gf4_ffn[which]
    rng = np.random.default_rng(500 + nb)
    x = _outlier_x(rng, nb, w.k)
    a = rng.uniform(0.5, 2.0, w.k).astype(np.float32)
    y = _rt().decode_matvec(w, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy().astype(np.float64)
    want = om.matvec_f64(deq, x, a)
    assert om.rel_l2(y, want) <= GEMV_REL_L2
    wn = np.linalg.norm(deq.astype(np.float64), axis=1)
    xn = np.linalg.norm(x.astype(np.float64) * a.astype(np.float64), axis=1)
    bound = 1e-3 * wn[None, :] * xn[:, None]
    assert np.all(np.abs(y - want) <= bound)


@pytest.mark.parametrize("name", ["gf4", "gf2", "q8_0", "q4_k", "q5_k", "q6_k"])
@pytest.mark.parametrize("nb", [1, 2, 8])
def test_extreme_activation_magnitudes(cuda, name, nb):
    """Activations scaled by 1e-12 .. 1e12: the per-chunk power-of-two
    staging must neither overflow fp16 nor fall into its subnormals."""
    type_id = TYPES[name]
    rows, k = 48, 4096
    w, raw = _gpu_weight(cuda, type_id, rows, k, seed=9)
    deq = om.dequant(type_id, raw, rows, k)
    rng = np.random.default_rng(60 + nb)
    for mag in (1e-12, 1e-6, 1e6, 1e12):
        x = rng.standard_normal((nb, k), dtype=np.float32) * np.float32(mag)
        y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
        assert np.all(np.isfinite(y)), mag
        assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2, mag


# k = 12288 on at most 256 row tiles splits; k = 4096 takes the workspace and ignores it
SPLIT_CASES = [("gf4", 4096, 12288), ("q4_k", 4096, 12288), ("q8_0", 4096, 12288), ("q6_k", 4000, 12288),
               ("q5_k", 1000, 12288), ("gf2", 4096, 12288), ("gf4", 2072, 12288), ("q8_0", 4096, 4096)]


@pytest.mark.parametrize("nb", [4, 5, 8])
@pytest.mark.parametrize("name,rows,k", SPLIT_CASES)
def test_k_split_workspace(cuda, name, rows, k, nb):
    """The K-split launch (batch 3..8, k = 12288, at most 256 row tiles, with a workspace):
    each workgroup sums one K slice, the last of a row group adds the partials
    in a fixed order.  Against the oracle (with AWQ and the residual add), equal
    on 12 repeated calls bit for bit (no dependence on which workgroup finishes
    last; the counters return to zero), and within the bar of the unsplit call;
    the same workspace then serves a second shape."""
    import torch

    rt = _rt()
    print(f"k-split {name} {rows}x{k} b{nb}", flush=True)
    w, raw = _gpu_weight(cuda, TYPES[name], rows, k, seed=rows + k + nb)
    assert (rt.gemv_kernel(w, nb, workspace=True)["workspace_bytes"] > 0) == (k == 12288)
    deq = _oracle_deq(cuda, w, raw)
    rng = np.random.default_rng(700 + nb)
    x = rng.standard_normal((nb, k), dtype=np.float32)
    a = rng.uniform(0.5, 2.0, k).astype(np.float32)
    base = rng.standard_normal((nb, rows)).astype(np.float32)
    ws = rt.decode_matvec_workspace(w, nb, device=cuda)
    xt, at, bt = _t(x, cuda), _t(a, cuda), _t(base, cuda)
    first = None
    for _ in range(12):
        dst = bt.clone()
        rt.decode_matvec(w, xt, dst=dst, residual=True, awq=at, workspace=ws)
        if first is None:
            first = dst
        else:
            assert torch.equal(dst, first)
    want = base.astype(np.float64) + om.matvec_f64(deq, x, a)
    assert om.rel_l2(first.cpu().numpy(), want) <= GEMV_REL_L2
    plain = rt.decode_matvec(w, xt, dst=bt.clone(), residual=True, awq=at)
    assert om.rel_l2(first.cpu().numpy(), plain.double().cpu().numpy()) <= GEMV_REL_L2
    # the same workspace for another split shape right after (16 row groups)
    w2, raw2 = _gpu_weight(cuda, TYPES["gf4"], 1000, 12288, seed=5)
    need = rt.gemv_kernel(w2, nb, workspace=True)["workspace_bytes"]
    assert need > 0
    x2 = rng.standard_normal((nb, 12288), dtype=np.float32)
    y2 = rt.decode_matvec(w2, _t(x2, cuda), workspace=ws if ws is not None and ws.numel() >= need else
                          rt.decode_matvec_workspace(w2, nb, device=cuda))
    assert om.rel_l2(y2.cpu().numpy(), om.matvec_f64(om.dequant(w2.type_id, raw2, 1000, 12288), x2)) \
        <= GEMV_REL_L2


HEAD_ROWS = 65549  # > 4096 row tiles: the LM-head launch plans, ragged last tile


@pytest.fixture(scope="module")
def heads(cuda):
    """LM-head-sized weights (65549 x 4096) of every k-quant codec and GF2, made on the GPU."""
    out = {}
    for i, name in enumerate(("q8_0", "q4_k", "q5_k", "q6_k", "gf2")):
        out[name] = _gpu_weight(cuda, TYPES[name], HEAD_ROWS, 4096, seed=900 + i)[0]
    return out


def _deq64(w):
    return _rt().dequantize(w).double()


@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q5_k", "q6_k", "gf2"])
def test_head_dequant_pinned_to_oracle(cuda, heads, name):
    """The dequantisation the head checks use is the oracle's on these
    65549-row weights: the first and last 1024 rows and every 61st row, bit
    for bit against the oracle on the same bytes."""
    from tests.helpers import assert_dequant_pinned, pinned_rows

    assert_dequant_pinned(heads[name], pinned_rows(HEAD_ROWS))


@pytest.mark.parametrize("nb", [1, 4, 8])
@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q5_k", "q6_k", "gf2"])
def test_head_sized_gemv(cuda, heads, name, nb):
    """The LM-head plans against fp64 on the library's dequantised weights
    (pinned bit for bit to the oracle by the dequantisation tests)."""
    import torch

    w = heads[name]
    g = torch.Generator(device=cuda)
    g.manual_seed(nb)
    x = torch.randn((nb, 4096), generator=g, device=cuda)
    y = _rt().decode_matvec(w, x).double()
    want = (_deq64(w) @ x.double().T).T
    assert om.rel_l2(y.cpu().numpy(), want.cpu().numpy()) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [1, 4, 8])
@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q5_k", "q6_k", "gf2"])
def test_greedy_head_plans(cuda, heads, name, nb):
    """The fused greedy head on the LM-head plans (several row tiles per
    workgroup, waves covering several batch rows, the partial-workspace size):
    token and logit bit for bit the reference rule on decode_matvec's logits."""
    import torch

    w = heads[name]
    g = torch.Generator(device=cuda)
    g.manual_seed(20 + nb)
    x = torch.randn((nb, 4096), generator=g, device=cuda)
    awq = torch.rand((4096,), generator=g, device=cuda) * 1.5 + 0.5
    logits = _rt().decode_matvec(w, x, awq=awq).cpu().numpy()
    tok, lg = _rt().output_argmax(w, x, awq=awq)
    ids, best = om.argmax_rule(logits)
    assert np.array_equal(tok.cpu().numpy().view(np.uint32), ids)
    assert np.array_equal(lg.cpu().numpy().view(np.uint32), best.view(np.uint32))
