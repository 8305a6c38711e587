"""GPU parity of q8_0 rows whose length is a multiple of 32 columns but not of
256 (k = 32, 96, 4160, 12320), which the reference decodes through
n_blocks = ceil(k / 32) (qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:240;
qw35_decode_matmul_q8_0{,_residual}_f32, qw35_matvec.metal:630-683).

Such a row is only 2-byte aligned, so the decode GEMV runs the row-wise kernel
q8_gemv_rows (one wave per row, fp32 FMAs) instead of the chunked MFMA kernel.
Bars: within GEMV_REL_L2 of the fp64 matvec of the oracle-dequantised weights,
as every decode GEMV; a merged plan launch equals each segment's own call bit
for bit; the prefill matmul and greedy head refuse such a k."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import GEMV_REL_L2, activations, awq_scales, make_weight

pytestmark = pytest.mark.gpu

T = om.TYPE_Q8_0


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


@pytest.mark.parametrize("k", [32, 96, 4160, 12320])
@pytest.mark.parametrize("nb", [1, 3, 8])
def test_q8_0_any_k_gemv(cuda, k, nb):
    import torch

    rt = _rt()
    rows = 37  # ragged: the last workgroup holds one row
    print(f"q8_0 rows {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(k + 7 * nb)
    raw, deq = make_weight(T, rows, k, seed=k + rows)
    w = rt.HipWeight.upload(raw, T, rows, k)
    info = rt.gemv_kernel(w, nb)
    assert info["name"].startswith("q8_gemv_rows<"), info["name"]
    x = activations(rng, nb, k)
    y = rt.decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2
    # AWQ + residual; a workspace passed in is not used (no K-split here)
    a = awq_scales(rng, k)
    base = rng.standard_normal((nb, rows)).astype(np.float32)
    dst = torch.from_numpy(base.copy()).to(cuda)
    ws = rt.decode_matvec_workspace(w, nb, device=cuda)
    rt.decode_matvec(w, _t(x, cuda), dst=dst, residual=True, awq=_t(a, cuda), workspace=ws)
    want = base.astype(np.float64) + om.matvec_f64(deq, x, a)
    assert om.rel_l2(dst.cpu().numpy(), want) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [1, 8])
def test_q8_0_any_k_longest_row(cuda, nb):
    """k = 65504 (2047 blocks, the longest such row under the ABI's 65536):
    each lane walks 32 blocks, the last lanes 31."""
    rt = _rt()
    rows, k = 9, 65504
    print(f"q8_0 rows {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(nb)
    raw, deq = make_weight(T, rows, k, seed=5)
    w = rt.HipWeight.upload(raw, T, rows, k)
    assert rt.gemv_kernel(w, nb)["name"].startswith("q8_gemv_rows<")
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    y = rt.decode_matvec(w, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x, a)) <= GEMV_REL_L2


@pytest.mark.parametrize("k", [96, 4160])
@pytest.mark.parametrize("nb", [1, 8])
def test_q8_0_any_k_swiglu(cuda, k, nb):
    rt = _rt()
    rows = 70
    print(f"q8_0 rows swiglu {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(3 * k + nb)
    rg, dg = make_weight(T, rows, k, seed=11)
    ru, du = make_weight(T, rows, k, seed=12)
    g = rt.HipWeight.upload(rg, T, rows, k)
    u = rt.HipWeight.upload(ru, T, rows, k)
    assert rt.gemv_kernel(g, nb, w_up=u, awq=True)["name"].startswith("q8_gemv_rows<")
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    y = rt.ffn_gate_up_swiglu(g, u, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.swiglu_f64(dg, du, x, a)) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [1, 5])
def test_q8_0_any_k_plan_merge(cuda, nb):
    """Matvecs over one input with k % 256 != 0 merge into one row-wise launch;
    every segment equals its own single call bit for bit (the same kernel sums
    in the same order), replayed twice."""
    import torch

    rt = _rt()
    k = 4160
    rows = [33, 8, 61]
    print(f"q8_0 rows plan merge k={k} nb={nb}", flush=True)
    rng = np.random.default_rng(50 + nb)
    ws = [rt.HipWeight.upload(make_weight(T, r, k, seed=200 + i)[0], T, r, k, device=cuda)
          for i, r in enumerate(rows)]
    x = _t(activations(rng, nb, k), cuda)
    awq = _t(awq_scales(rng, k), cuda)
    outs = [torch.full((nb, r), float("nan"), dtype=torch.float32, device=cuda) for r in rows]
    want = [rt.decode_matvec(w, x, awq=awq) for w in ws]
    plan = rt.DecodePlan()
    for w, o in zip(ws, outs):
        plan.matvec(w, x, o, awq=awq)
    plan.record()
    assert len(plan) == 3  # ops recorded (the three share one launch)
    for _ in range(2):
        for o in outs:
            o.fill_(float("nan"))
        plan.launch()
        torch.cuda.synchronize()
        for o, wv in zip(outs, want):
            assert torch.equal(o, wv)
    plan.close()


def test_q8_0_any_k_matvec_batch(cuda):
    """A 20-token chunk of a k % 256 != 0 weight runs as 8-token GEMVs."""
    rt = _rt()
    rows, k, n = 45, 4160, 20
    print(f"q8_0 rows matvec_batch {rows}x{k} n={n}", flush=True)
    rng = np.random.default_rng(9)
    raw, deq = make_weight(T, rows, k, seed=21)
    w = rt.HipWeight.upload(raw, T, rows, k)
    x = activations(rng, n, k)
    y = rt.matvec_batch(w, _t(x, cuda)).cpu().numpy()
    assert y.shape == (n, rows)
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


def test_q8_0_any_k_chunked_paths_refuse(cuda):
    import torch

    rt = _rt()
    rows, k = 16, 4160
    raw, _ = make_weight(T, rows, k, seed=1)
    w = rt.HipWeight.upload(raw, T, rows, k)
    x = torch.zeros((1, k), dtype=torch.float32, device=cuda)
    with pytest.raises(rt.Qw35Error, match="needs k % 256 == 0"):
        rt.output_argmax(w, x)
    a = torch.zeros((16, k), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(rt.Qw35Error, match="needs k % 256 == 0"):
        rt.matmul_prefill(w, a)
