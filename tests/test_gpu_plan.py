"""Decode-step plans (qw35_hip_plan_*): a recorded hipGraph of projection GEMVs
must reproduce, bit for bit, the same calls made one by one, on every replay,
with the caller's eager work between replays, and must read inputs that were
updated in place since it was recorded."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import GEMV_REL_L2, TYPES, make_weight

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _layer(cuda, nb, seed):
    """One miniature decoder layer: q8_0 projection, GF4 gate/up SwiGLU with
    AWQ, GF4 down with residual, Q4_K head."""
    import torch

    rt = _rt()
    rng = np.random.default_rng(seed)
    k, f, v = 1024, 512, 768
    spec = {
        "proj": (TYPES["q8_0"], k, k),
        "gate": (TYPES["gf4"], f, k),
        "up": (TYPES["gf4"], f, k),
        "down": (TYPES["gf4"], k, f),
        "head": (TYPES["q4_k"], v, k),
    }
    ws, deq = {}, {}
    for i, (name, (t, rows, kk)) in enumerate(spec.items()):
        raw, d = make_weight(t, rows, kk, seed=seed * 10 + i, std=0.05)
        ws[name] = rt.HipWeight.upload(raw, t, rows, kk, device=cuda)
        deq[name] = d
    bufs = {
        "x": _t(rng.standard_normal((nb, k), dtype=np.float32), cuda),
        "awq": _t(rng.uniform(0.5, 2, k).astype(np.float32), cuda),
        "h": torch.zeros((nb, k), dtype=torch.float32, device=cuda),
        "g": torch.zeros((nb, f), dtype=torch.float32, device=cuda),
        "res": _t(rng.standard_normal((nb, k), dtype=np.float32), cuda),
        "logits": torch.zeros((nb, v), dtype=torch.float32, device=cuda),
    }
    return ws, deq, bufs


def _eager(ws, b, res0):
    rt = _rt()
    b["res"].copy_(res0)
    rt.decode_matvec(ws["proj"], b["x"], b["h"])
    rt.ffn_gate_up_swiglu(ws["gate"], ws["up"], b["h"], b["g"], awq=b["awq"])
    rt.decode_matvec(ws["down"], b["g"], b["res"], residual=True)
    rt.decode_matvec(ws["head"], b["res"], b["logits"])


def _plan(ws, b):
    return (_rt().DecodePlan()
            .matvec(ws["proj"], b["x"], b["h"])
            .swiglu(ws["gate"], ws["up"], b["h"], b["g"], awq=b["awq"])
            .matvec(ws["down"], b["g"], b["res"], residual=True)
            .matvec(ws["head"], b["res"], b["logits"])
            .record())


@pytest.mark.parametrize("nb", [1, 3, 8])
def test_plan_replays_match_eager_calls(cuda, nb):
    import torch

    ws, deq, b = _layer(cuda, nb, seed=nb)
    res0 = b["res"].clone()
    _eager(ws, b, res0)
    torch.cuda.synchronize()
    want = {n: b[n].clone() for n in ("h", "g", "res", "logits")}
    plan = _plan(ws, b)
    assert len(plan) == 4
    for rep in range(3):
        for n in ("h", "g", "logits"):
            b[n].fill_(float("nan"))      # eager work between replays
        b["res"].copy_(res0)
        plan.launch()
        torch.cuda.synchronize()
        for n, v in want.items():
            assert torch.equal(b[n], v), (rep, n)
    plan.close()


def test_plan_reads_inputs_updated_in_place(cuda):
    import torch

    ws, deq, b = _layer(cuda, 2, seed=11)
    res0 = b["res"].clone()
    plan = _plan(ws, b)
    rng = np.random.default_rng(5)
    for _ in range(2):
        x = rng.standard_normal((2, 1024), dtype=np.float32)
        b["x"].copy_(_t(x, cuda))
        b["res"].copy_(res0)
        plan.launch()
        torch.cuda.synchronize()
        # the layer in fp64 on the oracle's dequantised weights
        a = b["awq"].cpu().numpy()
        h = om.matvec_f64(deq["proj"], x)
        g = om.swiglu_f64(deq["gate"], deq["up"], b["h"].cpu().numpy(), a)
        assert om.rel_l2(b["h"].cpu().numpy(), h) <= GEMV_REL_L2
        assert om.rel_l2(b["g"].cpu().numpy(), g) <= GEMV_REL_L2
        res = res0.cpu().numpy().astype(np.float64) + om.matvec_f64(deq["down"], b["g"].cpu().numpy())
        assert om.rel_l2(b["res"].cpu().numpy(), res) <= GEMV_REL_L2
        logits = om.matvec_f64(deq["head"], b["res"].cpu().numpy())
        assert om.rel_l2(b["logits"].cpu().numpy(), logits) <= GEMV_REL_L2
    plan.close()


@pytest.mark.parametrize("name", ["gf2", "q8_0", "q4_k", "q5_k", "q6_k"])
@pytest.mark.parametrize("nb", [1, 5])
def test_plan_merges_projections_sharing_inputs(cuda, name, nb):
    """Consecutive k-quant matvecs over one input (a mixer's q/k/v or
    qkv/z/beta/alpha) are recorded as one multi-segment launch; every segment
    must equal its own single call, bit for bit, including ragged row counts."""
    import torch

    rt = _rt()
    t = TYPES[name]
    k = 2048 if name == "q6_k" else 512  # Q6_K: a 7-row matrix is a multiple of 16 bytes at k = 2048
    rng = np.random.default_rng(40 + nb)
    rows = [160, 32, 48, 7, 96]
    ws = [rt.HipWeight.upload(make_weight(t, r, k, seed=100 + i)[0], t, r, k, device=cuda)
          for i, r in enumerate(rows)]
    x = _t(rng.standard_normal((nb, k), dtype=np.float32), cuda)
    awq = _t(rng.uniform(0.5, 2, k).astype(np.float32), cuda)
    outs = [torch.full((nb, r), float("nan"), dtype=torch.float32, device=cuda) for r in rows]
    want = [rt.decode_matvec(w, x, awq=awq) for w in ws]
    plan = rt.DecodePlan()
    for w, o in zip(ws, outs):
        plan.matvec(w, x, o, awq=awq)
    plan.record()
    for _ in range(2):
        for o in outs:
            o.fill_(float("nan"))
        plan.launch()
        torch.cuda.synchronize()
        for o, wv in zip(outs, want):
            assert torch.equal(o, wv)
    plan.close()
