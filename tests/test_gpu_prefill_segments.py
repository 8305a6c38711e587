"""GPU parity of merged prefill launches.  Consecutive MATMUL plan ops over the
same activations -- a mixer's input projections (delta qkv / gate / beta /
alpha, attention q / k / v; the per-layer encodeMatvecBatch calls of
evalTokens, qw35-server/src/metal/bridge/Qw35MetalRuntime.m:1308-1311) -- are
recorded as one prefill launch whose grid holds the weight tiles of all of
them, each segment writing its own output.

* every segment's output passes tests/helpers.py:check_prefill's bars (fp64 of
  the staged operand per element, of the unrounded activations and of the
  exact weights in rel-L2), at ragged token counts, for q8_0, GF4, Q4_K and F16
  weights, with and without AWQ, STORE and ADD epilogues;
* it is within 2^-20 rel-L2 of the single call of the same weight: the same
  fp16 operands and fp32 accumulation, planned for the summed rows, so the K
  split and the association of the partial sums may differ from the single
  call's;
* two replays give the same bits; ops that do not merge (a row count that is
  not a multiple of 4, another weight form, an output that is another op's
  input) still give their single calls' bits.

The gate/up op (MATMUL_SWIGLU) of GF4 weights runs as one launch holding a
gate and an up tile per wave.  Where the gate's planned launch is an unsplit
8-wave tile (K halves, quarters or neither) the fused launch uses that tile
and its output equals, bit for bit, the gate call (STORE) followed by the up
call (SWIGLU epilogue); at other chunk lengths it runs on another tile (or as
those two launches) within 2^-20 rel-L2 of them.
"""
from __future__ import annotations

import re

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import GEMV_REL_L2, activations, awq_scales, check_prefill, make_weight, prefill_rel_l2_bar

pytestmark = pytest.mark.gpu

MERGED_REL_L2 = 2.0 ** -20


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _workspace(ws_list, n, cuda, merged_rows=None):
    """A workspace for the single calls and for the merged launch of merged_rows."""
    import ctypes as C

    import torch

    from qwowl35_amd import _ffi

    lib = _ffi.load()
    size = max(int(lib.qw35_hip_matmul_prefill_workspace_size(C.byref(w.view), n)) for w in ws_list)
    if merged_rows:
        v = _ffi.Weight.from_buffer_copy(ws_list[0].view)
        v.bytes = v.bytes // v.rows * merged_rows
        v.rows = merged_rows
        size = max(size, int(lib.qw35_hip_matmul_prefill_workspace_size(C.byref(v), n)))
    return torch.empty(size, dtype=torch.uint8, device=cuda)


def _run_plan(ws_list, x, outs, workspace, awq=None, residual=False, replays=2):
    import torch

    plan = _rt().DecodePlan()
    for w, o in zip(ws_list, outs):
        plan.matmul(w, x, o, workspace, residual=residual, awq=awq)
    plan.record()
    inits = [o.clone() for o in outs]
    results = []
    for _ in range(replays):
        for o, i in zip(outs, inits):
            o.copy_(i)
        plan.launch()
        torch.cuda.synchronize()
        results.append([o.clone() for o in outs])
    plan.close()
    for r in results[1:]:
        for a, b in zip(r, results[0]):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    return results[0]


CASES = [  # (type name, segment rows, k)
    ("q8_0", [2048, 1024, 32, 32], 1024),
    ("gf4", [1024, 512, 64], 2048),
    ("q4_k", [768, 256, 32, 32], 1024),
    ("f16", [512, 256, 128], 1024),
]


@pytest.mark.parametrize("name,rows,k", CASES)
@pytest.mark.parametrize("n", [9, 64, 128, 300])
@pytest.mark.parametrize("awq_on", [False, True])
def test_merged_mixer_matches_single_calls_and_oracle(cuda, name, rows, k, n, awq_on):
    import torch

    rt = _rt()
    print(f"prefill segments {name} rows={rows} k={k} n={n} awq={awq_on}", flush=True)
    t = {"q8_0": rt.TYPE_Q8_0, "gf4": rt.TYPE_GF4, "q4_k": rt.TYPE_Q4_K, "f16": rt.TYPE_F16}[name]
    rng = np.random.default_rng(n * 13 + len(rows) + awq_on)
    raws, ws_list = [], []
    for i, r in enumerate(rows):
        raw, deq = make_weight(t, r, k, seed=300 + 7 * i + n)
        raws.append((raw, deq))
        ws_list.append(rt.HipWeight.upload(raw, t, r, k, device=cuda))
    x32 = activations(rng, n, k)
    awq = awq_scales(rng, k) if awq_on else None
    x = _t(x32, cuda)
    aw = _t(awq, cuda) if awq is not None else None
    ws = _workspace(ws_list, n, cuda, merged_rows=sum(rows))
    outs = [torch.full((n, r), float("nan"), dtype=torch.float32, device=cuda) for r in rows]
    got = _run_plan(ws_list, x, outs, ws, awq=aw)
    for (raw, deq), w, g, r in zip(raws, ws_list, got, rows):
        single = rt.matmul_prefill(w, x, awq=aw, out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert om.rel_l2(g.cpu().numpy().astype(np.float64), single.cpu().numpy().astype(np.float64)) <= MERGED_REL_L2
        img = om.prefill_image(t, raw, r, k).astype(np.float32) if t != rt.TYPE_GF4 else deq
        check_prefill(g, x32, awq, img, w_exact=deq if t != rt.TYPE_GF4 else None)


def test_merged_residual_epilogue(cuda):
    """Output projections with the ADD epilogue merge too (distinct outputs)."""
    import torch

    rt = _rt()
    t, k, n = rt.TYPE_Q8_0, 2048, 100
    rows = [1024, 512]
    rng = np.random.default_rng(5)
    pairs = [make_weight(t, r, k, seed=50 + r) for r in rows]
    ws_list = [rt.HipWeight.upload(raw, t, r, k, device=cuda) for (raw, _), r in zip(pairs, rows)]
    x32 = activations(rng, n, k)
    x = _t(x32, cuda)
    base = [rng.standard_normal((n, r)).astype(np.float32) for r in rows]
    outs = [_t(b, cuda) for b in base]
    ws = _workspace(ws_list, n, cuda, merged_rows=sum(rows))
    got = _run_plan(ws_list, x, outs, ws, residual=True)
    for (raw, deq), r, g, b in zip(pairs, rows, got, base):
        # the product the launch added to the old values: against the fp16
        # image the kernel contracts and against the exact q8_0 weights
        prod = g.cpu().numpy().astype(np.float64) - b.astype(np.float64)
        img = om.prefill_image(t, raw, r, k).astype(np.float64)
        assert om.rel_l2(prod, om.prefill_f64(img, x32, None)) <= prefill_rel_l2_bar(True, False)
        assert om.rel_l2(prod, om.prefill_f64(deq.astype(np.float64), x32, None)) <= GEMV_REL_L2


def test_ops_that_do_not_merge_keep_their_single_call_bits(cuda):
    """A 30-row op (not a multiple of 4), a GF4 op between q8_0 ops, and an op
    whose output is the next op's input: each runs as its own launch, so every
    output equals its single call bit for bit."""
    import torch

    rt = _rt()
    k, n = 1024, 40
    rng = np.random.default_rng(8)
    q8 = [rt.HipWeight.upload(make_weight(rt.TYPE_Q8_0, r, k, seed=70 + r)[0], rt.TYPE_Q8_0, r, k, device=cuda)
          for r in (512, 30, 256)]
    gf4 = rt.HipWeight.upload(make_weight(rt.TYPE_GF4, 256, k, seed=9)[0], rt.TYPE_GF4, 256, k, device=cuda)
    x = _t(activations(rng, n, k), cuda)
    ws = _workspace(q8 + [gf4], n, cuda)
    seq = [q8[0], q8[1], gf4, q8[2]]
    outs = [torch.empty((n, w.rows), dtype=torch.float32, device=cuda) for w in seq]
    got = _run_plan(seq, x, outs, ws)
    for w, g in zip(seq, got):
        want = rt.matmul_prefill(w, x, out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(g.view(torch.int32), want.view(torch.int32))
    # chained: op 2 reads op 1's output (k = 1024 = rows of op 1)
    w1 = rt.HipWeight.upload(make_weight(rt.TYPE_Q8_0, 1024, k, seed=11)[0], rt.TYPE_Q8_0, 1024, k, device=cuda)
    w2 = rt.HipWeight.upload(make_weight(rt.TYPE_Q8_0, 512, 1024, seed=12)[0], rt.TYPE_Q8_0, 512, 1024, device=cuda)
    mid = torch.empty((n, 1024), dtype=torch.float32, device=cuda)
    fin = torch.empty((n, 512), dtype=torch.float32, device=cuda)
    plan = rt.DecodePlan()
    plan.matmul(w1, x, mid, ws)
    plan.matmul(w2, mid, fin, ws)
    plan.record()
    plan.launch()
    torch.cuda.synchronize()
    plan.close()
    want_mid = rt.matmul_prefill(w1, x, out_dtype=torch.float32, workspace=ws)
    want_fin = rt.matmul_prefill(w2, want_mid, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(mid.view(torch.int32), want_mid.view(torch.int32))
    assert torch.equal(fin.view(torch.int32), want_fin.view(torch.int32))


@pytest.mark.parametrize("n", [128, 256])
def test_merged_delta_mixer_full_size(cuda, n):
    """The 9B's delta-layer mixer (qkv 8192, gate 4096, beta 32, alpha 32 rows
    of q8_0 at k = 4096) as one launch: against the single calls and against
    the oracle on 32 sampled rows of each segment."""
    import torch

    rt = _rt()
    from qwowl35_amd import qwen35

    print(f"prefill segments delta mixer n={n}", flush=True)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(n + 3)
    rows = [8192, 4096, 32, 32]
    k = 4096
    ws_list = [qwen35.synthetic_weight(gen, rt.TYPE_Q8_0, r, k) for r in rows]
    x = torch.randn((n, k), generator=gen, device=cuda)
    ws = _workspace(ws_list, n, cuda, merged_rows=sum(rows))
    outs = [torch.empty((n, r), dtype=torch.float32, device=cuda) for r in rows]
    got = _run_plan(ws_list, x, outs, ws)
    x32 = x.cpu().numpy()
    for w, g, r in zip(ws_list, got, rows):
        single = rt.matmul_prefill(w, x, out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert om.rel_l2(g.cpu().numpy().astype(np.float64), single.cpu().numpy().astype(np.float64)) <= MERGED_REL_L2
        sel = np.random.default_rng(r).choice(r, min(r, 32), replace=False)
        raw = w.storage.cpu().numpy()
        rb = k // 32 * 34
        sub = np.concatenate([raw[i * rb:(i + 1) * rb] for i in sel])
        img = om.prefill_image(rt.TYPE_Q8_0, sub, len(sel), k).astype(np.float32)
        check_prefill(g[:, sel], x32, None, img, w_exact=om.dequant(rt.TYPE_Q8_0, sub, len(sel), k))


@pytest.mark.parametrize("name", ["q8_0", "gf4"])
@pytest.mark.parametrize("room", ["planned", "staging_only"])
def test_more_mergeable_ops_than_segments(cuda, name, room):
    """Six mergeable ops run as launches of at most four segments (four, then
    two), each output within 2^-20 rel-L2 of its single call and passing the
    oracle bars.  With a workspace of only the staging bytes (room for no K
    split, less than a merged launch would plan) the launches run unsplit and
    give the same results."""
    import torch

    rt = _rt()
    t = {"q8_0": rt.TYPE_Q8_0, "gf4": rt.TYPE_GF4}[name]
    rows, k, n = [256, 128, 64, 32, 512, 96], 1024, 64
    print(f"prefill segments {name} six ops rows={rows} workspace={room}", flush=True)
    rng = np.random.default_rng(61 + len(name) + len(room))
    raws, ws_list = [], []
    for i, r in enumerate(rows):
        raw, deq = make_weight(t, r, k, seed=900 + 11 * i)
        raws.append((raw, deq))
        ws_list.append(rt.HipWeight.upload(raw, t, r, k, device=cuda))
    x32 = activations(rng, n, k)
    x = _t(x32, cuda)
    if room == "planned":
        ws = _workspace(ws_list, n, cuda, merged_rows=max(sum(rows[:4]), sum(rows[4:])))
    else:
        staged_rows = 64 * ((n + 31) // 32)  # fp32 tokens: a hi and a lo row each, 32-token groups
        ws = torch.empty((staged_rows * k * 2 + 255) // 256 * 256 + (n * 4 + 255) // 256 * 256, dtype=torch.uint8,
                         device=cuda)
    outs = [torch.full((n, r), float("nan"), dtype=torch.float32, device=cuda) for r in rows]
    got = _run_plan(ws_list, x, outs, ws)
    big = _workspace(ws_list, n, cuda)
    for (raw, deq), w, g, r in zip(raws, ws_list, got, rows):
        single = rt.matmul_prefill(w, x, out_dtype=torch.float32, workspace=big)
        torch.cuda.synchronize()
        assert om.rel_l2(g.cpu().numpy().astype(np.float64), single.cpu().numpy().astype(np.float64)) <= MERGED_REL_L2
        img = om.prefill_image(t, raw, r, k).astype(np.float32) if t != rt.TYPE_GF4 else deq
        check_prefill(g, x32, None, img, w_exact=deq if t != rt.TYPE_GF4 else None)


@pytest.mark.parametrize("rows,k,n", [(12288, 4096, 128), (12288, 4096, 9), (12288, 4096, 32), (12288, 4096, 48),
                                      (1024, 2048, 100), (512, 1024, 40), (2048, 4096, 64), (12288, 4096, 200),
                                      (12288, 4096, 256), (520, 1024, 77), (4096, 4096, 20)])
@pytest.mark.parametrize("awq_on", [False, True])
def test_plan_gate_up_equals_gate_then_up(cuda, rows, k, n, awq_on):
    import torch

    from qwowl35_amd import _ffi

    rt = _rt()
    t = rt.TYPE_GF4
    rng = np.random.default_rng(rows + k + n + awq_on)
    gate = rt.HipWeight.upload(make_weight(t, rows, k, seed=rows + 1)[0], t, rows, k, device=cuda)
    up = rt.HipWeight.upload(make_weight(t, rows, k, seed=rows + 2)[0], t, rows, k, device=cuda)
    x = _t(activations(rng, n, k), cuda)
    aw = _t(awq_scales(rng, k), cuda) if awq_on else None
    desc = rt.prefill_kernel(gate, n, a_dtype=torch.float32, awq=awq_on, out_dtype=torch.float32)
    # the gate launches the plan fuses: unsplit 8-wave tiles of one weight tile per wave, 64 or 128 tokens
    # with K halves or none, 64 tokens with K quarters
    m = re.fullmatch(r"gf4_prefill_f16_kernel<(\d+), (\d+), (\d+), \d+, true, false, false, (\d), false, false>",
                     desc["name"])
    bm, nw, fn, kh = (int(v) for v in m.groups()) if m else (0, 0, 0, 0)
    fused = (desc["splits"] == 1 and nw == 8 and fn == 1 and
             ((kh in (1, 2) and bm in (64, 128)) or (kh == 4 and bm == 64)))
    print(f"gate/up {rows}x{k} n={n} awq={awq_on} gate launch {desc['name']} splits {desc['splits']} "
          f"fused with its tile={fused}", flush=True)
    if (rows, k) == (12288, 4096) and (n <= 32 or 65 <= n <= 128):
        assert fused  # the 9B's FFN at these chunk lengths takes the fused launch of the gate's own tile
    ws = _workspace([gate, up], n, cuda)
    dst = torch.full((n, rows), float("nan"), dtype=torch.float32, device=cuda)
    plan = rt.DecodePlan()
    plan.matmul_swiglu(gate, up, x, dst, ws, awq=aw)
    plan.record()
    outs = []
    for _ in range(2):
        dst.fill_(float("nan"))
        plan.launch()
        torch.cuda.synchronize()
        outs.append(dst.clone())
    plan.close()
    want = rt.matmul_prefill(gate, x, awq=aw, out_dtype=torch.float32, workspace=ws)
    rt.matmul_prefill(up, x, awq=aw, out_dtype=torch.float32, dst=want, workspace=ws, epilogue=_ffi.EPILOGUE_SWIGLU)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    if fused:
        assert torch.equal(outs[0].view(torch.int32), want.view(torch.int32))
    else:
        # the two launches, or the fused launch on another tile (K summed in another grouping)
        got64, want64 = outs[0].cpu().numpy().astype(np.float64), want.cpu().numpy().astype(np.float64)
        assert om.rel_l2(got64, want64) <= MERGED_REL_L2
