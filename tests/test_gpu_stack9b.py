"""Config 5 at its real shapes: the 32-layer Qwen3.5-9B decode-step projection
stack (q8_0 mixers, GF4 FFN, Q4_K head; 217 GEMVs recorded as one plan) at
batch 1 and 8, and its 128-token prefill chunk.  Every layer has its own weights (distinct seeds) and its own
output buffers, so every output of every projection is checked against the
fp64 product of the library's dequantised weights (which the dequantisation
tests pin bit for bit to the oracle), within GEMV_REL_L2; the residual
stream, which every output and down projection adds into, against the fp64
sum of all 64 contributions; and every replay of the plan against the first,
bit for bit.
"""
from __future__ import annotations

import pytest

from oracle import matvec as om
from tests.helpers import GEMV_REL_L2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stack9b(cuda):
    from qwowl35_amd import qwen35

    st = qwen35.ProjectionStack.synthetic(qwen35.QWEN35_9B, seed=11, distinct=True, device=cuda)
    assert st.weight_bytes == qwen35.projection_bytes(st.hp, st.types) == 5_205_131_264
    return st


def _deq64(w, rows_per_block=32768):
    """The library's dequantised weight in fp64, [rows, k] (row blocks keep the head's fp32 copy small)."""
    import torch

    from qwowl35_amd import runtime as rt

    if w.rows <= rows_per_block:
        return rt.dequantize(w).double()
    out = torch.empty((w.rows, w.k), dtype=torch.float64, device=w.storage.device)
    for r0 in range(0, w.rows, rows_per_block):
        n = min(rows_per_block, w.rows - r0)
        ids = torch.arange(r0, r0 + n, dtype=torch.int32, device=w.storage.device)
        out[r0:r0 + n] = rt.dequantize(w, ids).double()
    return out


def _rel(got, want):
    return om.rel_l2(got.cpu().numpy(), want.cpu().numpy())


@pytest.mark.parametrize("awq", [True, False])
@pytest.mark.parametrize("nb", [1, 8])
def test_stack9b_every_output(cuda, stack9b, nb, awq):
    import torch

    from qwowl35_amd import qwen35

    hp = stack9b.hp
    gen = torch.Generator(device=cuda)
    gen.manual_seed(100 + nb)
    bufs = qwen35.StepBuffers.make(hp, nb, gen, awq=awq, shared_outputs=False)
    act0 = bufs.act.clone()
    plan = qwen35.build_plan(stack9b, bufs)
    assert len(plan) == qwen35.gemv_count(hp) == 217
    print(f"stack9b nb={nb} awq={awq}: launching the recorded plan", flush=True)
    plan.launch()
    torch.cuda.synchronize()
    first = {"act": bufs.act.clone(), "logits": bufs.logits.clone(),
             "ffn_act": [a.clone() for a in bufs.ffn_act]}

    x = bufs.norm.double().T
    fx = (bufs.ffn_norm.double() * (bufs.awq.double() if awq else 1.0)).T
    want_act = act0.double().clone()
    worst = 0.0
    for il, ws in enumerate(stack9b.layers):
        mix = qwen35.mixer_projections(hp, il)
        for p in mix[:-1]:
            want = (_deq64(ws[p.name]) @ x).T
            e = _rel(bufs.mixer_out[il][p.name], want)
            worst = max(worst, e)
            assert e <= GEMV_REL_L2, (il, p.name, e)
        out = mix[-1]
        want_act += (_deq64(ws[out.name]) @ bufs.core[out.k].double().T).T
        gate = _deq64(ws["ffn_gate"]) @ fx
        up = _deq64(ws["ffn_up"]) @ fx
        want_g = (gate / (1.0 + torch.exp(-gate)) * up).T
        e = _rel(bufs.ffn_act[il], want_g)
        worst = max(worst, e)
        assert e <= GEMV_REL_L2, (il, "ffn_gate_up_swiglu", e)
        # the down projection reads the SwiGLU output the plan produced
        want_act += (_deq64(ws["ffn_down"]) @ bufs.ffn_act[il].double().T).T
    e = _rel(bufs.act, want_act)
    assert e <= GEMV_REL_L2, ("residual stream", e)
    want_logits = (_deq64(stack9b.head) @ x).T
    e_head = _rel(bufs.logits, want_logits)
    assert e_head <= GEMV_REL_L2, ("output.weight", e_head)
    print(f"stack9b nb={nb}: worst projection rel-L2 {worst:.2e}, head {e_head:.2e}", flush=True)

    # replays: the residual stream restored, outputs poisoned in between
    for rep in range(2):
        bufs.act.copy_(act0)
        bufs.logits.fill_(float("nan"))
        for a in bufs.ffn_act:
            a.fill_(float("nan"))
        plan.launch()
        torch.cuda.synchronize()
        assert torch.equal(bufs.act, first["act"]), rep
        assert torch.equal(bufs.logits, first["logits"]), rep
        for il, a in enumerate(bufs.ffn_act):
            assert torch.equal(a, first["ffn_act"][il]), (rep, il)
    plan.close()


@pytest.mark.parametrize("n", [128, 48, 192])
def test_stack9b_chunk_every_output(cuda, stack9b, n):
    """Prefill chunks of the same stack (qwen35.build_chunk_plan: fp32
    activations on the prefill matmul, each layer's mixer input projections as
    one merged launch, gate/up/SwiGLU as one fused launch -- on the gate's own
    tile at 128 tokens, on tiles of its own at 48 and 192 -- the head on the
    last token): every projection output, the residual stream and the last
    token's logits against fp64 on the dequantised weights within
    GEMV_REL_L2, and two replays bit for bit."""
    import torch

    from qwowl35_amd import qwen35

    hp = stack9b.hp
    gen = torch.Generator(device=cuda)
    gen.manual_seed(300 + n)
    bufs = qwen35.StepBuffers.make(hp, n, gen, awq=True, shared_outputs=False)
    act0 = bufs.act.clone()
    ws = qwen35.chunk_workspace(stack9b, n)
    plan = qwen35.build_chunk_plan(stack9b, bufs, ws)
    print(f"stack9b chunk n={n}: launching the recorded chunk plan", flush=True)
    plan.launch()
    torch.cuda.synchronize()
    first = {"act": bufs.act.clone(), "logits": bufs.logits[0:1].clone(),
             "mix": [{k: v.clone() for k, v in d.items()} for d in bufs.mixer_out],
             "ffn_act": [a.clone() for a in bufs.ffn_act]}

    x = bufs.norm.double().T
    fx = (bufs.ffn_norm.double() * bufs.awq.double()).T
    want_act = act0.double().clone()
    worst = 0.0
    for il, layer in enumerate(stack9b.layers):
        mix = qwen35.mixer_projections(hp, il)
        for p in mix[:-1]:
            e = _rel(bufs.mixer_out[il][p.name], (_deq64(layer[p.name]) @ x).T)
            worst = max(worst, e)
            assert e <= GEMV_REL_L2, (il, p.name, e)
        out = mix[-1]
        want_act += (_deq64(layer[out.name]) @ bufs.core[out.k].double().T).T
        gate = _deq64(layer["ffn_gate"]) @ fx
        up = _deq64(layer["ffn_up"]) @ fx
        e = _rel(bufs.ffn_act[il], (gate / (1.0 + torch.exp(-gate)) * up).T)
        worst = max(worst, e)
        assert e <= GEMV_REL_L2, (il, "ffn_gate_up_swiglu", e)
        want_act += (_deq64(layer["ffn_down"]) @ bufs.ffn_act[il].double().T).T
    e = _rel(bufs.act, want_act)
    assert e <= GEMV_REL_L2, ("residual stream", e)
    e_head = _rel(bufs.logits[0:1], (_deq64(stack9b.head) @ x[:, n - 1:n]).T)
    assert e_head <= GEMV_REL_L2, ("output.weight", e_head)
    print(f"stack9b chunk: worst projection rel-L2 {worst:.2e}, residual {e:.2e}, head {e_head:.2e}", flush=True)

    for rep in range(2):
        bufs.act.copy_(act0)
        bufs.logits.fill_(float("nan"))
        for d in bufs.mixer_out:
            for v in d.values():
                v.fill_(float("nan"))
        for a in bufs.ffn_act:
            a.fill_(float("nan"))
        plan.launch()
        torch.cuda.synchronize()
        assert torch.equal(bufs.act, first["act"]), rep
        assert torch.equal(bufs.logits[0:1], first["logits"]), rep
        for il in range(hp.transformer_layers):
            assert torch.equal(bufs.ffn_act[il], first["ffn_act"][il]), (rep, il)
            for k, v in bufs.mixer_out[il].items():
                assert torch.equal(v, first["mix"][il][k]), (rep, il, k)
    plan.close()


def test_stack9b_shared_buffers_match_distinct(cuda, stack9b):
    """The benchmark's form (one set of mixer / FFN output buffers reused by
    every layer, as the reference runtime does) gives the same residual stream
    and logits as the checked form above, bit for bit."""
    import torch

    from qwowl35_amd import qwen35

    hp = stack9b.hp
    res = []
    for shared in (False, True):
        gen = torch.Generator(device=cuda)
        gen.manual_seed(7)
        bufs = qwen35.StepBuffers.make(hp, 2, gen, awq=True, shared_outputs=shared)
        plan = qwen35.build_plan(stack9b, bufs)
        plan.launch()
        torch.cuda.synchronize()
        res.append((bufs.act.clone(), bufs.logits.clone(), bufs.ffn_act[-1].clone()))
        plan.close()
    for a, b in zip(*res):
        assert torch.equal(a, b)



def test_stack9b_dequant_pinned_to_oracle(cuda, stack9b):
    """The dequantisation the checks above use is the oracle's at the stack's
    real shapes: for the 248320-row Q4_K head and one weight of every other
    shape (q8_0 mixers, GF4 gate / up / down), the first and last 1024 rows
    and every 61st row, bit for bit against the oracle on the same bytes."""
    from tests.helpers import assert_dequant_pinned, pinned_rows

    seen = set()
    for il, layer in enumerate(stack9b.layers):
        for name, w in layer.items():
            key = (w.type_id, w.rows, w.k)
            if key in seen:
                continue
            seen.add(key)
            print(f"dequant pin blk.{il}.{name} {w.rows}x{w.k}", flush=True)
            assert_dequant_pinned(w, pinned_rows(w.rows))
    want = {(w.type_id, w.rows, w.k) for layer in stack9b.layers for w in layer.values()}
    assert seen == want and len(want) == 6  # q8_0 8192 / 4096 / 32 / 1024 rows x 4096; GF4 gate/up and down
    print("dequant pin output.weight", flush=True)
    assert_dequant_pinned(stack9b.head, pinned_rows(stack9b.head.rows))
