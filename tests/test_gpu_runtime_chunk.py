"""The projection runtime's multi-token step (qw35_hip_runtime_eval_chunk): the
projection part of qw35_metal_runtime_eval_tokens (qw35-server/src/metal/
bridge/Qw35FFI.h:97-105; evalTokens, Qw35MetalRuntime.m:1227-1333), on the
synthetic GGUF images of test_gpu_runtime.py (q8_0 mixers, GF4 FFN, Q6_K head)
and on one with Q4_K mixers (dequantised in the kernel) and a Q5_K FFN (fp16
prefill images made by the runtime).

* Chunks of 9, 128 and 256 tokens (the reference server's default chunk is
  128, its maximum 256: qw35-server/src/model.rs:30-31): every output -- the
  last writer of each mixer buffer, the SwiGLU output, the residual stream
  and the last token's logits -- equals, bit for bit, the same sequence of
  calls (qw35_hip_matmul_prefill_epilogue with fp32 activations: SWIGLU for
  ffn_up after ffn_gate's STORE, ADD for the output projections and ffn_down;
  qw35_hip_decode_matvec for the head on the last token; a layer's mixer input
  projections as one plan of MATMUL ops, which records them as one merged
  launch as the runtime does -- tests/test_gpu_prefill_segments.py checks
  that launch against the single calls);
* the same outputs on sampled tokens within 1e-3 relative L2 of fp64 on the
  oracle-dequantised weights (the residual stream as act + sum over layers);
* chunks of up to 8 tokens equal eval_step's projections; the greedy head
  picks the reference rule's token of the FULL logits;
* buffers shared by ops of different row lengths hold each op's rows packed
  at its own length (QKV: attn_q vs attn_qkv; CORE: attn_output vs ssm_out),
  at batch 3 for eval_step and at 40 tokens for eval_chunk.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import GEMV_REL_L2
from tests.test_gpu_runtime import _hp, _image

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(cuda):
    from qwowl35_amd import qwen35

    stack = qwen35.ProjectionStack.synthetic(_hp(), qwen35.StackTypes(head=14), seed=5, distinct=True, device=cuda)
    return stack, _image(stack)


def _inputs(cuda, hp, n, core_k, seed):
    import torch

    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    norm = torch.randn((n, hp.embedding_length), generator=g, device=cuda)
    core = torch.randn((n, core_k), generator=g, device=cuda)
    act = torch.randn((n, hp.embedding_length), generator=g, device=cuda)
    return norm, core, act


def _workspace(stack, n, device):
    """A prefill workspace that holds every projection's planned launch at n
    tokens, the merged mixer launches included."""
    from qwowl35_amd import qwen35

    return qwen35.chunk_workspace(stack, n, device=device)


def _single_calls(stack, n, norm, core, act):
    """The chunk's projections as single calls, in the runtime's order; returns
    (mixer outputs per (layer, name), SwiGLU output of the last layer, act, logits of the last token)."""
    import torch

    from qwowl35_amd import _ffi
    from qwowl35_amd import qwen35
    from qwowl35_amd import runtime as rt

    hp = stack.hp
    f32 = torch.float32
    ws = _workspace(stack, n, norm.device)
    act = act.clone()
    mix = {}
    ffn = torch.empty((n, hp.feed_forward_length), dtype=f32, device=norm.device)
    for il, layer in enumerate(stack.layers):
        projs = qwen35.mixer_projections(hp, il)
        plan = rt.DecodePlan()
        for p in projs[:-1]:
            mix[(il, p.name)] = torch.empty((n, p.rows), dtype=f32, device=norm.device)
            plan.matmul(layer[p.name].prefill, norm, mix[(il, p.name)], ws)
        plan.record()
        plan.launch()
        torch.cuda.synchronize()
        plan.close()
        out = projs[-1]
        rt.matmul_prefill(layer[out.name].prefill, core[:, :out.k].contiguous(), out_dtype=f32, dst=act, workspace=ws,
                          epilogue=_ffi.EPILOGUE_ADD)
        rt.matmul_prefill(layer["ffn_gate"].prefill, norm, out_dtype=f32, dst=ffn, workspace=ws)
        rt.matmul_prefill(layer["ffn_up"].prefill, norm, out_dtype=f32, dst=ffn, workspace=ws,
                          epilogue=_ffi.EPILOGUE_SWIGLU)
        rt.matmul_prefill(layer["ffn_down"].prefill, ffn, out_dtype=f32, dst=act, workspace=ws,
                          epilogue=_ffi.EPILOGUE_ADD)
    logits = rt.decode_matvec(stack.head, norm[n - 1:n].contiguous())
    torch.cuda.synchronize()
    return mix, ffn, act, logits


LAST_WRITERS = (("RT_QKV", 3, "attn_q"), ("RT_K", 3, "attn_k"), ("RT_V", 3, "attn_v"), ("RT_Z", 2, "attn_gate"),
                ("RT_BETA", 2, "ssm_beta"), ("RT_ALPHA", 2, "ssm_alpha"))


def _oracle_rows(stack, rows, norm, core, act):
    """fp64 outputs of the chunk for token rows `rows` on oracle-dequantised weights."""
    from qwowl35_amd import qwen35

    hp = stack.hp

    def deq(w):
        return om.dequant(w.type_id, w.storage.cpu().numpy(), w.rows, w.k).astype(np.float64)

    x = norm.cpu().numpy()[rows].astype(np.float64)
    c = core.cpu().numpy()[rows].astype(np.float64)
    a = act.cpu().numpy()[rows].astype(np.float64)
    mix = {}
    ffn = None
    for il, layer in enumerate(stack.layers):
        projs = qwen35.mixer_projections(hp, il)
        for p in projs[:-1]:
            mix[(il, p.name)] = x @ deq(layer[p.name]).T
        out = projs[-1]
        a = a + c[:, :out.k] @ deq(layer[out.name]).T
        ffn = om.silu_f64(x @ deq(layer["ffn_gate"]).T) * (x @ deq(layer["ffn_up"]).T)
        a = a + ffn @ deq(layer["ffn_down"]).T
    return mix, ffn, a


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


def _check_chunk(r, stack, n, norm, core, act, oracle_rows=8):
    import torch

    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    hp = stack.hp
    r.write(_ffi.RT_NORM, norm)
    r.write(_ffi.RT_CORE, core)
    r.write(_ffi.RT_ACT, act)
    print(f"runtime chunk n={n}", flush=True)
    r.eval_chunk(n, _ffi.LOGITS_FULL)
    logits = r.copy_logits()
    assert tuple(logits.shape) == (1, hp.vocab)
    mix, ffn, act_ref, logits_ref = _single_calls(stack, n, norm, core, act)
    assert np.array_equal(logits.numpy().view(np.uint32), _bits(logits_ref))
    got_act = r.read(_ffi.RT_ACT, n * hp.embedding_length).reshape(n, -1)
    assert np.array_equal(got_act.numpy().view(np.uint32), _bits(act_ref))
    got_ffn = r.read(_ffi.RT_FFN, n * hp.feed_forward_length).reshape(n, -1)
    assert np.array_equal(got_ffn.numpy().view(np.uint32), _bits(ffn))
    got_mix = {}
    for which, il, name in LAST_WRITERS:
        want = mix[(il, name)]
        got = r.read(getattr(_ffi, which), want.numel()).reshape(want.shape)
        assert np.array_equal(got.numpy().view(np.uint32), _bits(want)), name
        got_mix[(il, name)] = got.numpy()
    # sampled tokens against fp64 on the oracle's dequantisation
    rows = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(n).choice(n, min(n, oracle_rows))]))
    o_mix, o_ffn, o_act = _oracle_rows(stack, rows, norm, core, act)
    for _, il, name in LAST_WRITERS:
        assert om.rel_l2(got_mix[(il, name)][rows], o_mix[(il, name)]) <= GEMV_REL_L2, name
    assert om.rel_l2(got_ffn.numpy()[rows], o_ffn) <= GEMV_REL_L2
    assert om.rel_l2(got_act.numpy()[rows], o_act) <= GEMV_REL_L2
    head64 = rt.dequantize(stack.head).double().cpu().numpy()
    assert om.rel_l2(logits.numpy()[0], head64 @ norm.cpu().numpy()[n - 1].astype(np.float64)) <= GEMV_REL_L2
    return logits


def test_chunk_equals_single_calls(cuda, small):
    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    stack, image = small
    hp = stack.hp
    r = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=8, prefill_chunk=256)
    for n in (9, 128, 256, 128):  # the second 128 replays the recorded graph on new inputs
        norm, core, act = _inputs(cuda, hp, n, 1024, seed=n + r.last_batch)
        logits = _check_chunk(r, stack, n, norm, core, act)
        r.write(_ffi.RT_ACT, act)
        r.eval_chunk(n, _ffi.LOGITS_ARGMAX)
        tok, lg = r.argmax()
        ids, best = om.argmax_rule(logits.numpy())
        assert tok == [int(ids[0])] and np.float32(lg[0]).view(np.uint32) == best.view(np.uint32)[0]
    r.close()


def test_short_chunk_runs_the_decode_gemvs(cuda, small):
    """Up to 8 tokens: eval_step's projections; the head on the last token only."""
    import torch

    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    stack, image = small
    hp = stack.hp
    a = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=8)  # prefill_chunk 0: up to max_batch tokens
    b = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=8)
    n = 5
    norm, core, act = _inputs(cuda, hp, n, 1024, seed=77)
    for r in (a, b):
        r.write(_ffi.RT_NORM, norm)
        r.write(_ffi.RT_CORE, core)
        r.write(_ffi.RT_ACT, act)
    a.eval_chunk(n, _ffi.LOGITS_FULL)
    b.eval_step(n, _ffi.LOGITS_NONE)
    for which, width in ((_ffi.RT_ACT, hp.embedding_length), (_ffi.RT_FFN, hp.feed_forward_length),
                         (_ffi.RT_QKV, 2048), (_ffi.RT_Z, 1024)):
        assert np.array_equal(a.read(which, n * width).numpy().view(np.uint32),
                              b.read(which, n * width).numpy().view(np.uint32))
    last = rt.decode_matvec(stack.head, norm[n - 1:n].contiguous())
    torch.cuda.synchronize()
    assert np.array_equal(a.copy_logits().numpy().view(np.uint32), _bits(last))
    with pytest.raises(rt.Qw35Error, match="n_tokens=9 must be in 1..8"):
        a.eval_chunk(9, _ffi.LOGITS_FULL)
    with pytest.raises(rt.Qw35Error, match="unknown logits mode"):
        a.eval_chunk(4, 7)
    a.close()
    b.close()


def test_chunk_with_kquant_projections(cuda):
    """Q4_K mixers (dequantised in the prefill kernel) and a Q5_K FFN (the
    runtime makes its fp16 prefill images): both give the half weights of the
    reference's tiled matmul, qw35_tiled_mm.metal:199-255; the same bars."""
    from qwowl35_amd import qwen35
    from qwowl35_amd import runtime as rt

    hp = _hp()
    stack = qwen35.ProjectionStack.synthetic(hp, qwen35.StackTypes(mixer=rt.TYPE_Q4_K, ffn=rt.TYPE_Q5_K, head=14),
                                             seed=9, distinct=True, device=cuda)
    r = rt.ProjectionRuntime(_image(stack), hp, vocab=hp.vocab, max_batch=1, prefill_chunk=64)
    norm, core, act = _inputs(cuda, hp, 64, 1024, seed=3)
    _check_chunk(r, stack, 64, norm, core, act)
    r.close()


def _mixed_width_hp():
    # attn_q rows 2048 vs attn_qkv rows 1536 (QKV); attn_output k 512 vs ssm_out k 1024 (CORE)
    return replace(_hp(), ssm_state_size=64, attention_value_length=128)


def test_buffers_hold_each_op_packed_at_its_own_length(cuda):
    """QKV and CORE serve ops of different lengths: each op's rows are packed at
    its own length, at batch 3 (eval_step, against the plan API on views of
    one buffer) and over a 40-token chunk (against single calls)."""
    import torch

    from qwowl35_amd import _ffi
    from qwowl35_amd import qwen35
    from qwowl35_amd import runtime as rt

    hp = _mixed_width_hp()
    stack = qwen35.ProjectionStack.synthetic(hp, qwen35.StackTypes(head=14), seed=11, distinct=True, device=cuda)
    r = rt.ProjectionRuntime(_image(stack), hp, vocab=hp.vocab, max_batch=8, prefill_chunk=64)
    assert r.buffer(_ffi.RT_QKV)[1] == 2048 and r.buffer(_ffi.RT_CORE)[1] == 1024
    nb = 3
    g = torch.Generator(device=cuda)
    g.manual_seed(21)
    norm = torch.randn((nb, hp.embedding_length), generator=g, device=cuda)
    core_flat = torch.randn(nb * 1024, generator=g, device=cuda)
    act = torch.randn((nb, hp.embedding_length), generator=g, device=cuda)
    r.write(_ffi.RT_NORM, norm)
    r.write(_ffi.RT_CORE, core_flat)
    r.write(_ffi.RT_ACT, act)
    r.eval_step(nb, _ffi.LOGITS_FULL)
    bufs = qwen35.StepBuffers.make(hp, nb, g, awq=False, shared_outputs=True)
    bufs.norm.copy_(norm)
    bufs.ffn_norm = bufs.norm
    ref_core = core_flat.clone()
    bufs.core = {512: ref_core[:nb * 512].view(nb, 512), 1024: ref_core.view(nb, 1024)}
    bufs.act.copy_(act)
    plan = qwen35.build_plan(stack, bufs)
    plan.launch()
    torch.cuda.synchronize()
    plan.close()
    assert np.array_equal(r.read(_ffi.RT_ACT, nb * hp.embedding_length).numpy().view(np.uint32),
                          _bits(bufs.act).reshape(-1))
    q = bufs.mixer_out[3]["attn_q"]  # the last writer of QKV: layer 3, packed at 2048
    assert np.array_equal(r.read(_ffi.RT_QKV, q.numel()).numpy().view(np.uint32), _bits(q).reshape(-1))
    assert np.array_equal(r.copy_logits().numpy().view(np.uint32), _bits(bufs.logits))
    # the chunk: CORE packed at 512 for layer 3's attn_output, at 1024 for the delta layers' ssm_out
    n = 40
    norm, core, act = _inputs(cuda, hp, n, 1024, seed=5)
    r.write(_ffi.RT_NORM, norm)
    r.write(_ffi.RT_CORE, core)
    r.write(_ffi.RT_ACT, act)
    r.eval_chunk(n, _ffi.LOGITS_NONE)
    ws = _workspace(stack, n, cuda)
    want = act.clone()
    flat = core.reshape(-1)
    for il, layer in enumerate(stack.layers):
        out = qwen35.mixer_projections(hp, il)[-1]
        x = flat[:n * out.k].view(n, out.k)
        rt.matmul_prefill(layer[out.name], x, out_dtype=torch.float32, dst=want, workspace=ws,
                          epilogue=_ffi.EPILOGUE_ADD)
        ffn = rt.matmul_prefill(layer["ffn_gate"], norm, out_dtype=torch.float32, workspace=ws)
        rt.matmul_prefill(layer["ffn_up"], norm, out_dtype=torch.float32, dst=ffn, workspace=ws,
                          epilogue=_ffi.EPILOGUE_SWIGLU)
        rt.matmul_prefill(layer["ffn_down"], ffn, out_dtype=torch.float32, dst=want, workspace=ws,
                          epilogue=_ffi.EPILOGUE_ADD)
    torch.cuda.synchronize()
    assert np.array_equal(r.read(_ffi.RT_ACT, n * hp.embedding_length).numpy().view(np.uint32),
                          _bits(want).reshape(-1))
    r.close()


def test_epilogue_validation(cuda):
    import torch

    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    from oracle import gf4 as ogf4
    from tests.helpers import bf16_normal

    words = ogf4.gf4_pack(bf16_normal(np.random.default_rng(1), (32, 256), 0.02))
    hw = rt.HipWeight.upload(words.view(np.uint8), om.TYPE_GF4, 32, 256)
    a = torch.zeros((9, 256), dtype=torch.float32, device=cuda)
    with pytest.raises(rt.Qw35Error, match="take fp32 c and a workspace"):
        rt.matmul_prefill(hw, a, out_dtype=torch.bfloat16, epilogue=_ffi.EPILOGUE_ADD)
    with pytest.raises(rt.Qw35Error, match="unknown epilogue 3"):
        rt.matmul_prefill(hw, a, out_dtype=torch.float32, epilogue=3)
