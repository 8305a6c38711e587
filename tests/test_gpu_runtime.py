"""The projection runtime (qw35_hip_runtime_*), the in-scope part of the
reference's runtime-level ABI (qw35-server/src/metal/bridge/Qw35FFI.h:19-118),
on a synthetic GGUF image with the Qwen3.5 tensor names at small dimensions
(3 DeltaNet layers and 1 attention layer; q8_0 mixers, GF4 FFN, Q6_K head),
plus the non-projection tensors a real image carries.

* Every step's results equal, bit for bit, the same projections recorded
  through the kernel-level plan API (qwen35.build_plan) on the same bytes,
  for FULL logits at batch 1, 3 and 8 and after inputs change in place;
* the greedy head (ARGMAX) equals the reference rule on the FULL logits;
* the logits against fp64 on the library's dequantised head;
* two runtimes over one image share one device store (qw35_shared_tensor_store,
  Qw35MetalRuntime.m:42-80), which outlives the first runtime;
* creation and readback errors name their cause (missing tensor, shape that
  does not match the hyper-parameters, vocabulary, batch, mode).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests import gguf_image
from tests.helpers import GEMV_REL_L2

pytestmark = pytest.mark.gpu


def _hp():
    from qwowl35_amd import qwen35

    return qwen35.Hparams(transformer_layers=4, embedding_length=2048, feed_forward_length=3072,
                          attention_heads=4, attention_kv_heads=2, attention_key_length=256,
                          attention_value_length=256, ssm_state_size=128, ssm_group_count=4, ssm_time_step_rank=8,
                          ssm_inner_size=1024, full_attention_interval=4, attn_gate=1, vocab=3001)


def _image(stack, drop=None, extra=()):
    """GGUF bytes of the stack's projections (minus `drop`) plus non-projection tensors."""
    hp = stack.hp
    tensors = [("token_embd.weight", (hp.embedding_length, hp.vocab), 8,
                bytes(hp.vocab * hp.embedding_length // 32 * 34)),
               ("output_norm.weight", (hp.embedding_length,), 0, bytes(4 * hp.embedding_length))]
    for il in range(hp.transformer_layers):
        tensors.append((f"blk.{il}.attn_norm.weight", (hp.embedding_length,), 0, bytes(4 * hp.embedding_length)))
    from qwowl35_amd import qwen35

    for name, dims, t, dev in qwen35.stack_tensors(stack):
        if name == drop:
            continue
        tensors.append((name, dims, t, dev.cpu().numpy().tobytes()))
    tensors.extend(extra)
    kv = [("general.architecture", gguf_image.STRING, "qwen35"), ("qwen35.block_count", gguf_image.U32,
                                                                  hp.transformer_layers)]
    image, _ = gguf_image.build(kv, tensors)
    return np.frombuffer(image, dtype=np.uint8)


@pytest.fixture(scope="module")
def small(cuda):
    from qwowl35_amd import qwen35

    stack = qwen35.ProjectionStack.synthetic(_hp(), qwen35.StackTypes(head=14), seed=5, distinct=True, device=cuda)
    return stack, _image(stack)


def _reference(stack, nb, norm, core, act, head_mode_full=True):
    """The same step through the kernel-level plan API, with the runtime's
    buffer sharing (one norm for mixers, FFN and head; no AWQ)."""
    import torch

    from qwowl35_amd import qwen35

    gen = torch.Generator(device=norm.device)
    bufs = qwen35.StepBuffers.make(stack.hp, nb, gen, awq=False, shared_outputs=True)
    bufs.norm.copy_(norm)
    bufs.ffn_norm = bufs.norm
    for w, t in bufs.core.items():
        t.copy_(core[:, :w])
    bufs.act.copy_(act)
    plan = qwen35.build_plan(stack, bufs, head=head_mode_full)
    plan.launch()
    torch.cuda.synchronize()
    plan.close()
    return bufs


def _inputs(cuda, hp, nb, seed):
    import torch

    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    norm = torch.randn((nb, hp.embedding_length), generator=g, device=cuda)
    core = torch.randn((nb, 1024), generator=g, device=cuda)
    act = torch.randn((nb, hp.embedding_length), generator=g, device=cuda)
    return norm, core, act


@pytest.mark.parametrize("nb", [1, 3, 8])
def test_runtime_step_equals_plan_api(cuda, small, nb):
    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    stack, image = small
    hp = stack.hp
    r = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=8)
    for seed in (nb, 100 + nb):  # the second round rewrites the inputs in place
        norm, core, act = _inputs(cuda, hp, nb, seed)
        r.write(_ffi.RT_NORM, norm)
        r.write(_ffi.RT_CORE, core)
        r.write(_ffi.RT_ACT, act)
        print(f"runtime step nb={nb} seed={seed}", flush=True)
        r.eval_step(nb, _ffi.LOGITS_FULL)
        logits = r.copy_logits()
        ref = _reference(stack, nb, norm, core, act)
        assert np.array_equal(logits.numpy().view(np.uint32), ref.logits.cpu().numpy().view(np.uint32))
        got_act = r.read(_ffi.RT_ACT, nb * hp.embedding_length).reshape(nb, -1)
        assert np.array_equal(got_act.numpy().view(np.uint32), ref.act.cpu().numpy().view(np.uint32))
        got_ffn = r.read(_ffi.RT_FFN, nb * hp.feed_forward_length).reshape(nb, -1)
        assert np.array_equal(got_ffn.numpy().view(np.uint32), ref.ffn_act[-1].cpu().numpy().view(np.uint32))
        # the last writer of each mixer buffer: layer 3 (attention) q / k / v, layer 2 (delta) gate / beta / alpha
        for which, il, name in ((_ffi.RT_QKV, 3, "attn_q"), (_ffi.RT_K, 3, "attn_k"), (_ffi.RT_V, 3, "attn_v"),
                                (_ffi.RT_Z, 2, "attn_gate"), (_ffi.RT_BETA, 2, "ssm_beta"),
                                (_ffi.RT_ALPHA, 2, "ssm_alpha")):
            want = ref.mixer_out[il][name]
            got = r.read(which, want.numel()).reshape(want.shape)
            assert np.array_equal(got.numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), name
        # logits against fp64 on the dequantised head
        head64 = rt.dequantize(stack.head).double()
        want64 = (head64 @ norm.double().T).T.cpu().numpy()
        assert om.rel_l2(logits.numpy(), want64) <= GEMV_REL_L2
    r.close()


@pytest.mark.parametrize("nb", [1, 4, 8])
def test_runtime_greedy_head_and_modes(cuda, small, nb):
    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    stack, image = small
    hp = stack.hp
    r = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=8)
    norm, core, act = _inputs(cuda, hp, nb, 7 + nb)
    r.write(_ffi.RT_NORM, norm)
    r.write(_ffi.RT_CORE, core)
    r.write(_ffi.RT_ACT, act)
    r.eval_step(nb, _ffi.LOGITS_FULL)
    logits = r.copy_logits().numpy()
    r.write(_ffi.RT_ACT, act)
    r.eval_step(nb, _ffi.LOGITS_ARGMAX)
    tok, lg = r.argmax()
    ids, best = om.argmax_rule(logits)
    assert np.array_equal(np.array(tok, dtype=np.uint32), ids)
    assert np.array_equal(np.array(lg, dtype=np.float32).view(np.uint32), best.view(np.uint32))
    with pytest.raises(rt.Qw35Error, match="did not compute the logits"):
        r.copy_logits()
    # NONE: no head; the logits buffer keeps the FULL step's values
    r.write(_ffi.RT_ACT, act)
    r.eval_step(nb, _ffi.LOGITS_NONE)
    kept = r.read(_ffi.RT_LOGITS, nb * hp.vocab).reshape(nb, -1).numpy()
    assert np.array_equal(kept.view(np.uint32), logits.view(np.uint32))
    with pytest.raises(rt.Qw35Error, match="did not run the greedy head"):
        r.argmax()
    with pytest.raises(rt.Qw35Error, match="n_batch=9"):
        r.eval_step(9, _ffi.LOGITS_FULL)
    with pytest.raises(rt.Qw35Error, match="unknown logits mode"):
        r.eval_step(1, 3)
    r.close()


def test_runtimes_share_one_store(cuda, small):
    from qwowl35_amd import _ffi
    from qwowl35_amd import runtime as rt

    stack, image = small
    hp = stack.hp
    a = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=2)
    b = rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=1)
    assert a.store_base and a.store_base == b.store_base
    norm, core, act = _inputs(cuda, hp, 1, 3)
    for r in (a, b):
        r.write(_ffi.RT_NORM, norm)
        r.write(_ffi.RT_CORE, core)
        r.write(_ffi.RT_ACT, act)
    a.eval_step(1, _ffi.LOGITS_FULL)
    la = a.copy_logits()
    a.close()  # the store stays alive for b
    b.eval_step(1, _ffi.LOGITS_FULL)
    assert np.array_equal(b.copy_logits().numpy().view(np.uint32), la.numpy().view(np.uint32))
    b.close()


def test_runtime_create_errors(cuda, small):
    from dataclasses import replace

    from qwowl35_amd import runtime as rt

    stack, image = small
    hp = stack.hp
    with pytest.raises(rt.Qw35Error, match=r"blk\.1\.ffn_up\.weight: store_weight: no tensor named"):
        rt.ProjectionRuntime(_image(stack, drop="blk.1.ffn_up.weight"), hp, vocab=hp.vocab)
    # ungated attention expects attn_q of heads * key_length rows
    with pytest.raises(rt.Qw35Error, match=r"blk\.3\.attn_q\.weight is 2048 x 2048 .* expected 1024 x 2048"):
        rt.ProjectionRuntime(image, replace(hp, attn_gate=0), vocab=hp.vocab)
    with pytest.raises(rt.Qw35Error, match=r"output\.weight is 3001 x 2048 .* expected 3000 x 2048"):
        rt.ProjectionRuntime(image, hp, vocab=3000)
    with pytest.raises(rt.Qw35Error, match="max_batch=9"):
        rt.ProjectionRuntime(image, hp, vocab=hp.vocab, max_batch=9)
    with pytest.raises(rt.Qw35Error, match="decode GEMVs do not take"):
        rt.ProjectionRuntime(_image(stack, drop="blk.0.ssm_beta.weight",
                                    extra=[("blk.0.ssm_beta.weight", (2048, 8), 1, bytes(2 * 2048 * 8))]),
                             hp, vocab=hp.vocab)
