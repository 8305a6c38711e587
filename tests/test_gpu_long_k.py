"""GPU parity of rows longer than the Qwen3.5-9B's (k beyond 12288, up to the
65536 limit of the C ABI), as other family sizes have them.

The reference's decode takes any k through n_blocks = ceil(k / block)
(qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:240), and its tiled
prefill matmul loops over K.  Here a decode GEMV whose row is longer than its
plan covers in one round runs as kq_mfma_gemv_long (rounds of 8 waves x 4
chunks), and the prefill staging pass reads rows past 12288 columns twice.
Bars are those of the 9B shapes: GEMVs within GEMV_REL_L2 of the fp64 matvec of
the oracle-dequantised weights; prefill within 1e-3 relative L2 (fp32 output)
or one bf16 ulp plus the fp32-accumulation allowance (bf16 output) of the
fp64 product of the operands the kernel contracts.  k = 17408 = 68 chunks
leaves the last round four chunks long (waves partly idle)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests.helpers import GEMV_REL_L2, TYPES, activations, awq_scales, check_prefill, make_weight

pytestmark = pytest.mark.gpu

K_LONG = 17408


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


@pytest.mark.parametrize("name", ["gf4", "q8_0", "q4_k", "q6_k", "q5_k", "gf2"])
@pytest.mark.parametrize("nb", [1, 3, 8])
def test_long_k_gemv_parity(cuda, name, nb):
    import torch

    type_id = TYPES[name]
    rows, k = 100, K_LONG  # Q6_K: 14280-byte rows, 8 bytes past 16-byte boundaries on odd rows
    print(f"long-k gemv {name} {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(k + nb)
    raw, deq = make_weight(type_id, rows, k, seed=rows + k)
    w = _rt().HipWeight.upload(raw, type_id, rows, k)
    info = _rt().gemv_kernel(w, nb)
    assert info["name"].startswith("kq_mfma_gemv_long<"), info["name"]
    x = activations(rng, nb, k)
    y = _rt().decode_matvec(w, _t(x, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2
    # AWQ + residual, and the K-split entry point (no split plan at this k: same kernel)
    a = awq_scales(rng, k)
    base = rng.standard_normal((nb, rows)).astype(np.float32)
    dst = torch.from_numpy(base.copy()).to(cuda)
    ws = _rt().decode_matvec_workspace(w, nb, device=cuda) if nb >= 3 else None
    _rt().decode_matvec(w, _t(x, cuda), dst=dst, residual=True, awq=_t(a, cuda), workspace=ws)
    want = base.astype(np.float64) + om.matvec_f64(deq, x, a)
    assert om.rel_l2(dst.cpu().numpy(), want) <= GEMV_REL_L2


@pytest.mark.parametrize("name", ["gf4", "q8_0", "q4_k"])
@pytest.mark.parametrize("nb", [1, 5])
def test_longest_k_gemv(cuda, name, nb):
    """k = 65536, the ABI's limit: 256 chunks, eight full rounds."""
    type_id = TYPES[name]
    rows, k = 40, 65536
    print(f"longest-k gemv {name} {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(nb)
    raw, deq = make_weight(type_id, rows, k, seed=17)
    w = _rt().HipWeight.upload(raw, type_id, rows, k)
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    y = _rt().decode_matvec(w, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x, a)) <= GEMV_REL_L2


@pytest.mark.parametrize("name", ["gf4", "q8_0", "q4_k"])
@pytest.mark.parametrize("nb", [1, 8])
def test_long_k_swiglu(cuda, name, nb):
    type_id = TYPES[name]
    rows, k = 96, K_LONG
    print(f"long-k swiglu {name} {rows}x{k} nb={nb}", flush=True)
    rng = np.random.default_rng(31 + nb)
    rg, dg = make_weight(type_id, rows, k, seed=3, std=0.02)
    ru, du = make_weight(type_id, rows, k, seed=4, std=0.02)
    x = activations(rng, nb, k)
    a = awq_scales(rng, k)
    g = _rt().HipWeight.upload(rg, type_id, rows, k)
    u = _rt().HipWeight.upload(ru, type_id, rows, k)
    assert _rt().gemv_kernel(g, nb, w_up=u, awq=True)["name"].startswith("kq_mfma_gemv_long<")
    y = _rt().ffn_gate_up_swiglu(g, u, _t(x, cuda), awq=_t(a, cuda)).cpu().numpy()
    assert om.rel_l2(y, om.swiglu_f64(dg, du, x, a)) <= GEMV_REL_L2


@pytest.mark.parametrize("nb", [1, 5])
def test_long_k_greedy_head(cuda, nb):
    """The fused greedy head at k = 17408 picks exactly what the reference's
    rule picks on the same launch shape's logits (ties to the smaller row, NaN
    never chosen), on a ragged row count whose Q6_K rows are not 16-byte
    aligned; the weight is quantised on the GPU."""
    import torch

    rt = _rt()
    rows, k = 3002, K_LONG
    print(f"long-k head q6_k {rows}x{k} nb={nb}", flush=True)
    g = torch.Generator(device=cuda)
    g.manual_seed(nb)
    src = torch.randn((rows, k), generator=g, device=cuda) * 0.02
    w = rt.quantize_weight(src, om.TYPE_Q6_K)
    del src
    x = torch.randn((nb, k), generator=g, device=cuda)
    logits = rt.decode_matvec(w, x).cpu().numpy()
    tok, lg = rt.output_argmax(w, x)
    ids, best = om.argmax_rule(logits)
    assert np.array_equal(tok.cpu().numpy().view(np.uint32), ids)
    assert np.array_equal(lg.cpu().numpy().view(np.uint32), best.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("staged", [True, False])
@pytest.mark.parametrize("out_f32", [True, False])
def test_long_k_gf4_prefill(cuda, staged, out_f32):
    from tests.test_gpu_prefill import _case

    print(f"long-k gf4 prefill staged={staged} f32={out_f32}", flush=True)
    # the direct path (no workspace) takes bf16 activations without AWQ only
    _case(cuda, 37, 100, K_LONG, seed=5, awq_on=staged, out_f32=out_f32, staged=staged)


def test_long_k_gf4_prefill_fp32_input(cuda):
    from tests.test_gpu_prefill import _case

    print("long-k gf4 prefill fp32 input", flush=True)
    _case(cuda, 130, 64, K_LONG, seed=6, awq_on=True, out_f32=True, a_f32=True, staged=True)


@pytest.mark.parametrize("name", ["q8_0", "q4_k"])
def test_long_k_kquant_prefill(cuda, name):
    """q8_0 and Q4_K dequantised in the kernel (no fp16 image)."""
    import torch

    type_id = TYPES[name]
    m, n, k = 130, 64, K_LONG
    print(f"long-k prefill {name} m={m} {n}x{k}", flush=True)
    rng = np.random.default_rng(8)
    raw, _ = make_weight(type_id, n, k, seed=9)
    w = _rt().HipWeight.upload(raw, type_id, n, k)
    a32 = activations(rng, m, k)
    awq = awq_scales(rng, k)
    bits = om.f32_to_bf16_bits(a32)
    a_dev = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    img = om.prefill_image(type_id, raw, n, k).astype(np.float32)
    pw = w.prefill
    assert pw is w
    for a_host, a in ((bits, a_dev), (a32, _t(a32, cuda))):
        out = _rt().matmul_prefill(pw, a, awq=_t(awq, cuda), out_dtype=torch.float32)
        check_prefill(out, a_host, awq, img, w_exact=om.dequant(type_id, raw, n, k))
