"""GPU weight producers (qw35_hip_quantize) against the CPU oracle, bit for bit.

GF4: the reference packer pack_gf4_prepared(scale_search=False) with the AWQ
column multiply of pack_ffn_gf4 (tools/qw35_cook_common.py:83-119,182-199), as
restated in oracle/gf4.py.  q8_0 / Q4_K: the library's encoders against the
oracle's numpy statements of the same encoders (oracle/q8_0.py, oracle/q4_k.py).
Inputs span many binades (fp16 subnormal scales, e5m2 overflow to inf, ties of
|x| inside a group, zero groups) so a wrong rounding or tie rule shows.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import gf4 as ogf4
from oracle import matvec as om
from tests.helpers import TYPES, awq_scales

pytestmark = pytest.mark.gpu


def _rt():
    from qwowl35_amd import runtime

    return runtime


def _t(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _wide_range(rng, rows, k):
    """N(0,1) rows scaled per row by 2^U(-30, 18): subnormal fp16 scales up to e5m2 inf."""
    x = rng.standard_normal((rows, k), dtype=np.float32)
    return (x * np.exp2(rng.uniform(-30, 18, (rows, 1))).astype(np.float32)).astype(np.float32)


def _special_groups(k):
    """Rows of hand-made groups: ties of |x|, zeros, signed maxima, exact levels."""
    g = [
        [0.5, -0.25, 0.0, 0.125, -0.5, 0.375, 0.25, -0.125],
        [-0.5, 0.5, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
        [0.0] * 8,
        [1.0, 0.375, 0.125, 0.875, 0.625, -0.875, -0.625, -0.375],
        [-0.0] * 8,
        [3.0, -3.0, 3.0, -3.0, 1.5, -1.5, 0.75, -0.75],
        [65504.0, 1.0, -1.0, 0.0, 0.0, 0.0, 0.0, 0.0],
        [7e4, -7e4, 1.0, 0.0, 0.0, 0.0, 0.0, 0.0],
        [6e-8, -3e-8, 1e-9, 0.0, 0.0, 0.0, 0.0, 0.0],
    ]
    reps = k // 8
    rows = [np.array((g[i % len(g)] * reps)[:k], dtype=np.float32) for i in range(len(g))]
    return np.stack(rows)


@pytest.mark.parametrize("rows,k", [(1, 8), (3, 40), (64, 4096), (17, 12288)])
def test_gf4_pack_bit_exact(cuda, rows, k):
    rng = np.random.default_rng(rows * 13 + k)
    w = om.bf16_round(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02))
    got = _rt().quantize(_t(w, cuda), om.TYPE_GF4).cpu().numpy().view("<u4").reshape(rows, k // 8)
    assert np.array_equal(got, ogf4.gf4_pack(w))


def test_gf4_pack_wide_range_and_special_groups(cuda):
    rng = np.random.default_rng(77)
    w = np.concatenate([_wide_range(rng, 200, 256), _special_groups(256)])
    got = _rt().quantize(_t(w, cuda), om.TYPE_GF4).cpu().numpy().view("<u4").reshape(w.shape[0], 32)
    assert np.array_equal(got, ogf4.gf4_pack(w))


def test_gf4_pack_with_awq_columns(cuda):
    """pack_ffn_gf4: src * col_scale (fp32) then pack (tools/qw35_cook_common.py:198)."""
    rng = np.random.default_rng(5)
    rows, k = 48, 4096
    w = om.bf16_round(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02))
    s = awq_scales(rng, k)
    got = _rt().quantize(_t(w, cuda), om.TYPE_GF4, col_scale=_t(s, cuda)).cpu().numpy().view("<u4")
    want = ogf4.gf4_pack((w * s[None, :]).astype(np.float32))
    assert np.array_equal(got.reshape(rows, k // 8), want)


@pytest.mark.parametrize("name", ["gf2", "q8_0", "q4_k", "q5_k"])
@pytest.mark.parametrize("rows,k", [(1, 256), (33, 4096), (7, 12288)])
def test_kquant_encoders_bit_exact(cuda, name, rows, k):
    type_id = TYPES[name]
    rng = np.random.default_rng(rows + k)
    w = rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02)
    w[0, :64] = 0.0  # an all-zero block / sub-block
    got = _rt().quantize(_t(w, cuda), type_id).cpu().numpy().reshape(rows, -1)
    assert np.array_equal(got, om.quantize(type_id, w))


@pytest.mark.parametrize("name", ["gf2", "q8_0", "q4_k", "q5_k"])
def test_kquant_encoders_wide_range_and_awq(cuda, name):
    type_id = TYPES[name]
    rng = np.random.default_rng(9)
    rows, k = 64, 512
    w = _wide_range(rng, rows, k) * np.float32(1e-6)
    s = awq_scales(rng, k)
    got = _rt().quantize(_t(w, cuda), type_id, col_scale=_t(s, cuda)).cpu().numpy().reshape(rows, -1)
    assert np.array_equal(got, om.quantize(type_id, (w * s[None, :]).astype(np.float32)))


def test_quantize_then_gemv_roundtrip(cuda):
    """Producer -> dequant -> GEMV: a weight made on the GPU is a valid tensor of each type."""
    rng = np.random.default_rng(3)
    rows, k = 256, 4096
    w = om.bf16_round(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal((2, k), dtype=np.float32)
    for name, type_id in TYPES.items():
        hw = _rt().quantize_weight(_t(w, cuda), type_id)
        deq = _rt().dequantize(hw).cpu().numpy()
        raw = hw.storage.cpu().numpy().reshape(rows, -1)
        assert np.array_equal(deq.view(np.uint32), om.dequant(type_id, raw, rows, k).view(np.uint32)), name
        y = _rt().decode_matvec(hw, _t(x, cuda)).cpu().numpy()
        assert om.rel_l2(y, om.matvec_f64(deq, x)) <= 1e-3, name


def test_mfma_probe_sums(cuda):
    """Every lane's 8 accumulators hold iters * sum_k a_k b_k of exact small
    fp16 products, so the sink is a closed form of the lane index."""
    rt = _rt()
    iters = 64
    sink = rt.mfma_probe(3, iters).cpu().numpy().reshape(3, 256)
    # lane l of a wave supplies A row l % 32 = ((l + i) & 15) * 2^-12 for its 8 k values
    # (i = 0..7, k block 8 * (l // 32)); B column j = (i + 1) * 2^-10 for every column.
    # D[row][col] = sum over 16 k of A[row][k] B[k][col]; each lane sums its 16 D values.
    a = np.array([[((t + i) & 15) * 2.0 ** -12 for i in range(8)] for t in range(64)])
    b = np.array([(i + 1) * 2.0 ** -10 for i in range(8)])
    d = np.zeros((32, 32))
    for l in range(64):
        for i in range(8):
            d[l % 32, :] += a[l, i] * b[i]  # k = 8 * (l // 32) + i contributes A[l%32][k] * B[k][*]
    want = np.zeros(64)
    for l in range(64):
        rows = [8 * (r // 4) + 4 * (l // 32) + r % 4 for r in range(16)]
        want[l] = 8 * iters * sum(d[rr, l % 32] for rr in rows)
    for w in range(3):
        for wave in range(4):
            np.testing.assert_allclose(sink[w, 64 * wave:64 * wave + 64], want, rtol=1e-5)


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 25_165_824])
def test_stream_read_probe_reads_every_word(cuda, nbytes):
    """The read probe's per-workgroup XOR digests fold to the XOR of all words."""
    import torch

    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).to(cuda)
    sink = _rt().stream_read(buf).cpu().numpy().view(np.uint32)
    assert int(np.bitwise_xor.reduce(sink)) == int(np.bitwise_xor.reduce(host))
