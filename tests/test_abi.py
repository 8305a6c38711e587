"""C-ABI checks that need no GPU: the library loads, exports every symbol that
include/qw35_hip.h declares, its structs match the ctypes mirrors, and the
host-side validation rejects bad calls with a message (the 0 + err-buffer
convention of qw35-server/src/metal/bridge/Qw35FFI.h:1-4)."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from qwowl35_amd import _ffi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qw35_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qw35_hip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _ffi.load()


def test_library_exports_every_declared_symbol(lib):
    syms = declared_symbols()
    assert syms, "no declarations parsed"
    for name in syms:
        assert hasattr(lib, name), name
    assert set(syms) == set(_ffi.PROTOTYPES), "ctypes prototypes must cover exactly the header"


def test_struct_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "qw35_hip.h"\n'
        "int main(void){\n"
        'printf("%zu %zu %zu %zu %zu\\n", sizeof(qw35_hip_tensor_desc), offsetof(qw35_hip_tensor_desc, dims),'
        " offsetof(qw35_hip_tensor_desc, type_id), offsetof(qw35_hip_tensor_desc, abs_offset),"
        " offsetof(qw35_hip_tensor_desc, elements));\n"
        'printf("%zu %zu %zu %zu\\n", sizeof(qw35_hip_weight), offsetof(qw35_hip_weight, rows),'
        " offsetof(qw35_hip_weight, bytes), offsetof(qw35_hip_weight, type_id));\n"
        "return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    a, b = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")[:2]
    td = _ffi.TensorDesc
    assert [int(v) for v in a.split()] == [C.sizeof(td), td.dims.offset, td.type_id.offset, td.abs_offset.offset,
                                           td.elements.offset]
    w = _ffi.Weight
    assert [int(v) for v in b.split()] == [C.sizeof(w), w.rows.offset, w.bytes.offset, w.type_id.offset]


def test_runtime_struct_layouts_match_header(tmp_path):
    """qw35_hip_hparams (the reference's qw35_metal_hparams, Qw35MetalTypes.h:30-59:
    96 bytes, n_cls_out last) and qw35_hip_plan_op against their ctypes mirrors."""
    src = tmp_path / "layout2.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "qw35_hip.h"\n'
        "int main(void){\n"
        'printf("%zu %zu %zu %zu %zu %zu %zu\\n", sizeof(qw35_hip_hparams), offsetof(qw35_hip_hparams, rope_sections),'
        " offsetof(qw35_hip_hparams, rope_freq_base), offsetof(qw35_hip_hparams, ssm_inner_size),"
        " offsetof(qw35_hip_hparams, full_attention_interval), offsetof(qw35_hip_hparams, attn_gate),"
        " offsetof(qw35_hip_hparams, n_cls_out));\n"
        'printf("%zu %zu %zu %zu\\n", sizeof(qw35_hip_plan_op), offsetof(qw35_hip_plan_op, dst),'
        " offsetof(qw35_hip_plan_op, token), offsetof(qw35_hip_plan_op, workspace_bytes));\n"
        'printf("%d %d %d %d\\n", (int)QW35_HIP_LOGITS_NONE, (int)QW35_HIP_LOGITS_ARGMAX, (int)QW35_HIP_LOGITS_FULL,'
        " (int)QW35_HIP_RT_NBUF);\n"
        "return 0;}\n"
    )
    exe = tmp_path / "layout2"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    a, b, c = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")[:3]
    h = _ffi.Hparams
    assert [int(v) for v in a.split()] == [96, 32, 48, 72, 76, 88, 92]
    assert [int(v) for v in a.split()] == [C.sizeof(h), h.rope_sections.offset, h.rope_freq_base.offset,
                                           h.ssm_inner_size.offset, h.full_attention_interval.offset,
                                           h.attn_gate.offset, h.n_cls_out.offset]
    op = _ffi.PlanOp
    assert [int(v) for v in b.split()] == [C.sizeof(op), op.dst.offset, op.token.offset, op.workspace_bytes.offset]
    assert [int(v) for v in c.split()] == [_ffi.LOGITS_NONE, _ffi.LOGITS_ARGMAX, _ffi.LOGITS_FULL, _ffi.RT_NBUF]


def test_runtime_create_rejects_bad_inputs_without_a_device(lib):
    """Argument checks that come before any device work."""
    hp = _ffi.Hparams()
    d = _ffi.TensorDesc()
    img = (C.c_uint8 * 64)()
    with pytest.raises(_ffi.Qw35Error, match="invalid runtime creation inputs"):
        _ffi.call("qw35_hip_runtime_create", None, 64, C.byref(d), 1, C.byref(hp), 10, 1, 0)
    with pytest.raises(_ffi.Qw35Error, match="must be positive"):
        _ffi.call("qw35_hip_runtime_create", img, 64, C.byref(d), 1, C.byref(hp), 10, 1, 0)
    hp.transformer_layers, hp.embedding_length, hp.feed_forward_length, hp.n_cls_out = 1, 256, 256, 2
    with pytest.raises(_ffi.Qw35Error, match="classification heads"):
        _ffi.call("qw35_hip_runtime_create", img, 64, C.byref(d), 1, C.byref(hp), 10, 1, 0)
    hp.n_cls_out = 0
    with pytest.raises(_ffi.Qw35Error, match="max_batch=0"):
        _ffi.call("qw35_hip_runtime_create", img, 64, C.byref(d), 1, C.byref(hp), 10, 0, 0)
    with pytest.raises(_ffi.Qw35Error, match="prefill_chunk=4097"):
        _ffi.call("qw35_hip_runtime_create", img, 64, C.byref(d), 1, C.byref(hp), 10, 1, _ffi.MAX_PREFILL_CHUNK + 1)
    with pytest.raises(_ffi.Qw35Error, match="invalid runtime"):
        _ffi.call("qw35_hip_runtime_eval_step", None, 1, 2)
    with pytest.raises(_ffi.Qw35Error, match="invalid runtime"):
        _ffi.call("qw35_hip_runtime_eval_chunk", None, 16, 2)


def _weight(type_id=100, k=4096, rows=16, data=4096, nbytes=None):
    w = _ffi.Weight()
    w.data = data
    w.k = k
    w.rows = rows
    rb = {100: k // 8 * 4, 8: k // 32 * 34, 12: k // 256 * 144, 14: k // 256 * 210}.get(type_id, 0)
    w.bytes = nbytes if nbytes is not None else rb * rows
    w.type_id = type_id
    return w


def _call_matvec(w, x=4096, dst=4096, nb=1, awq=None):
    return _ffi.call("qw35_hip_decode_matvec", C.byref(w), C.c_void_p(x), C.c_void_p(awq), C.c_void_p(dst), nb, 0,
                     None)


@pytest.mark.parametrize(
    "kwargs,needle",
    [
        (dict(type_id=15), "unsupported tensor type 15"),
        (dict(k=100), "multiple of 256"),
        (dict(k=65792), "<= 65536"),
        (dict(rows=0), "rows=0"),
        (dict(nbytes=5), "must be 32768 bytes, got 5"),
        (dict(data=4097), "16-byte aligned"),
    ],
)
def test_decode_matvec_rejects_bad_weights(lib, kwargs, needle):
    with pytest.raises(_ffi.Qw35Error, match=re.escape(needle)):
        _call_matvec(_weight(**kwargs))


def test_decode_matvec_rejects_bad_batch_and_pointers(lib):
    w = _weight()
    with pytest.raises(_ffi.Qw35Error, match="n_batch=0"):
        _call_matvec(w, nb=0)
    with pytest.raises(_ffi.Qw35Error, match="n_batch=9"):
        _call_matvec(w, nb=9)
    with pytest.raises(_ffi.Qw35Error, match="null input"):
        _call_matvec(w, x=0)
    with pytest.raises(_ffi.Qw35Error, match="16-byte aligned"):
        _call_matvec(w, x=4100)


def test_swiglu_rejects_mismatched_pair(lib):
    g = _weight()
    u = _weight(k=8192)
    with pytest.raises(_ffi.Qw35Error, match="share type and shape"):
        _ffi.call("qw35_hip_ffn_gate_up_swiglu", C.byref(g), C.byref(u), C.c_void_p(4096), None, C.c_void_p(4096), 1,
                  None)


def test_weight_view_validates_descriptor(lib):
    d = _ffi.TensorDesc()
    d.dims[0], d.dims[1], d.dims[2], d.dims[3] = 4096, 8, 1, 1
    d.n_dims = 2
    d.type_id = 100
    d.abs_offset = 256
    d.bytes = 8 * 2048
    d.elements = 4096 * 8
    out = _ffi.Weight()
    _ffi.call("qw35_hip_weight_view", C.byref(d), C.c_void_p(1 << 20), C.byref(out))
    assert out.data == (1 << 20) + 256 and out.k == 4096 and out.rows == 8 and out.type_id == 100
    d.elements = 7
    with pytest.raises(_ffi.Qw35Error, match="elements"):
        _ffi.call("qw35_hip_weight_view", C.byref(d), C.c_void_p(1 << 20), C.byref(out))
    d.elements = 4096 * 8
    d.n_dims = 1
    with pytest.raises(_ffi.Qw35Error, match="not a matrix"):
        _ffi.call("qw35_hip_weight_view", C.byref(d), C.c_void_p(1 << 20), C.byref(out))


def test_error_buffer_truncates_safely(lib):
    w = _weight(type_id=15)
    err = C.create_string_buffer(8)
    rc = lib.qw35_hip_decode_matvec(C.byref(w), C.c_void_p(4096), None, C.c_void_p(4096), 1, 0, None, err, 8)
    assert rc == 0 and len(err.value) == 7


@pytest.mark.parametrize(
    "type_id,k,rows,needle",
    [
        (15, 256, 1, "unsupported tensor type 15"),
        (14, 512 + 32, 1, "multiple of 256 for q6_k"),
        (100, 12, 1, "multiple of 8 for gf4"),
        (8, 48, 1, "multiple of 32 for q8_0"),
        (12, 512 + 32, 1, "multiple of 256 for q4_k"),
        (100, 256, 0, "rows=0"),
    ],
)
def test_quantize_rejects_bad_shapes(lib, type_id, k, rows, needle):
    with pytest.raises(_ffi.Qw35Error, match=re.escape(needle)):
        _ffi.call("qw35_hip_quantize", type_id, C.c_void_p(4096), rows, k, None, C.c_void_p(4096), None)


def test_quantize_rejects_bad_pointers(lib):
    with pytest.raises(_ffi.Qw35Error, match="null input"):
        _ffi.call("qw35_hip_quantize", 100, None, 1, 256, None, C.c_void_p(4096), None)
    with pytest.raises(_ffi.Qw35Error, match="16-byte aligned"):
        _ffi.call("qw35_hip_quantize", 100, C.c_void_p(4096), 1, 256, C.c_void_p(4100), C.c_void_p(4096), None)


def _plan_op(kind=0, w=None, up=None, x=4096, dst=4096, nb=1, residual=0):
    op = _ffi.PlanOp()
    op.kind = kind
    op.n_batch = nb
    op.residual = residual
    op.w = C.pointer(w) if w is not None else None
    op.w_up = C.pointer(up) if up is not None else None
    op.x = x
    op.awq = None
    op.dst = dst
    return op


@pytest.mark.parametrize(
    "ops,needle",
    [
        ([], "no ops"),
        ([dict(kind=7)], "op 0: unknown kind 7"),
        ([dict(), dict(nb=9)], "op 1: n_batch=9"),
        ([dict(), dict(wkw=dict(type_id=15))], "op 1: unsupported tensor type 15"),
        ([dict(kind=0, up=True)], "op 0: a MATVEC op takes no w_up"),
        ([dict(kind=1, up=True, residual=1)], "op 0: a SWIGLU op has no residual form"),
        ([dict(kind=1, up=True, upkw=dict(k=8192))], "op 0: gate and up must share type and shape"),
        ([dict(x=0)], "op 0: null input"),
    ],
)
def test_plan_create_validates_every_op(lib, ops, needle):
    built, keep = [], []
    for o in ops:
        w = _weight(**o.get("wkw", {}))
        up = _weight(**o.get("upkw", {})) if o.get("up") else None
        keep += [w, up]
        built.append(_plan_op(kind=o.get("kind", 0), w=w, up=up, x=o.get("x", 4096), nb=o.get("nb", 1),
                              residual=o.get("residual", 0)))
    arr = (_ffi.PlanOp * max(1, len(built)))(*built)
    with pytest.raises(_ffi.Qw35Error, match=re.escape(needle)):
        _ffi.call("qw35_hip_plan_create", arr if built else None, len(built))


def test_plan_null_handles(lib):
    assert lib.qw35_hip_plan_size(None) == 0
    lib.qw35_hip_plan_destroy(None)
    with pytest.raises(_ffi.Qw35Error, match="null plan"):
        _ffi.call("qw35_hip_plan_launch", None, None)


def test_mfma_probe_validates(lib):
    with pytest.raises(_ffi.Qw35Error, match="n_workgroups"):
        _ffi.call("qw35_hip_mfma_probe", 0, 10, C.c_void_p(4096), None)
    with pytest.raises(_ffi.Qw35Error, match="iters"):
        _ffi.call("qw35_hip_mfma_probe", 4, 0, C.c_void_p(4096), None)
    with pytest.raises(_ffi.Qw35Error, match="null sink"):
        _ffi.call("qw35_hip_mfma_probe", 4, 10, None, None)


def test_stream_read_validates(lib):
    assert lib.qw35_hip_stream_read_sink_len(16) >= 1
    with pytest.raises(_ffi.Qw35Error, match="zero bytes"):
        _ffi.call("qw35_hip_stream_read", C.c_void_p(4096), 0, C.c_void_p(4096), None)
    with pytest.raises(_ffi.Qw35Error, match="16-byte aligned"):
        _ffi.call("qw35_hip_stream_read", C.c_void_p(4096), 24, C.c_void_p(4096), None)


def test_q6k_weight_needs_aligned_rows(lib):
    needle = "q6_k needs k % 512 == 0 and rows * row bytes % 16 == 0"
    with pytest.raises(_ffi.Qw35Error, match=re.escape(needle + ", got k=1280 rows=16")):
        _call_matvec(_weight(type_id=14, k=1280))  # 1050-byte rows: 2-byte aligned
    # 2100-byte rows (4 mod 16): 4-byte aligned, the matrix a multiple of 16 bytes only for rows % 4 == 0
    with pytest.raises(_ffi.Qw35Error, match=re.escape(needle + ", got k=2560 rows=6")):
        _call_matvec(_weight(type_id=14, k=2560, rows=6))
    for k, rows in ((4096, 8), (2560, 8), (5120, 2)):
        _ffi.call("qw35_hip_weight_view", C.byref(_q6k_desc(k, rows)), C.c_void_p(1 << 20), C.byref(_ffi.Weight()))


def _q6k_desc(k, rows=8):
    d = _ffi.TensorDesc()
    d.dims[0], d.dims[1], d.dims[2], d.dims[3] = k, rows, 1, 1
    d.n_dims = 2
    d.type_id = 14
    d.abs_offset = 0
    d.bytes = rows * k // 256 * 210
    d.elements = k * rows
    return d


def test_swiglu_rejects_q6k(lib):
    g = _weight(type_id=14)
    with pytest.raises(_ffi.Qw35Error, match="no fused gate/up"):
        _ffi.call("qw35_hip_ffn_gate_up_swiglu", C.byref(g), C.byref(g), C.c_void_p(4096), None, C.c_void_p(4096), 1,
                  None)


@pytest.mark.parametrize("type_id", [8, 12, 13, 14, 101])
@pytest.mark.parametrize("rows", [65549, 248320])
def test_argmax_partials_match_the_launched_grid(lib, type_id, rows):
    """The greedy head sizes its partials from the launch planner (one (token,
    logit) pair per workgroup and batch row, tokens and logits each rounded up to
    256 bytes), and its GEMV launch refuses any other grid. So every shape the
    planner picks for a head must be compiled at every batch: a plan without an
    instantiation falls back to one row tile per workgroup, a different grid. The
    decode GEMV of these types launches the same kernel and plan, so its grid
    (queried without a GPU) must match the partial count at batch 1..8."""
    from qwowl35_amd import runtime as rt

    k = 4096
    w = _weight(type_id=type_id, k=k, rows=rows, nbytes=rows * rt.row_bytes(type_id, k))
    name = C.create_string_buffer(160)
    g, b, l, ws = C.c_uint32(), C.c_uint32(), C.c_uint32(), C.c_uint64()
    for nb in range(1, 9):
        part = lib.qw35_hip_output_argmax_workspace_size(C.byref(w), nb) // 2
        _ffi.call("qw35_hip_gemv_kernel", C.byref(w), None, nb, 0, 0, name, C.sizeof(name), C.byref(g), C.byref(b),
                  C.byref(l), C.byref(ws))
        assert name.value.startswith(b"kq_mfma_gemv<"), name.value
        assert part == (g.value * nb * 4 + 255) // 256 * 256, (nb, name.value, g.value, part)


def test_output_argmax_workspace_and_validation(lib):
    w = _weight(type_id=14, k=4096, rows=248320)
    n1 = lib.qw35_hip_output_argmax_workspace_size(C.byref(w), 1)
    n8 = lib.qw35_hip_output_argmax_workspace_size(C.byref(w), 8)
    assert n1 > 0 and n8 > n1 and n1 % 256 == 0 and n8 % 256 == 0
    assert lib.qw35_hip_output_argmax_workspace_size(C.byref(w), 0) == 0
    assert lib.qw35_hip_output_argmax_workspace_size(C.byref(w), 9) == 0
    assert lib.qw35_hip_output_argmax_workspace_size(C.byref(_weight(type_id=15)), 1) == 0

    def call(x=4096, tok=4096, lg=4096, ws=1 << 20, ws_bytes=None, nb=1):
        return _ffi.call("qw35_hip_output_argmax", C.byref(w), C.c_void_p(x), None, nb, C.c_void_p(tok),
                         C.c_void_p(lg), C.c_void_p(ws), C.c_uint64(n1 if ws_bytes is None else ws_bytes), None)

    with pytest.raises(_ffi.Qw35Error, match="null input, output or workspace"):
        call(ws=0)
    with pytest.raises(_ffi.Qw35Error, match="n_batch=9"):
        call(nb=9)
    with pytest.raises(_ffi.Qw35Error, match="workspace must be 256-byte aligned"):
        call(ws_bytes=n1 - 256)
    with pytest.raises(_ffi.Qw35Error, match="workspace must be 256-byte aligned"):
        call(ws=(1 << 20) + 16)
    with pytest.raises(_ffi.Qw35Error, match="16-byte aligned"):
        call(x=4100)


def test_matmul_prefill_rejects_oversized_token_rows(lib):
    """n_tokens * k beyond 2^30 is refused before anything is launched (the
    staged fp16 token rows are addressed with 32-bit byte offsets)."""
    w = _weight(type_id=100, k=65536, rows=16)
    assert lib.qw35_hip_matmul_prefill_workspace_size(C.byref(w), 16385) == 0
    with pytest.raises(_ffi.Qw35Error, match=re.escape("n_tokens * k = 1073807360 must be <= 1073741824")):
        _ffi.call("qw35_hip_matmul_prefill", C.byref(w), C.c_void_p(4096), 1, None, C.c_void_p(4096), 0, 16385,
                  C.c_void_p(4096), C.c_uint64(1 << 40), None)


def test_q8_0_rows_of_32_column_blocks(lib):
    """q8_0 weights take any k % 32 == 0 (the row-wise GEMV); the chunked paths
    (prefill matmul, greedy head) still need k % 256 == 0 and say so."""
    w = _weight(type_id=8, k=4160, rows=16)
    assert lib.qw35_hip_matmul_prefill_workspace_size(C.byref(w), 16) == 0
    assert lib.qw35_hip_output_argmax_workspace_size(C.byref(w), 1) == 0
    with pytest.raises(_ffi.Qw35Error, match=re.escape("matmul_prefill: needs k % 256 == 0, got k=4160")):
        _ffi.call("qw35_hip_matmul_prefill", C.byref(w), C.c_void_p(4096), 1, None, C.c_void_p(4096), 0, 16,
                  C.c_void_p(4096), C.c_uint64(1 << 30), None)
    with pytest.raises(_ffi.Qw35Error, match=re.escape("output_argmax: needs k % 256 == 0, got k=4160")):
        _ffi.call("qw35_hip_output_argmax", C.byref(w), C.c_void_p(4096), None, 1, C.c_void_p(4096),
                  C.c_void_p(4096), C.c_void_p(4096), C.c_uint64(1 << 20), None)
    with pytest.raises(_ffi.Qw35Error, match=re.escape("k=4160 must be a positive multiple of 256")):
        _call_matvec(_weight(type_id=100, k=4160))
    with pytest.raises(_ffi.Qw35Error, match=re.escape("k=4100 must be a positive multiple of 32")):
        _call_matvec(_weight(type_id=8, k=4100))
    info = _ffi.LaunchInfo() if hasattr(_ffi, "LaunchInfo") else None
    name = C.create_string_buffer(160)
    g, b, l, ws = C.c_uint32(), C.c_uint32(), C.c_uint32(), C.c_uint64()
    _ffi.call("qw35_hip_gemv_kernel", C.byref(w), None, 3, 1, 0, name, C.sizeof(name), C.byref(g), C.byref(b),
              C.byref(l), C.byref(ws))
    # 16 rows at batch 3 (the 4-row instantiation): one workgroup of 8 waves, two rows each,
    # activations of 4 batch rows x 64 blocks x 36 floats in LDS
    assert name.value.decode() == "q8_gemv_rows<4, false, true>"
    assert (g.value, b.value, l.value, ws.value) == (1, 512, 4 * 64 * 36 * 4, 0)
