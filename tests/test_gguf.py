"""GGUF v3 reader (qw35_hip_gguf_parse) and device tensor store.

The parser restates the reference loader (qw35-server/src/loader/tensors.rs:23-172,
metadata.rs:206-288); the images come from tests/gguf_image.py.  CPU tests:
descriptors against the writer's record (offsets, sizes, dims padding as
bridge.rs:279-290), the per-type size table, and the error paths, including
every truncation of a valid image.  GPU tests: weights served by the store
against the oracle on the same bytes.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import matvec as om
from tests import gguf_image as gi
from tests.helpers import GEMV_REL_L2, make_weight


def _rt():
    from qwowl35_amd import runtime

    return runtime


# (block elements, block bytes) of every GGUF type the reference sizes
# (loader/tensors.rs:136-170); GF2 (101) is 5 bytes per 16 elements.
SIZES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 40),
         10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
         16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 110), 20: (32, 18), 21: (256, 110),
         22: (256, 82), 23: (256, 136), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
         29: (256, 56), 30: (1, 2), 100: (8, 4), 101: (16, 5)}


def _model(alignment=32):
    """A small mixed-codec model image: (image, writer info, {name: (type, rows, k, raw, deq)})."""
    mats = {}
    tensors = []
    for i, (name, t, rows, k) in enumerate([("blk.0.ffn_gate.weight", om.TYPE_GF4, 64, 512),
                                            ("blk.0.attn_q.weight", om.TYPE_Q8_0, 48, 256),
                                            ("blk.0.ffn_down.weight", om.TYPE_Q4_K, 32, 1024),
                                            ("blk.1.ffn_up.weight", om.TYPE_GF2, 40, 512),
                                            ("blk.1.ffn_down.weight", om.TYPE_Q5_K, 24, 768),
                                            ("output.weight", om.TYPE_Q6_K, 80, 2048)]):
        raw, deq = make_weight(t, rows, k, seed=100 + i)
        mats[name] = (t, rows, k, raw, deq)
        tensors.append((name, (k, rows), t, raw.tobytes()))
    tensors.insert(2, ("blk.0.attn_norm.weight", (512,), 0, np.ones(512, np.float32).tobytes()))
    kv = [("general.architecture", gi.STRING, "qwen35"),
          ("general.alignment", gi.U32, alignment),
          ("qwen35.block_count", gi.U32, 2),
          ("tokenizer.ggml.tokens", gi.ARRAY, (gi.STRING, ["a", "bb", "é"])),
          ("tokenizer.ggml.scores", gi.ARRAY, (gi.F32, [0.5, -1.0, 2.0])),
          ("nested", gi.ARRAY, (gi.ARRAY, [(gi.U8, [1, 2, 3]), (gi.I64, [7])])),
          ("flags", gi.BOOL, True), ("eps", gi.F64, 1e-6), ("ctx", gi.U64, 262144)]
    image, info = gi.build(kv, tensors, alignment=alignment)
    return image, info, mats


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_parse_matches_the_writer(alignment):
    image, info, _ = _model(alignment)
    tensors, data_off, _ = _rt().gguf_parse(image)
    assert data_off % alignment == 0
    assert [t.name for t in tensors] == [i["name"] for i in info]
    for t, i in zip(tensors, info):
        assert t.abs_offset == i["abs_offset"] and t.abs_offset % alignment == 0
        assert t.bytes == i["bytes"]
        assert t.type_id == i["type_id"] and t.dims == i["dims"]
        assert t.elements == int(np.prod(i["dims"]))


def test_dims_padding_and_byte_sizes_of_every_type():
    tensors = []
    for t, (be, bb) in SIZES.items():
        n = 512
        tensors.append((f"t{t}", (n,), t, b"\x00" * (-(-n // be) * bb)))
    tensors.append(("five_d", (4, 3, 2, 2, 2), 0, b"\x00" * (96 * 4)))
    image, info = gi.build([], tensors)
    got, _, (descs, n, _) = _rt().gguf_parse(image)
    for g, i in zip(got, info):
        assert g.bytes == i["bytes"], g.name
    five = descs[n - 1]
    assert five.n_dims == 5 and list(five.dims) == [4, 3, 2, 2] and five.elements == 96
    one = descs[0]
    assert one.n_dims == 1 and list(one.dims) == [512, 1, 1, 1]


def test_oracle_sizes_agree_with_the_parser():
    for t in (om.TYPE_GF4, om.TYPE_GF2, om.TYPE_Q8_0, om.TYPE_Q4_K, om.TYPE_Q5_K, om.TYPE_Q6_K):
        be, bb = SIZES[t]
        assert om.tensor_nbytes(t, 3, 2048) == 3 * 2048 // be * bb


def _err(image):
    with pytest.raises(_rt().Qw35Error) as e:
        _rt().gguf_parse(image)
    return str(e.value)


def test_rejects_bad_headers():
    image, _, _ = _model()
    assert "not a GGUF file" in _err(b"GGML" + image[4:])
    v2 = bytearray(image)
    v2[4] = 2
    assert "only GGUF v3 is supported, found v2" in _err(bytes(v2))
    assert "unexpected end" in _err(image[:10])


def test_every_truncation_fails_cleanly():
    image, info, _ = _model()
    last_end = max(i["abs_offset"] + i["bytes"] for i in info)
    for cut in list(range(0, 600)) + list(range(600, last_end, 97)):
        msg = _err(image[:cut])
        assert "unexpected end" in msg or "points outside GGUF file" in msg, (cut, msg)
    _rt().gguf_parse(image[:last_end])  # the data need not be padded at the end


def test_rejects_bad_tensors_and_metadata():
    assert "unsupported GGUF type 4" in _err(gi.build([], [("x", (32,), 4, b"")])[0])
    assert "unsupported dimension count 0" in _err(gi.build([], [("x", (), 0, b"")])[0])
    assert "unsupported dimension count 9" in _err(gi.build([], [("x", (1,) * 9, 0, b"\0" * 4)])[0])
    img, _ = gi.build([], [("w", (8,), 0, b"\0" * 32)])
    assert "w points outside GGUF file" in _err(img[:-1])
    assert "unknown GGUF metadata type 13" in _err(gi.build([("k", gi.U32, 1)], [])[0].replace(
        b"\x01\x00\x00\x00\x00\x00\x00\x00k\x04\x00\x00\x00", b"\x01\x00\x00\x00\x00\x00\x00\x00k\x0d\x00\x00\x00"))
    deep = (gi.U8, [1])
    for _ in range(9):
        deep = (gi.ARRAY, [deep])
    assert "nesting is too deep" in _err(gi.build([("deep", gi.ARRAY, deep)], [])[0])


@pytest.mark.gpu
def test_store_serves_every_codec(cuda):
    import torch

    rt = _rt()
    image, info, mats = _model(64)
    store = rt.TensorStore(np.frombuffer(image, np.uint8))
    assert store.device_bytes == max(i["abs_offset"] + i["bytes"] for i in info)
    rng = np.random.default_rng(1)
    for name, (t, rows, k, raw, deq) in mats.items():
        w = store.weight(name)
        assert (w.type_id, w.rows, w.k) == (t, rows, k)
        back = rt.dequantize(w).cpu().numpy()
        assert np.array_equal(back.view(np.uint32), deq.view(np.uint32)), name
        x = rng.standard_normal((2, k)).astype(np.float32)
        y = rt.decode_matvec(w, torch.from_numpy(x).to(cuda)).cpu().numpy()
        assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2, name
    with pytest.raises(rt.Qw35Error, match="no tensor named nope"):
        store.weight("nope")
    with pytest.raises(rt.Qw35Error, match="not a matrix"):
        store.weight("blk.0.attn_norm.weight")
    store.close()


@pytest.mark.gpu
def test_store_outlives_the_host_image(cuda, tmp_path):
    import torch

    rt = _rt()
    image, _, mats = _model()
    path = tmp_path / "m.gguf"
    path.write_bytes(image)
    store = rt.TensorStore.from_file(path)
    path.unlink()  # names and bytes were copied at creation
    t, rows, k, raw, deq = mats["output.weight"]
    w = store.weight("output.weight")
    x = np.ones((1, k), np.float32)
    y = rt.decode_matvec(w, torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert om.rel_l2(y, om.matvec_f64(deq, x)) <= GEMV_REL_L2


@pytest.mark.gpu
def test_store_shared_only_for_the_same_descriptors(cuda):
    """Two creates over one image share a store only when every descriptor
    matches: the same count with one tensor renamed gets a store of its own,
    which serves the new name."""
    import ctypes as C

    from qwowl35_amd import _ffi

    rt = _rt()
    image, _, mats = _model(64)
    _, _, (descs, n, keep) = rt.gguf_parse(np.frombuffer(image, np.uint8))
    ptr, size, _ = rt._image_ptr(keep)
    a = _ffi.call("qw35_hip_store_create", ptr, size, descs, n)
    b = _ffi.call("qw35_hip_store_create", ptr, size, descs, n)
    other = (_ffi.TensorDesc * n)()
    C.memmove(other, descs, C.sizeof(other))
    i = next(j for j in range(n) if C.string_at(descs[j].name, descs[j].name_len) == b"output.weight")
    new_name = C.create_string_buffer(b"output.renamed")
    other[i].name = C.cast(new_name, C.c_void_p).value
    other[i].name_len = len(b"output.renamed")
    c = _ffi.call("qw35_hip_store_create", ptr, size, other, n)
    try:
        assert a == b and c != a
        w = _ffi.Weight()
        _ffi.call("qw35_hip_store_weight", C.c_void_p(c), b"output.renamed", len(b"output.renamed"), C.byref(w))
        assert (w.rows, w.k) == (mats["output.weight"][1], mats["output.weight"][2])
        with pytest.raises(_ffi.Qw35Error, match="no tensor named output.renamed"):
            _ffi.call("qw35_hip_store_weight", C.c_void_p(a), b"output.renamed", len(b"output.renamed"),
                      C.byref(w))
    finally:
        for h in (a, b, c):
            _ffi.load().qw35_hip_store_destroy(C.c_void_p(h))
