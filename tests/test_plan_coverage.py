"""Every GEMV kernel instantiation that the benchmark and the 9B decode stack
launch is also launched by a GPU parity test.

The launch planners pick a kernel (template parameters: batch, row tiles,
waves, chunks per wave, loads in flight, fused SwiGLU, AWQ) from the weight's
shape, so a parity test at a small shape does not cover a large shape's
kernel.  qw35_hip_gemv_kernel names the kernel a call would launch without a
GPU; this test lists the shapes each GPU parity test runs and the shapes the
benchmark and the 9B stack run, and checks the second set of kernels is inside
the first.
"""
from __future__ import annotations

import ctypes as C

import pytest

from qwowl35_amd import _ffi

GF4, Q8, Q4K, Q5K, Q6K, GF2 = 100, 8, 12, 13, 14, 101
ROW_BYTES = {GF4: lambda k: k // 8 * 4, Q8: lambda k: k // 32 * 34, Q4K: lambda k: k // 256 * 144,
             Q5K: lambda k: k // 256 * 176, Q6K: lambda k: k // 256 * 210, GF2: lambda k: k // 256 * 80}


def kernel(t, rows, k, nb, swiglu=False, awq=False, ws=False) -> str:
    """Kernel name, with "+split<S>" when the launch splits K (a plan or a workspace call)."""
    w = _ffi.Weight()
    w.data, w.k, w.rows, w.type_id = 256, k, rows, t
    w.bytes = ROW_BYTES[t](k) * rows
    name = C.create_string_buffer(160)
    g = C.c_uint32()
    wsb = C.c_uint64()
    _ffi.call("qw35_hip_gemv_kernel", C.byref(w), C.byref(w) if swiglu else None, nb, int(awq), int(ws), name, 160,
              C.byref(g), None, None, C.byref(wsb))
    n = name.value.decode()
    return n + (f"+split/{g.value}" if wsb.value else "")


def nine_b_stack(nb, ffn_awq):
    """Launches of one 9B decode step as a plan records them (with its K-split
    workspace; merged mixer launches are planned on their total rows)."""
    out = {kernel(Q8, 8192 + 4096 + 32 + 32, 4096, nb, ws=True),     # DeltaNet qkv + gate + beta + alpha
           kernel(Q8, 8192 + 1024 + 1024, 4096, nb, ws=True),        # attention q + k + v
           kernel(Q8, 4096, 4096, nb, ws=True),                      # ssm_out / attn_output
           kernel(GF4, 12288, 4096, nb, swiglu=True, awq=ffn_awq, ws=True),
           kernel(GF4, 4096, 12288, nb, ws=True),                    # ffn_down
           kernel(Q4K, 248320, 4096, nb, ws=True)}                   # output.weight
    return out


# tests/test_gpu_full_shapes.py::test_k_split_workspace
SPLIT_CASES = [(GF4, 4096, 12288), (Q4K, 4096, 12288), (Q8, 4096, 12288), (Q6K, 4000, 12288), (Q5K, 1000, 12288),
               (GF2, 4096, 12288), (GF4, 2072, 12288), (Q8, 4096, 4096), (GF4, 1000, 12288)]


def parity_test_kernels() -> set[str]:
    s = set()
    # tests/test_gpu_stack9b.py (AWQ on and off on the FFN)
    for nb in (1, 8):
        s |= nine_b_stack(nb, ffn_awq=True) | nine_b_stack(nb, ffn_awq=False)
    # tests/test_gpu_full_shapes.py
    for nb in (1, 2, 8):
        for rows, k in ((8192, 4096), (12288, 4096), (4096, 12288)):
            s.add(kernel(Q8, rows, k, nb))
    for nb in (1, 8):
        s.add(kernel(Q8, 12352, 4096, nb))
    for nb in (1, 2, 4, 8):
        s.add(kernel(GF4, 12288, 4096, nb, swiglu=True, awq=True))
        s.add(kernel(GF4, 4096, 12288, nb, awq=True))
        s.add(kernel(GF4, 4096, 12288, nb))
        s.add(kernel(GF4, 12288, 4096, nb))
    for nb in (1, 4, 8):
        for t in (Q8, Q4K, Q5K, Q6K, GF2):
            s.add(kernel(t, 65549, 4096, nb))
    for nb in (4, 5, 8):  # test_k_split_workspace
        for t, rows, k in SPLIT_CASES:
            s.add(kernel(t, rows, k, nb, ws=True))
    # tests/test_gpu_gemv.py::test_gemv_parity (small shapes; q8_0 37 x 4096 takes the 16-wave plan)
    for nb in (1, 2, 3, 8):
        for t in (GF4, GF2, Q8, Q4K, Q5K):
            for rows, k in ((1, 256), (37, 4096), (130, 12288), (5, 8192), (64, 1024)):
                s.add(kernel(t, rows, k, nb))
    return s


def benchmarked() -> dict[str, str]:
    """kernel -> the bench line that launches it."""
    b = {}

    def add(what, *args, **kw):
        b.setdefault(kernel(*args, **kw), what)

    # bench.py's GEMV lines take a K-split workspace (gemv_line)
    add("headline gf4 b1", GF4, 12288, 4096, 1, ws=True)
    for nb in (2, 4, 8):
        add(f"gf4 b{nb} 12288x4096", GF4, 12288, 4096, nb, ws=True)
    for nb in (1, 8):
        add(f"gf4 b{nb} 4096x12288", GF4, 4096, 12288, nb, ws=True)
    for rows, k in ((8192, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (4096, 12288)):
        add(f"q8_0 layer set {rows}x{k}", Q8, rows, k, 1)
    add("q8_0 plan q/k/v", Q8, 10240, 4096, 1, ws=True)
    add("q8_0 plan gate/up", Q8, 24576, 4096, 1, ws=True)
    for nb in (1, 8):
        add(f"q4_k down b{nb}", Q4K, 4096, 12288, nb, ws=True)
        add(f"q4_k head b{nb}", Q4K, 248320, 4096, nb, ws=True)
        add(f"q6_k head b{nb}", Q6K, 248320, 4096, nb, ws=True)
        for k in nine_b_stack(nb, ffn_awq=False):
            b.setdefault(k, f"9B stack b{nb}")
    return b


@pytest.fixture(scope="module")
def lib():
    return _ffi.load()


def test_every_benchmarked_kernel_has_a_parity_test(lib):
    covered = parity_test_kernels()
    missing = {k: what for k, what in benchmarked().items() if k not in covered}
    assert not missing, missing


def test_kernel_query_matches_launch_shape(lib):
    """The query's grid is the row-tile count of the named plan."""
    w = _ffi.Weight()
    w.data, w.k, w.rows, w.type_id = 256, 4096, 12288, GF4
    w.bytes = ROW_BYTES[GF4](4096) * 12288
    name = C.create_string_buffer(160)
    g, b, lds = C.c_uint32(), C.c_uint32(), C.c_uint32()
    _ffi.call("qw35_hip_gemv_kernel", C.byref(w), None, 1, 0, 0, name, 160, C.byref(g), C.byref(b), C.byref(lds),
              None)
    rt, ks = [int(v) for v in name.value.decode().split("<")[1].split(",")[1:3]]
    assert g.value == -(-12288 // (16 * rt)) and b.value == 64 * ks and 0 < lds.value <= 160 * 1024
    with pytest.raises(_ffi.Qw35Error, match="n_batch=9"):
        kernel(GF4, 12288, 4096, 9)
