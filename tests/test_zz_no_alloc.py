"""The greedy head's no-allocation entry point (qw35_hip_output_argmax_noalloc),
called through the C ABI: it must give the same token and logit, bit for
bit, as qw35_hip_output_argmax with a caller-owned workspace (the same
kernels), on two calls in a row on one device (the second with a smaller
head and batch, so the library's array holds the first call's partials when
the second starts), and reject a head whose partials exceed its array."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _call_noalloc(w, x, awq):
    import torch

    from qwowl35_amd import _ffi

    nb = 1 if x.dim() == 1 else int(x.shape[0])
    token = torch.full((nb,), -7, dtype=torch.int32, device=x.device)
    logit = torch.full((nb,), float("nan"), dtype=torch.float32, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    _ffi.call("qw35_hip_output_argmax_noalloc", C.byref(w.view), C.c_void_p(x.data_ptr()),
              C.c_void_p(awq.data_ptr() if awq is not None else None), nb, C.c_void_p(token.data_ptr()),
              C.c_void_p(logit.data_ptr()), C.c_void_p(stream))
    return token, logit


def _head(cuda, type_id, rows, k, seed):
    import torch

    from qwowl35_amd import qwen35

    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    return qwen35.synthetic_weight(g, type_id, rows, k)


@pytest.mark.parametrize("type_id", [14, 12, 8, 100])
def test_noalloc_argmax_matches_workspace_entry_point(cuda, type_id):
    import torch

    from qwowl35_amd import runtime as rt

    cases = [(65549, 8, 1), (3001, 2, 2)]  # second call: fewer rows and batch rows
    for rows, nb, seed in cases:
        print(f"noalloc argmax type {type_id} rows {rows} nb {nb}", flush=True)
        w = _head(cuda, type_id, rows, 4096, seed)
        g = torch.Generator(device=cuda)
        g.manual_seed(100 + seed)
        x = torch.randn((nb, 4096), generator=g, device=cuda)
        awq = torch.rand((4096,), generator=g, device=cuda) * 1.5 + 0.5
        tok_ws, lg_ws = rt.output_argmax(w, x, awq=awq)
        tok, lg = _call_noalloc(w, x, awq)
        torch.cuda.synchronize()
        assert torch.equal(tok, tok_ws), (rows, nb)
        assert np.array_equal(lg.cpu().numpy().view(np.uint32), lg_ws.cpu().numpy().view(np.uint32)), (rows, nb)
        tok2, lg2 = _call_noalloc(w, x, None)
        tok2_ws, lg2_ws = rt.output_argmax(w, x)
        torch.cuda.synchronize()
        assert torch.equal(tok2, tok2_ws) and torch.equal(lg2, lg2_ws), (rows, nb)


def test_noalloc_argmax_rejects_oversized_head(cuda):
    """A head whose per-workgroup partials exceed the library's array is
    refused before any launch (the weight is only described, never read)."""
    import torch

    from qwowl35_amd import _ffi

    rows, k = 1 << 24, 4096
    w = _ffi.Weight()
    w.data = 256  # never dereferenced: validation fails first
    w.k = k
    w.rows = rows
    w.bytes = rows * k // 2
    w.type_id = 100
    x = torch.zeros((8, k), dtype=torch.float32, device=cuda)
    out = torch.zeros(8, dtype=torch.int32, device=cuda)
    err = C.create_string_buffer(512)
    rc = _ffi.load().qw35_hip_output_argmax_noalloc(C.byref(w), C.c_void_p(x.data_ptr()), None, 8,
                                                    C.c_void_p(out.data_ptr()), C.c_void_p(out.data_ptr()), None,
                                                    err, C.sizeof(err))
    assert rc == 0
    assert b"exceed" in err.value
