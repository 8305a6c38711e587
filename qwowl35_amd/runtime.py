"""Host-side mirror of the reference's per-op encoder API, over the C ABI.

Names and argument meaning follow the reference runtime's encoders
(qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m):

* ``decode_matvec``       <- ``encodeDecodeMatvecTensor:weight:input:inputOffset:dst:residual:`` (:184-256)
* ``ffn_gate_up_swiglu``  <- ``encodeGf4FusedFfn`` / ``qw35_ffn_gate_up_swiglu_gf4_f32`` (:13-35)
* ``matvec_batch``        <- ``encodeMatvecBatch`` (:260-306)
* ``matmul_prefill``      <- ``encodeTiledKMatmul`` / ``qw35_mul_mm_gf4_f32`` (:309-366)
* ``output_argmax``       <- the greedy path of ``encodeOutputHead`` (Qw35MetalRuntime+Output.m:11-65)
* ``dequantize``          <- the per-codec dequant helpers / ``qw35_get_rows_*`` gathers
* ``prefill_image``       <- the half dequantisation of ``qw35_kernel_mul_mm``'s weight tiles
  (qw35_tiled_mm.metal:199-255), made once: an F16 weight for ``matmul_prefill``
* ``DecodePlan``          <- the per-token recording of ``evalToken`` (Qw35MetalRuntime.m:807-880)
* ``quantize``            <- ``pack_ffn_gf4`` / ``pack_gf4_prepared`` (tools/qw35_cook_common.py:83-119,182-199)

Device memory and streams come from torch (plumbing only); every computation
is a call into ``libqw35_hip.so``.  Errors raise ``Qw35Error`` with the
library's message, the Python form of the reference's 0 + err-buffer return.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _ffi
from ._ffi import Qw35Error, TYPE_F16, TYPE_GF2, TYPE_GF4, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0  # noqa: F401

_ROW_BYTES = {
    TYPE_GF4: lambda k: (k + 7) // 8 * 4,
    TYPE_Q8_0: lambda k: (k + 31) // 32 * 34,
    TYPE_Q4_K: lambda k: (k + 255) // 256 * 144,
    TYPE_Q5_K: lambda k: (k + 255) // 256 * 176,
    TYPE_GF2: lambda k: (k + 15) // 16 * 5,
    TYPE_Q6_K: lambda k: (k + 255) // 256 * 210,
    TYPE_F16: lambda k: 2 * k,
}


def row_bytes(type_id: int, k: int) -> int:
    try:
        return _ROW_BYTES[type_id](k)
    except KeyError:
        raise Qw35Error(f"unsupported tensor type {type_id}") from None


@dataclass
class HipWeight:
    """A weight tensor in HBM plus its C-ABI view (``qw35_hip_weight``)."""

    storage: torch.Tensor | None  # uint8 device tensor holding the raw GGUF bytes (None: owned by `owner`)
    view: _ffi.Weight
    owner: object = None  # keeps a TensorStore alive while its weights are in use

    @property
    def type_id(self) -> int:
        return int(self.view.type_id)

    @property
    def rows(self) -> int:
        return int(self.view.rows)

    @property
    def k(self) -> int:
        return int(self.view.k)

    @property
    def prefill(self) -> "HipWeight":
        """The weight ``matmul_prefill`` takes: itself for GF4 / F16 / q8_0 /
        Q4_K (q8_0 and Q4_K are dequantised inside the prefill kernel), else
        its fp16 prefill image (``prefill_image``), made on first use and kept."""
        if self.type_id in (TYPE_GF4, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K):
            return self
        img = getattr(self, "_prefill", None)
        if img is None:
            img = prefill_image(self)
            self._prefill = img
        return img

    @classmethod
    def upload(cls, raw, type_id: int, rows: int, k: int, device="cuda") -> "HipWeight":
        """Copy raw tensor bytes (numpy / torch, any shape) into HBM and validate."""
        t = torch.as_tensor(raw).reshape(-1).view(torch.uint8)
        if t.numel() != rows * row_bytes(type_id, k):
            raise Qw35Error(f"{rows}x{k} type {type_id} takes {rows * row_bytes(type_id, k)} bytes, got {t.numel()}")
        dev = torch.empty(t.numel(), dtype=torch.uint8, device=device)
        dev.copy_(t)
        return cls.from_device(dev, type_id, rows, k)

    @classmethod
    def from_device(cls, storage: torch.Tensor, type_id: int, rows: int, k: int, offset: int = 0,
                    nbytes: int | None = None) -> "HipWeight":
        """View ``nbytes`` at ``offset`` of a device byte buffer as a rows x k tensor
        through ``qw35_hip_weight_view`` (the descriptor path a GGUF loader uses)."""
        desc = _ffi.TensorDesc()
        desc.name = None
        desc.name_len = 0
        desc.dims[0] = k
        desc.dims[1] = rows
        desc.dims[2] = 1
        desc.dims[3] = 1
        desc.n_dims = 2
        desc.type_id = type_id
        desc.abs_offset = offset
        desc.bytes = nbytes if nbytes is not None else rows * row_bytes(type_id, k)
        desc.elements = rows * k
        have = storage.numel() * storage.element_size()
        if not storage.is_cuda or not storage.is_contiguous():
            raise Qw35Error("weight storage must be a contiguous device tensor")
        if offset < 0 or offset + desc.bytes > have:
            raise Qw35Error(f"weight bytes [{offset}, {offset + desc.bytes}) exceed the {have}-byte storage")
        w = _ffi.Weight()
        _ffi.call("qw35_hip_weight_view", C.byref(desc), C.c_void_p(storage.data_ptr()), C.byref(w))
        return cls(storage, w)


def _device_of(w: HipWeight) -> torch.device:
    if w.storage is not None:
        return w.storage.device
    return torch.device("cuda", torch.cuda.current_device())


@dataclass
class GgufTensor:
    """One tensor info of a GGUF image (``qw35_hip_gguf_parse``)."""

    name: str
    dims: tuple
    type_id: int
    abs_offset: int
    bytes: int
    elements: int


def _image_ptr(image) -> tuple[C.c_void_p, int, object]:
    """(pointer, size, keep-alive) of a host byte image (bytes, bytearray, mmap, numpy uint8)."""
    import numpy as np

    arr = np.frombuffer(image, dtype=np.uint8) if not isinstance(image, np.ndarray) else image.reshape(-1)
    if arr.dtype != np.uint8 or not arr.flags.c_contiguous:
        raise Qw35Error("GGUF image must be contiguous bytes")
    return C.c_void_p(arr.ctypes.data), int(arr.size), arr


def gguf_parse(image) -> tuple[list[GgufTensor], int, list]:
    """Parse a GGUF v3 image (host bytes).  Returns (tensors, data section
    offset, the raw ``TensorDesc`` array whose names point into ``image``)."""
    ptr, size, keep = _image_ptr(image)
    n = C.c_uint32(0)
    off = C.c_uint64(0)
    _ffi.call("qw35_hip_gguf_parse", ptr, size, None, 0, C.byref(n), C.byref(off))
    descs = (_ffi.TensorDesc * max(1, n.value))()
    _ffi.call("qw35_hip_gguf_parse", ptr, size, descs, n.value, C.byref(n), C.byref(off))
    out = []
    for i in range(n.value):
        d = descs[i]
        name = C.string_at(d.name, d.name_len).decode("utf-8", errors="replace") if d.name_len else ""
        out.append(GgufTensor(name, tuple(int(d.dims[j]) for j in range(min(4, d.n_dims))), int(d.type_id),
                              int(d.abs_offset), int(d.bytes), int(d.elements)))
    return out, int(off.value), (descs, n.value, keep)


class TensorStore:
    """GGUF tensors resident in HBM (``qw35_hip_store_*``, the counterpart of
    the reference's Qw35TensorStore): the image is parsed, copied to the device
    once, and ``weight(name)`` returns a ``HipWeight`` view."""

    def __init__(self, image):
        self.tensors, self.data_offset, (descs, n, keep) = gguf_parse(image)
        ptr, size, _ = _image_ptr(keep)
        self._h = _ffi.call("qw35_hip_store_create", ptr, size, descs, n)
        self.by_name = {t.name: t for t in self.tensors}

    @classmethod
    def from_file(cls, path) -> "TensorStore":
        import numpy as np

        return cls(np.memmap(path, dtype=np.uint8, mode="r"))

    def weight(self, name: str) -> HipWeight:
        w = _ffi.Weight()
        raw = name.encode()
        _ffi.call("qw35_hip_store_weight", C.c_void_p(self._h), raw, len(raw), C.byref(w))
        return HipWeight(None, w, owner=self)

    @property
    def device_bytes(self) -> int:
        return int(_ffi.load().qw35_hip_store_bytes(C.c_void_p(self._h)))

    def close(self) -> None:
        if getattr(self, "_h", None):
            torch.cuda.synchronize()
            _ffi.load().qw35_hip_store_destroy(C.c_void_p(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(t: torch.Tensor | None) -> C.c_void_p:
    return C.c_void_p(t.data_ptr() if t is not None else None)


def _stream(stream) -> C.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def _check_act(x: torch.Tensor, k: int, name: str) -> int:
    if x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous():
        raise Qw35Error(f"{name} must be a contiguous fp32 device tensor")
    if x.dim() not in (1, 2) or x.shape[-1] != k:
        raise Qw35Error(f"{name} must be [k] or [n_batch, k] with k={k}, got {tuple(x.shape)}")
    nb = 1 if x.dim() == 1 else int(x.shape[0])
    if not 1 <= nb <= _ffi.MAX_BATCH:
        raise Qw35Error(f"{name}: n_batch={nb} must be in 1..{_ffi.MAX_BATCH}")
    return nb


def _check_out(dst: torch.Tensor, nb: int, rows: int, x: torch.Tensor, name: str) -> None:
    """dst must be a contiguous fp32 tensor on x's device holding n_batch * rows values."""
    if dst.dtype != torch.float32 or not dst.is_cuda or not dst.is_contiguous() or dst.device != x.device:
        raise Qw35Error(f"{name} must be a contiguous fp32 tensor on {x.device}")
    if dst.numel() != nb * rows:
        raise Qw35Error(f"{name} holds {dst.numel()} values, expected n_batch*rows = {nb}*{rows}")


def _check_awq(awq: torch.Tensor | None, k: int, x: torch.Tensor, name: str = "awq") -> None:
    if awq is None:
        return
    if awq.dtype != torch.float32 or not awq.is_contiguous() or awq.device != x.device or awq.numel() != k:
        raise Qw35Error(f"{name} must be a contiguous fp32 tensor of k={k} values on {x.device}")


def decode_matvec_workspace(w: HipWeight, n_batch: int, device="cuda") -> torch.Tensor | None:
    """A zero-filled K-split workspace for ``decode_matvec(..., workspace=)``
    (``qw35_hip_decode_matvec_workspace_size``), or None when the shape never splits."""
    n = int(_ffi.load().qw35_hip_decode_matvec_workspace_size(C.byref(w.view), n_batch))
    return torch.zeros(n, dtype=torch.uint8, device=device) if n else None


def decode_matvec(w: HipWeight, x: torch.Tensor, dst: torch.Tensor | None = None, residual: bool = False,
                  awq: torch.Tensor | None = None, stream=None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``dst (+)= W @ (awq * x)`` for x [k] or [n_batch, k] (n_batch <= 8).
    ``workspace`` (from ``decode_matvec_workspace``) lets batch 3..8 split K
    across workgroups (``qw35_hip_decode_matvec_ws``)."""
    nb = _check_act(x, w.k, "x")
    _check_awq(awq, w.k, x)
    if dst is None:
        dst = torch.zeros((nb, w.rows) if x.dim() == 2 else (w.rows,), dtype=torch.float32, device=x.device)
    _check_out(dst, nb, w.rows, x, "dst")
    if workspace is None:
        _ffi.call("qw35_hip_decode_matvec", C.byref(w.view), _ptr(x), _ptr(awq), _ptr(dst), nb,
                  int(bool(residual)), _stream(stream))
        return dst
    if workspace.device != x.device or not workspace.is_contiguous() or workspace.data_ptr() % 256:
        raise Qw35Error("workspace must be a contiguous, 256-byte aligned tensor on x's device")
    _ffi.call("qw35_hip_decode_matvec_ws", C.byref(w.view), _ptr(x), _ptr(awq), _ptr(dst), nb, int(bool(residual)),
              _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(stream))
    return dst


def ffn_gate_up_swiglu(gate: HipWeight, up: HipWeight, x: torch.Tensor, dst: torch.Tensor | None = None,
                       awq: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """``dst = silu(gate @ (awq*x)) * (up @ (awq*x))``."""
    nb = _check_act(x, gate.k, "x")
    _check_awq(awq, gate.k, x)
    if dst is None:
        dst = torch.empty((nb, gate.rows) if x.dim() == 2 else (gate.rows,), dtype=torch.float32, device=x.device)
    _check_out(dst, nb, gate.rows, x, "dst")
    _ffi.call("qw35_hip_ffn_gate_up_swiglu", C.byref(gate.view), C.byref(up.view), _ptr(x), _ptr(awq), _ptr(dst),
              nb, _stream(stream))
    return dst


def gemv_kernel(w: HipWeight, n_batch: int = 1, w_up: HipWeight | None = None, awq: bool = False,
                workspace: bool = False) -> dict:
    """The kernel a ``decode_matvec`` (or, with ``w_up``, ``ffn_gate_up_swiglu``)
    call launches, with a K-split workspace when ``workspace``:
    ``{"name", "grid", "block", "lds", "workspace_bytes"}`` (``qw35_hip_gemv_kernel``)."""
    name = C.create_string_buffer(160)
    g, b, l, ws = C.c_uint32(), C.c_uint32(), C.c_uint32(), C.c_uint64()
    _ffi.call("qw35_hip_gemv_kernel", C.byref(w.view), C.byref(w_up.view) if w_up is not None else None, n_batch,
              int(bool(awq)), int(bool(workspace)), name, C.sizeof(name), C.byref(g), C.byref(b), C.byref(l),
              C.byref(ws))
    return {"name": name.value.decode(), "grid": g.value, "block": b.value, "lds": l.value,
            "workspace_bytes": ws.value}


def _refuse_unchunked(w: HipWeight, what: str) -> None:
    """The C ABI's error for a q8_0 weight of k % 256 != 0 on a path that works
    in 256-column chunks (its workspace-size queries return 0 for it)."""
    if w.type_id == TYPE_Q8_0 and w.k % 256:
        raise Qw35Error(f"{what}: needs k % 256 == 0, got k={w.k} (a q8_0 weight of such k runs the decode GEMV only)")


def output_argmax_workspace(w: HipWeight, n_batch: int, device="cuda") -> torch.Tensor:
    """Device bytes for ``output_argmax`` (size from the C ABI, +256 for alignment)."""
    need = int(_ffi.load().qw35_hip_output_argmax_workspace_size(C.byref(w.view), n_batch))
    if need == 0:
        _refuse_unchunked(w, "output_argmax")
        raise Qw35Error("output_argmax: invalid weight or batch")
    return torch.empty(need + 256, dtype=torch.uint8, device=device)


def output_argmax(w: HipWeight, x: torch.Tensor, awq: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None, stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Greedy head: per batch row, (token, logit) of the largest ``W @ (awq * x)``
    entry (ties to the smaller row, NaN never chosen), without materialising
    the logits.  Returns (tokens [n_batch] int32 holding the uint32 row ids --
    0xFFFFFFFF reads as -1 -- and fp32 logits [n_batch]), written on ``stream``."""
    nb = _check_act(x, w.k, "x")
    _check_awq(awq, w.k, x)
    need = int(_ffi.load().qw35_hip_output_argmax_workspace_size(C.byref(w.view), nb))
    if need == 0:
        _refuse_unchunked(w, "output_argmax")
        raise Qw35Error("output_argmax: invalid weight or batch")
    if workspace is None:
        workspace = output_argmax_workspace(w, nb, device=x.device)
    base = workspace.data_ptr()
    pad = (-base) % 256
    if workspace.numel() - pad < need:
        raise Qw35Error(f"output_argmax: workspace needs {need} bytes after 256-byte alignment")
    token = torch.empty(nb, dtype=torch.int32, device=x.device)
    logit = torch.empty(nb, dtype=torch.float32, device=x.device)
    _ffi.call("qw35_hip_output_argmax", C.byref(w.view), _ptr(x), _ptr(awq), nb, _ptr(token), _ptr(logit),
              C.c_void_p(base + pad), C.c_uint64(workspace.numel() - pad), _stream(stream))
    return token, logit


def prefill_workspace(w: HipWeight, n_tokens: int, device="cuda") -> torch.Tensor:
    """Device workspace for ``matmul_prefill`` of ``n_tokens`` tokens on ``w`` (256-byte aligned uint8)."""
    n = int(_ffi.load().qw35_hip_matmul_prefill_workspace_size(C.byref(w.view), n_tokens))
    if n == 0:
        _refuse_unchunked(w, "matmul_prefill")
        raise Qw35Error(f"prefill workspace: unsupported weight or n_tokens={n_tokens}")
    return torch.empty(n, dtype=torch.uint8, device=device)  # the caching allocator aligns to 512 B


def matmul_prefill(w: HipWeight, a: torch.Tensor, awq: torch.Tensor | None = None,
                   out_dtype: torch.dtype = torch.bfloat16, dst: torch.Tensor | None = None,
                   workspace: torch.Tensor | None | bool = True, stream=None,
                   epilogue: int = _ffi.EPILOGUE_STORE) -> torch.Tensor:
    """``C[t] = (awq * a[t]) @ W^T`` for a GF4, q8_0, Q4_K or F16 weight
    (``encodeTiledKMatmul``; the other k-quants enter as their fp16 image,
    ``w.prefill``).  q8_0, Q4_K and F16 need a workspace.

    ``a``: [n_tokens, k] bf16 or fp32 device tensor; result [n_tokens, rows] in
    ``out_dtype`` (bfloat16, rounded to nearest even, or float32).
    ``workspace``: True (allocate one), a tensor from ``prefill_workspace``, or
    None/False for the path without staging (bf16 MFMA; GF4 weights, bf16
    activations, no AWQ).  With a workspace fp32 activations keep fp32
    precision (an fp16 hi/lo pair per activation) and bf16 ones are carried
    exactly (with AWQ: the product rounded once to fp16).
    ``epilogue`` (fp32 ``dst`` given, workspace): ``_ffi.EPILOGUE_STORE``
    (dst = r), ``EPILOGUE_ADD`` (dst += r) or ``EPILOGUE_SWIGLU``
    (dst = silu(dst) * r), see ``qw35_hip_matmul_prefill_epilogue``.
    """
    if a.dim() != 2 or not a.is_cuda or not a.is_contiguous() or a.dtype not in (torch.bfloat16, torch.float32):
        raise Qw35Error("matmul_prefill: a must be a contiguous 2-D bf16/fp32 device tensor")
    if a.shape[1] != w.k:
        raise Qw35Error(f"matmul_prefill: a has {a.shape[1]} columns, weight k={w.k}")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise Qw35Error("matmul_prefill: out_dtype must be bfloat16 or float32")
    n = int(a.shape[0])
    if dst is None:
        dst = torch.empty((n, w.rows), dtype=out_dtype, device=a.device)
    elif dst.dtype != out_dtype or tuple(dst.shape) != (n, w.rows) or not dst.is_contiguous():
        raise Qw35Error("matmul_prefill: dst must be a contiguous [n_tokens, rows] tensor of out_dtype")
    a_dt = _ffi.DTYPE_BF16 if a.dtype == torch.bfloat16 else _ffi.DTYPE_F32
    c_dt = _ffi.DTYPE_BF16 if out_dtype == torch.bfloat16 else _ffi.DTYPE_F32
    if workspace is True:
        workspace = prefill_workspace(w, n, device=a.device)
    elif workspace is False:
        workspace = None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _ffi.call("qw35_hip_matmul_prefill_epilogue", C.byref(w.view), _ptr(a), a_dt, _ptr(awq), _ptr(dst), c_dt,
              int(epilogue), n, _ptr(workspace), ws_bytes, _stream(stream))
    return dst


def prefill_kernel(w: HipWeight, n_tokens: int, a_dtype: torch.dtype = torch.bfloat16, awq: bool = False,
                   out_dtype: torch.dtype = torch.bfloat16, workspace: bool = True) -> dict:
    """The matmul kernel ``matmul_prefill`` launches for this call shape
    (``qw35_hip_prefill_kernel``; nothing is launched): name as the profiler
    shows it, grid, block, LDS bytes and K splits."""
    name = C.create_string_buffer(160)
    grid, block, lds, splits = C.c_uint32(), C.c_uint32(), C.c_uint32(), C.c_uint32()
    a_dt = _ffi.DTYPE_F32 if a_dtype == torch.float32 else _ffi.DTYPE_BF16
    c_dt = _ffi.DTYPE_F32 if out_dtype == torch.float32 else _ffi.DTYPE_BF16
    _ffi.call("qw35_hip_prefill_kernel", C.byref(w.view), n_tokens, a_dt, int(awq), c_dt, int(workspace), name,
              C.sizeof(name), C.byref(grid), C.byref(block), C.byref(lds), C.byref(splits))
    return {"name": name.value.decode(), "grid": grid.value, "block": block.value, "lds": lds.value,
            "splits": splits.value}


def matvec_batch(w: HipWeight, x: torch.Tensor, dst: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Multi-token matvec of fp32 activations [n_tokens, k] (``encodeMatvecBatch``, +FFN.m:260-306).

    1..8 tokens run the decode GEMV (fp32 activations); longer chunks run the
    prefill matmul with fp32 output (GF4 and q8_0 directly, the other
    k-quants through their fp16 prefill image), as the reference switches to
    its tiled matmul for multi-token chunks.  Both keep the activations at fp32
    precision (fp16 hi/lo pairs on MFMA), as the reference's tiled matmul
    keeps src1 in fp32 (qw35_tiled_mm.metal:200-224).
    """
    if x.dim() != 2:
        raise Qw35Error("matvec_batch takes [n_tokens, k] activations")
    if x.shape[0] <= _ffi.MAX_BATCH and w.type_id != TYPE_F16:
        return decode_matvec(w, x, dst, residual=False, stream=stream)
    if w.type_id == TYPE_Q8_0 and w.k % 256 != 0:
        # q8_0 rows of k % 256 != 0: the prefill matmul works in 256-column chunks,
        # so such a chunk runs the row-wise decode GEMV MAX_BATCH tokens at a time
        if dst is None:
            dst = torch.empty((x.shape[0], w.rows), dtype=torch.float32, device=x.device)
        _check_out(dst, x.shape[0], w.rows, x, "dst")
        for t0 in range(0, x.shape[0], _ffi.MAX_BATCH):
            t1 = min(t0 + _ffi.MAX_BATCH, x.shape[0])
            decode_matvec(w, x[t0:t1], dst[t0:t1], residual=False, stream=stream)
        return dst
    return matmul_prefill(w.prefill, x, out_dtype=torch.float32, dst=dst, stream=stream)


def prefill_image(w: HipWeight, stream=None) -> HipWeight:
    """fp16_rne of the dequantised weight as a new F16 ``HipWeight``
    (``qw35_hip_dequantize_f16``), the operand of ``matmul_prefill``."""
    dst = torch.empty(w.rows * w.k * 2, dtype=torch.uint8, device=_device_of(w))
    _ffi.call("qw35_hip_dequantize_f16", C.byref(w.view), _ptr(dst), _stream(stream))
    return HipWeight.from_device(dst, TYPE_F16, w.rows, w.k)


def dequantize(w: HipWeight, row_ids: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """fp32 weights [rows, k], or the gathered rows ``row_ids`` (uint32/int32 device)."""
    if row_ids is not None:
        if row_ids.dtype not in (torch.int32,) or not row_ids.is_cuda:
            raise Qw35Error("row_ids must be an int32 device tensor (read as uint32)")
        n = int(row_ids.numel())
    else:
        n = w.rows
    dst = torch.empty((n, w.k), dtype=torch.float32, device=_device_of(w))
    _ffi.call("qw35_hip_dequantize", C.byref(w.view), _ptr(row_ids), n, _ptr(dst), _stream(stream))
    return dst


def quantize(src: torch.Tensor, type_id: int, col_scale: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Encode an fp32 [rows, k] device matrix; returns the raw tensor bytes (uint8, device).

    GF4 is the reference packer ``pack_gf4_prepared(scale_search=False)`` after
    the AWQ column multiply of ``pack_ffn_gf4`` (tools/qw35_cook_common.py:83-119,
    182-199); q8_0 / Q4_K are the library's own encoders.
    """
    if src.dtype != torch.float32 or not src.is_cuda or not src.is_contiguous() or src.dim() != 2:
        raise Qw35Error("quantize: src must be a contiguous 2-D fp32 device tensor")
    if col_scale is not None and (col_scale.dtype != torch.float32 or not col_scale.is_cuda
                                  or col_scale.numel() != src.shape[1] or not col_scale.is_contiguous()):
        raise Qw35Error("quantize: col_scale must be a contiguous fp32 device tensor of length k")
    rows, k = int(src.shape[0]), int(src.shape[1])
    out = torch.empty(rows * row_bytes(type_id, k), dtype=torch.uint8, device=src.device)
    _ffi.call("qw35_hip_quantize", type_id, _ptr(src), rows, k, _ptr(col_scale), _ptr(out), _stream(stream))
    return out


def quantize_weight(src: torch.Tensor, type_id: int, col_scale: torch.Tensor | None = None,
                    stream=None) -> HipWeight:
    """``quantize`` into a new HBM tensor, returned as a GEMV-ready ``HipWeight``."""
    raw = quantize(src, type_id, col_scale, stream)
    return HipWeight.from_device(raw, type_id, int(src.shape[0]), int(src.shape[1]))


class DecodePlan:
    """A per-token sequence of projection GEMVs recorded once into a hipGraph
    (``qw35_hip_plan_*``), the counterpart of the per-token recording in
    ``evalToken`` / ``encodeDecodeLayers`` (Qw35MetalRuntime.m:807-880,1170-1221).

    Build with ``matvec`` / ``swiglu`` calls naming device buffers, then
    ``record()``; ``launch()`` replays the whole sequence.  The tensors named in
    the ops are referenced by the plan and must stay alive (and in place).
    """

    def __init__(self):
        self._ops: list[_ffi.PlanOp] = []
        self._keep: list = []
        self._handle = None

    def matvec(self, w: HipWeight, x: torch.Tensor, dst: torch.Tensor, residual: bool = False,
               awq: torch.Tensor | None = None) -> "DecodePlan":
        nb = _check_act(x, w.k, "x")
        _check_awq(awq, w.k, x)
        _check_out(dst, nb, w.rows, x, "dst")
        self._add(_ffi.OP_MATVEC, nb, residual, w, None, x, awq, dst)
        return self

    def swiglu(self, gate: HipWeight, up: HipWeight, x: torch.Tensor, dst: torch.Tensor,
               awq: torch.Tensor | None = None) -> "DecodePlan":
        nb = _check_act(x, gate.k, "x")
        _check_awq(awq, gate.k, x)
        _check_out(dst, nb, gate.rows, x, "dst")
        self._add(_ffi.OP_SWIGLU, nb, False, gate, up, x, awq, dst)
        return self

    def argmax(self, w: HipWeight, x: torch.Tensor, token: torch.Tensor, logit: torch.Tensor,
               awq: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> "DecodePlan":
        """The greedy head as a plan op: ``token[b]`` / ``logit[b]`` (int32 / fp32
        device, n_batch each) of the largest ``W @ (awq * x[b])`` entry."""
        nb = _check_act(x, w.k, "x")
        _check_awq(awq, w.k, x)
        _check_out(logit, nb, 1, x, "logit")
        if token.dtype != torch.int32 or not token.is_contiguous() or token.numel() != nb or token.device != x.device:
            raise Qw35Error(f"token must be a contiguous int32 tensor of n_batch={nb} values on {x.device}")
        if workspace is None:
            workspace = output_argmax_workspace(w, nb, device=x.device)
        base = workspace.data_ptr()
        pad = (-base) % 256
        self._add(_ffi.OP_ARGMAX, nb, False, w, None, x, awq, logit)
        op = self._ops[-1]
        op.token = token.data_ptr()
        op.workspace = base + pad
        op.workspace_bytes = workspace.numel() - pad
        self._keep.extend([token, workspace])
        return self

    def matmul(self, w: HipWeight, x: torch.Tensor, dst: torch.Tensor, workspace: torch.Tensor,
               residual: bool = False, awq: torch.Tensor | None = None) -> "DecodePlan":
        """A prefill-chunk op: ``dst (+)= (awq * x) @ W^T`` for fp32 ``x`` [n_tokens, k]
        on the prefill matmul (``w.prefill``), through ``workspace`` (ops may share one)."""
        n = self._check_chunk(w.prefill, x, dst, awq, workspace)
        self._add(_ffi.OP_MATMUL, n, residual, w.prefill, None, x, awq, dst)
        self._set_ws(workspace)
        return self

    def matmul_swiglu(self, gate: HipWeight, up: HipWeight, x: torch.Tensor, dst: torch.Tensor,
                      workspace: torch.Tensor, awq: torch.Tensor | None = None) -> "DecodePlan":
        """``dst = silu((awq*x) @ Wg^T) * ((awq*x) @ Wu^T)`` over a chunk: two prefill
        matmul launches, the second applying SwiGLU in its epilogue."""
        n = self._check_chunk(gate.prefill, x, dst, awq, workspace)
        self._add(_ffi.OP_MATMUL_SWIGLU, n, False, gate.prefill, up.prefill, x, awq, dst)
        self._set_ws(workspace)
        return self

    def _check_chunk(self, w, x, dst, awq, workspace) -> int:
        if x.dim() != 2 or x.dtype != torch.float32 or not x.is_contiguous() or x.shape[1] != w.k:
            raise Qw35Error(f"chunk op: x must be a contiguous fp32 [n_tokens, {w.k}] tensor")
        _check_awq(awq, w.k, x)
        n = int(x.shape[0])
        if dst.dtype != torch.float32 or not dst.is_contiguous() or dst.numel() < n * w.rows:
            raise Qw35Error(f"chunk op: dst must be a contiguous fp32 tensor of >= {n} x {w.rows} values")
        if workspace is None or workspace.dtype != torch.uint8 or not workspace.is_cuda:
            raise Qw35Error("chunk op: a uint8 device workspace (prefill_workspace) is required")
        return n

    def _set_ws(self, workspace: torch.Tensor) -> None:
        base = workspace.data_ptr()
        pad = (-base) % 256
        op = self._ops[-1]
        op.workspace = base + pad
        op.workspace_bytes = workspace.numel() - pad
        self._keep.append(workspace)

    def _add(self, kind, nb, residual, w, up, x, awq, dst):
        if self._handle is not None:
            raise Qw35Error("plan already recorded")
        op = _ffi.PlanOp()
        op.kind = kind
        op.n_batch = nb
        op.residual = int(bool(residual))
        op.w = C.pointer(w.view)
        op.w_up = C.pointer(up.view) if up is not None else None
        op.x = x.data_ptr()
        op.awq = awq.data_ptr() if awq is not None else None
        op.dst = dst.data_ptr()
        self._ops.append(op)
        self._keep.extend([w, up, x, awq, dst])

    def record(self) -> "DecodePlan":
        arr = (_ffi.PlanOp * len(self._ops))(*self._ops)
        self._handle = C.c_void_p(_ffi.call("qw35_hip_plan_create", arr, len(self._ops)))
        return self

    def __len__(self) -> int:
        return int(_ffi.load().qw35_hip_plan_size(self._handle)) if self._handle else len(self._ops)

    def launch(self, stream=None) -> None:
        if self._handle is None:
            raise Qw35Error("plan_launch: plan not recorded")
        _ffi.call("qw35_hip_plan_launch", self._handle, _stream(stream))

    def close(self) -> None:
        if self._handle is not None:
            _ffi.load().qw35_hip_plan_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _hip_runtime() -> C.CDLL:
    """The process's HIP runtime (the one torch and libqw35_hip.so share, soname
    libamdhip64.so.7): plumbing for copies into library-owned device buffers."""
    _ffi.load()
    lib = C.CDLL("libamdhip64.so.7")
    lib.hipMemcpy.restype = C.c_int
    lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return lib


_HIP_MEMCPY_DEFAULT = 4  # hipMemcpyDefault: direction from the (unified) addresses


def hparams_struct(hp) -> _ffi.Hparams:
    """``qw35_hip_hparams`` from an object with the projection fields (e.g. ``qwen35.Hparams``)."""
    h = _ffi.Hparams()
    for name, _ in _ffi.Hparams._fields_:
        if name == "rope_sections" or not hasattr(hp, name):
            continue
        setattr(h, name, getattr(hp, name))
    return h


class ProjectionRuntime:
    """The projection runtime (``qw35_hip_runtime_*``): the in-scope part of the
    reference's ``qw35_metal_runtime_*`` ABI (Qw35FFI.h:19-118).

    Built from a GGUF image (host bytes or an mmap) and the hyper-parameters;
    ``write(which, x)`` fills an input buffer (``_ffi.RT_NORM`` / ``RT_CORE`` /
    ``RT_ACT``), ``eval_step(n_batch, mode)`` replays one decode step's
    projections, ``eval_chunk(n_tokens, mode)`` one prefill chunk's (the
    projection part of ``qw35_metal_runtime_eval_tokens``), and ``argmax()`` /
    ``copy_logits()`` / ``read(which, n)`` wait and read back, as
    ``qw35_metal_runtime_argmax`` / ``copy_logits`` do.
    """

    def __init__(self, image, hparams, vocab: int, max_batch: int = 1, prefill_chunk: int = 0):
        self._h = None
        tensors, _, (descs, n, keep) = gguf_parse(image)
        ptr, size, _ = _image_ptr(keep)
        self._keep = keep
        self.tensors = tensors
        self.hparams = hparams_struct(hparams)
        self.vocab = int(vocab)
        self.max_batch = int(max_batch)
        self.prefill_chunk = int(prefill_chunk)
        self.rows = max(self.max_batch, self.prefill_chunk)  # rows of the activation buffers
        self._h = C.c_void_p(_ffi.call("qw35_hip_runtime_create", ptr, size, descs, n, C.byref(self.hparams),
                                       self.vocab, self.max_batch, self.prefill_chunk))
        self._hip = _hip_runtime()
        self.last_batch = 0

    def buffer(self, which: int) -> tuple[int, int]:
        """(device address, width in floats) of runtime buffer ``which``."""
        p, w = C.c_void_p(), C.c_uint64()
        _ffi.call("qw35_hip_runtime_buffer", self._h, which, C.byref(p), C.byref(w))
        return int(p.value or 0), int(w.value)

    @property
    def store_base(self) -> int:
        return int(_ffi.load().qw35_hip_store_device_base(_ffi.load().qw35_hip_runtime_store(self._h)) or 0)

    def _copy(self, dst: int, src: int, nbytes: int) -> None:
        rc = self._hip.hipMemcpy(C.c_void_p(dst), C.c_void_p(src), nbytes, _HIP_MEMCPY_DEFAULT)
        if rc != 0:
            raise Qw35Error(f"hipMemcpy failed ({rc})")

    def _rows_of(self, which: int) -> int:
        return self.max_batch if which == _ffi.RT_LOGITS else self.rows

    def write(self, which: int, x: torch.Tensor) -> None:
        """Copy fp32 [n, width'] (contiguous, any device) into buffer ``which``:
        n rows packed at the row length width' of the op that reads them."""
        torch.cuda.synchronize()
        self.sync()
        ptr, width = self.buffer(which)
        cap = width * self._rows_of(which)
        if x.dtype != torch.float32 or not x.is_contiguous() or x.numel() > cap or not ptr:
            raise Qw35Error(f"write: fp32 contiguous data of at most {cap} floats")
        self._copy(ptr, x.data_ptr(), x.numel() * 4)

    def read(self, which: int, n_floats: int) -> torch.Tensor:
        """The first ``n_floats`` of buffer ``which`` (after waiting), as a CPU tensor."""
        self.sync()
        ptr, width = self.buffer(which)
        if n_floats > width * self._rows_of(which):
            raise Qw35Error("read: more floats than the buffer holds")
        out = torch.empty(n_floats, dtype=torch.float32)
        self._copy(out.data_ptr(), ptr, n_floats * 4)
        return out

    def eval_step(self, n_batch: int = 1, mode: int = _ffi.LOGITS_FULL) -> None:
        _ffi.call("qw35_hip_runtime_eval_step", self._h, n_batch, mode)
        self.last_batch = n_batch

    def eval_chunk(self, n_tokens: int, mode: int = _ffi.LOGITS_FULL) -> None:
        """One prefill chunk's projections over ``n_tokens`` rows; the head on the last token."""
        _ffi.call("qw35_hip_runtime_eval_chunk", self._h, n_tokens, mode)
        self.last_batch = 1

    def argmax(self) -> tuple[list[int], list[float]]:
        tok = (C.c_uint32 * self.last_batch)()
        lg = (C.c_float * self.last_batch)()
        _ffi.call("qw35_hip_runtime_argmax", self._h, tok, lg)
        return list(tok), list(lg)

    def copy_logits(self) -> torch.Tensor:
        out = torch.empty((self.last_batch, self.vocab), dtype=torch.float32)
        _ffi.call("qw35_hip_runtime_copy_logits", self._h, C.c_void_p(out.data_ptr()), out.numel())
        return out

    def sync(self) -> None:
        _ffi.call("qw35_hip_runtime_sync", self._h)

    def close(self) -> None:
        if self._h:
            _ffi.load().qw35_hip_runtime_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def stream_read(buf: torch.Tensor, sink: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Streaming-read probe over a device buffer (measures the HBM read ceiling);
    returns the per-workgroup XOR digests (int32 view of uint32)."""
    nbytes = buf.numel() * buf.element_size()
    n = int(_ffi.load().qw35_hip_stream_read_sink_len(nbytes))
    if sink is None:
        sink = torch.empty(n, dtype=torch.int32, device=buf.device)
    _ffi.call("qw35_hip_stream_read", _ptr(buf), nbytes, _ptr(sink), _stream(stream))
    return sink


MFMA_PROBE_FLOPS_PER_WG_ITER = 4 * 8 * 32768  # waves x MFMAs per round x flops per 32x32x16 MFMA


def mfma_probe(n_workgroups: int, iters: int, sink: torch.Tensor | None = None, stream=None,
               device="cuda") -> torch.Tensor:
    """MFMA throughput probe (fp16 32x32x16, no memory traffic): the work is
    ``n_workgroups * iters * MFMA_PROBE_FLOPS_PER_WG_ITER`` flops; returns the sink."""
    if sink is None:
        sink = torch.empty(n_workgroups * 256, dtype=torch.float32, device=device)
    _ffi.call("qw35_hip_mfma_probe", n_workgroups, iters, _ptr(sink), _stream(stream))
    return sink


def sync(stream=None) -> None:
    _ffi.call("qw35_hip_sync", _stream(stream))
