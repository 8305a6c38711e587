"""ctypes binding of ``include/qw35_hip.h`` (the library's C ABI).

The prototypes here are the ones a Rust/C host binds; tests and the benchmark
call the library only through them.  Loading fails loudly when the built
library is missing: there is no CPU fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqw35_hip.so"

TYPE_F16 = 1
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_GF2 = 101
TYPE_Q6_K = 14
TYPE_GF4 = 100
MAX_BATCH = 8
DTYPE_F32 = 0
DTYPE_BF16 = 1


class TensorDesc(C.Structure):
    """``qw35_hip_tensor_desc`` == ``qw35_metal_tensor_desc`` (Qw35MetalTypes.h:18-27)."""

    _fields_ = [
        ("name", C.c_void_p),
        ("name_len", C.c_size_t),
        ("dims", C.c_uint64 * 4),
        ("n_dims", C.c_uint32),
        ("type_id", C.c_uint32),
        ("abs_offset", C.c_uint64),
        ("bytes", C.c_uint64),
        ("elements", C.c_uint64),
    ]


class Weight(C.Structure):
    """``qw35_hip_weight``."""

    _fields_ = [
        ("data", C.c_void_p),
        ("k", C.c_uint64),
        ("rows", C.c_uint64),
        ("bytes", C.c_uint64),
        ("type_id", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


OP_MATVEC = 0
OP_SWIGLU = 1


class PlanOp(C.Structure):
    """``qw35_hip_plan_op``."""

    _fields_ = [
        ("kind", C.c_uint32),
        ("n_batch", C.c_uint32),
        ("residual", C.c_int32),
        ("reserved", C.c_uint32),
        ("w", C.POINTER(Weight)),
        ("w_up", C.POINTER(Weight)),
        ("x", C.c_void_p),
        ("awq", C.c_void_p),
        ("dst", C.c_void_p),
        ("token", C.c_void_p),
        ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_uint64),
    ]


OP_ARGMAX = 2
OP_MATMUL = 3
OP_MATMUL_SWIGLU = 4

# Prefill matmul epilogues (QW35_HIP_EPILOGUE_*).
EPILOGUE_STORE = 0
EPILOGUE_ADD = 1
EPILOGUE_SWIGLU = 2
MAX_PREFILL_CHUNK = 4096

LOGITS_NONE = 0
LOGITS_ARGMAX = 1
LOGITS_FULL = 2

# Runtime buffers (QW35_HIP_RT_*).
RT_NORM, RT_CORE, RT_ACT, RT_QKV, RT_K, RT_V, RT_Z, RT_BETA, RT_ALPHA, RT_FFN, RT_LOGITS = range(11)
RT_NBUF = 11


class Hparams(C.Structure):
    """``qw35_hip_hparams`` == ``qw35_metal_hparams`` (Qw35MetalTypes.h:30-59)."""

    _fields_ = [
        ("transformer_layers", C.c_uint32),
        ("embedding_length", C.c_uint32),
        ("feed_forward_length", C.c_uint32),
        ("attention_heads", C.c_uint32),
        ("attention_kv_heads", C.c_uint32),
        ("attention_key_length", C.c_uint32),
        ("attention_value_length", C.c_uint32),
        ("rope_dimension_count", C.c_uint32),
        ("rope_sections", C.c_int32 * 4),
        ("rope_freq_base", C.c_float),
        ("rms_epsilon", C.c_float),
        ("ssm_conv_kernel", C.c_uint32),
        ("ssm_state_size", C.c_uint32),
        ("ssm_group_count", C.c_uint32),
        ("ssm_time_step_rank", C.c_uint32),
        ("ssm_inner_size", C.c_uint32),
        ("full_attention_interval", C.c_uint32),
        ("attn_window", C.c_int32),
        ("attn_sink", C.c_int32),
        ("attn_gate", C.c_uint32),
        ("n_cls_out", C.c_uint32),
    ]


# name -> (restype, argtypes); every symbol declared in include/qw35_hip.h.
PROTOTYPES: dict[str, tuple] = {
    "qw35_hip_gguf_parse": (
        C.c_int,
        [C.c_void_p, C.c_uint64, C.POINTER(TensorDesc), C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
         C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_store_create": (
        C.c_void_p, [C.c_void_p, C.c_uint64, C.POINTER(TensorDesc), C.c_uint32, C.c_char_p, C.c_size_t]),
    "qw35_hip_store_device_base": (C.c_void_p, [C.c_void_p]),
    "qw35_hip_store_bytes": (C.c_uint64, [C.c_void_p]),
    "qw35_hip_store_weight": (
        C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t, C.POINTER(Weight), C.c_char_p, C.c_size_t]),
    "qw35_hip_store_destroy": (None, [C.c_void_p]),
    "qw35_hip_has_device": (C.c_int, []),
    "qw35_hip_weight_view": (C.c_int, [C.POINTER(TensorDesc), C.c_void_p, C.POINTER(Weight), C.c_char_p, C.c_size_t]),
    "qw35_hip_decode_matvec": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_int, C.c_void_p, C.c_char_p,
         C.c_size_t],
    ),
    "qw35_hip_ffn_gate_up_swiglu": (
        C.c_int,
        [C.POINTER(Weight), C.POINTER(Weight), C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
         C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_gemv_kernel": (
        C.c_int,
        [C.POINTER(Weight), C.POINTER(Weight), C.c_uint32, C.c_int, C.c_int, C.c_char_p, C.c_size_t,
         C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.c_char_p,
         C.c_size_t],
    ),
    "qw35_hip_decode_matvec_workspace_size": (C.c_uint64, [C.POINTER(Weight), C.c_uint32]),
    "qw35_hip_decode_matvec_ws": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_int, C.c_void_p, C.c_uint64,
         C.c_void_p, C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_output_argmax_workspace_size": (C.c_uint64, [C.POINTER(Weight), C.c_uint32]),
    "qw35_hip_output_argmax": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
         C.c_void_p, C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_output_argmax_noalloc": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_char_p,
         C.c_size_t],
    ),
    "qw35_hip_dequantize": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_dequantize_f16": (C.c_int, [C.POINTER(Weight), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_create": (
        C.c_void_p,
        [C.c_void_p, C.c_uint64, C.POINTER(TensorDesc), C.c_size_t, C.POINTER(Hparams), C.c_uint32, C.c_uint32,
         C.c_uint32, C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_runtime_destroy": (None, [C.c_void_p]),
    "qw35_hip_runtime_eval_step": (C.c_int, [C.c_void_p, C.c_uint32, C.c_int, C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_eval_chunk": (C.c_int, [C.c_void_p, C.c_uint32, C.c_int, C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_argmax": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_copy_logits": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_sync": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_buffer": (
        C.c_int, [C.c_void_p, C.c_uint32, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64), C.c_char_p, C.c_size_t]),
    "qw35_hip_runtime_stream": (C.c_void_p, [C.c_void_p]),
    "qw35_hip_runtime_store": (C.c_void_p, [C.c_void_p]),
    "qw35_hip_plan_create": (C.c_void_p, [C.POINTER(PlanOp), C.c_uint32, C.c_char_p, C.c_size_t]),
    "qw35_hip_plan_launch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]),
    "qw35_hip_plan_size": (C.c_uint32, [C.c_void_p]),
    "qw35_hip_plan_destroy": (None, [C.c_void_p]),
    "qw35_hip_matmul_prefill_workspace_size": (C.c_uint64, [C.c_void_p, C.c_uint32]),
    "qw35_hip_matmul_prefill": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
         C.c_uint64, C.c_void_p, C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_prefill_kernel": (
        C.c_int,
        [C.POINTER(Weight), C.c_uint32, C.c_uint32, C.c_int, C.c_uint32, C.c_int, C.c_char_p, C.c_size_t,
         C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_char_p,
         C.c_size_t],
    ),
    "qw35_hip_matmul_prefill_epilogue": (
        C.c_int,
        [C.POINTER(Weight), C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
         C.c_void_p, C.c_uint64, C.c_void_p, C.c_char_p, C.c_size_t],
    ),
    "qw35_hip_quantize": (
        C.c_int,
        [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_char_p,
         C.c_size_t],
    ),
    "qw35_hip_stream_read_sink_len": (C.c_uint32, [C.c_uint64]),
    "qw35_hip_stream_read": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]),
    "qw35_hip_mfma_probe": (C.c_int, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]),
    "qw35_hip_sync": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
}

_LIB: C.CDLL | None = None


class Qw35Error(RuntimeError):
    """A C-ABI call returned 0; the message is the library's err buffer."""


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load ``libqw35_hip.so`` and bind every prototype (raises if missing)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise Qw35Error(
            f"{p} is not built; run `python -m qwowl35_amd.build` (the HIP library is required, "
            "there is no fallback)"
        )
    lib = C.CDLL(str(p))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def call(name: str, *args) -> int:
    """Call ``name(*args, err, err_len)`` and raise ``Qw35Error`` on a 0 / NULL return."""
    lib = load()
    err = C.create_string_buffer(512)
    rc = getattr(lib, name)(*args, err, C.sizeof(err))
    if not rc:
        raise Qw35Error(f"{name}: {err.value.decode(errors='replace')}")
    return rc
