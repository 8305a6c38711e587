"""ctypes loader of the C restatement (oracle/c/qw35_oracle.c) — test infrastructure only.

Build it with ``make -C oracle`` (``__graft_entry__.build()`` does).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "_build" / "libqw35_oracle.so"
_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise FileNotFoundError(f"{LIB} missing; run `make -C oracle`")
        _lib = C.CDLL(str(LIB))
        for name in ("qw35o_gf4_dequant", "qw35o_q8_0_dequant", "qw35o_q4_k_dequant", "qw35o_q6_k_dequant",
                     "qw35o_q5_k_dequant", "qw35o_gf2_dequant"):
            getattr(_lib, name).argtypes = [C.c_void_p, C.c_size_t, C.c_void_p]
            getattr(_lib, name).restype = None
        _lib.qw35o_matvec_f64.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p]
        _lib.qw35o_matvec_f64.restype = None
    return _lib


def dequant(type_id: int, raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    out = np.empty((rows, k), dtype=np.float32)
    if type_id == 100:
        lib().qw35o_gf4_dequant(raw.ctypes.data, rows * k // 8, out.ctypes.data)
    elif type_id == 8:
        lib().qw35o_q8_0_dequant(raw.ctypes.data, rows * k // 32, out.ctypes.data)
    elif type_id == 12:
        lib().qw35o_q4_k_dequant(raw.ctypes.data, rows * k // 256, out.ctypes.data)
    elif type_id == 14:
        lib().qw35o_q6_k_dequant(raw.ctypes.data, rows * k // 256, out.ctypes.data)
    elif type_id == 13:
        lib().qw35o_q5_k_dequant(raw.ctypes.data, rows * k // 256, out.ctypes.data)
    elif type_id == 101:
        lib().qw35o_gf2_dequant(raw.ctypes.data, rows * k // 256, out.ctypes.data)
    else:
        raise ValueError(type_id)
    return out


def matvec_f64(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    x2 = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    y = np.empty((x2.shape[0], w.shape[0]), dtype=np.float64)
    lib().qw35o_matvec_f64(w.ctypes.data, w.shape[0], w.shape[1], x2.ctypes.data, x2.shape[0], y.ctypes.data)
    return y if np.ndim(x) == 2 else y[0]
