"""ctypes binding of the C ABI declared in include/iqmm.h.

This is the same binding a Rust/cgo/N-API caller would write: plain structs,
device pointers and a hipStream_t.  The library must be built
(``python -m ironmlx_amd.build``); nothing falls back to a CPU path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libiqmm.so")
MAX_NDIM = 8

# iqmm_dtype
FLOAT32, FLOAT16, BFLOAT16, UINT32, UINT8, INT32, INT64 = range(7)


class IqmmArray(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("shape", ctypes.c_int64 * MAX_NDIM),
                ("ndim", ctypes.c_int32), ("dtype", ctypes.c_int32)]


class OptionalInt(ctypes.Structure):
    _fields_ = [("value", ctypes.c_int), ("has_value", ctypes.c_bool)]


class OptionalDtype(ctypes.Structure):
    _fields_ = [("value", ctypes.c_int), ("has_value", ctypes.c_bool)]


EXPORTS = ("iqmm_quantized_matmul", "iqmm_dequantize", "iqmm_gather_qmm", "iqmm_quantize",
           "iqmm_quantized_swiglu", "iqmm_gather_qmm_swiglu", "iqmm_dequantize_rows",
           "iqmm_moe_route", "iqmm_moe_sort", "iqmm_moe_sort_noalloc", "iqmm_moe_combine",
           "iqmm_moe_token", "iqmm_workspace_reserve", "iqmm_last_error", "iqmm_version")

_lib = None


class IqmmError(RuntimeError):
    """A non-zero return from the library; the message is iqmm_last_error()
    (the analogue of Error::Mlx, mlx/src/error.rs:27-35)."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `python -m ironmlx_amd.build` "
                          "(the quantized ops have no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    A, P = IqmmArray, ctypes.POINTER(IqmmArray)
    OI, OD = OptionalInt, OptionalDtype
    vp, b, cs = ctypes.c_void_p, ctypes.c_bool, ctypes.c_char_p
    L.iqmm_quantized_matmul.argtypes = [P, A, A, A, A, b, OI, OI, cs, vp]
    L.iqmm_quantized_matmul.restype = ctypes.c_int
    L.iqmm_dequantize.argtypes = [P, A, A, A, OI, OI, cs, OD, vp]
    L.iqmm_dequantize.restype = ctypes.c_int
    L.iqmm_gather_qmm.argtypes = [P, A, A, A, A, A, A, b, OI, OI, cs, b, vp]
    L.iqmm_gather_qmm.restype = ctypes.c_int
    L.iqmm_quantize.argtypes = [P, P, P, A, OI, OI, cs, vp]
    L.iqmm_quantize.restype = ctypes.c_int
    L.iqmm_quantized_swiglu.argtypes = [P, A, A, A, A, OI, OI, cs, vp]
    L.iqmm_quantized_swiglu.restype = ctypes.c_int
    L.iqmm_gather_qmm_swiglu.argtypes = [P, A, A, A, A, A, A, OI, OI, cs, b, vp]
    L.iqmm_gather_qmm_swiglu.restype = ctypes.c_int
    L.iqmm_dequantize_rows.argtypes = [P, A, A, A, A, OI, OI, cs, OD, vp]
    L.iqmm_dequantize_rows.restype = ctypes.c_int
    i = ctypes.c_int
    L.iqmm_moe_route.argtypes = [P, P, A, i, b, vp]
    L.iqmm_moe_route.restype = ctypes.c_int
    L.iqmm_moe_sort.argtypes = [P, P, P, P, A, i, vp]
    L.iqmm_moe_sort.restype = ctypes.c_int
    L.iqmm_moe_sort_noalloc.argtypes = [P, P, P, P, A, i, vp]
    L.iqmm_moe_sort_noalloc.restype = ctypes.c_int
    L.iqmm_moe_combine.argtypes = [P, A, A, A, A, i, vp]
    L.iqmm_moe_combine.restype = ctypes.c_int
    L.iqmm_moe_token.argtypes = [P, A, A, A, A, A, A, A, A, i, b, i, i, vp]
    L.iqmm_moe_token.restype = ctypes.c_int
    L.iqmm_workspace_reserve.argtypes = [vp, ctypes.c_size_t]
    L.iqmm_workspace_reserve.restype = ctypes.c_int
    L.iqmm_last_error.restype = ctypes.c_char_p
    L.iqmm_last_error.argtypes = []
    L.iqmm_version.restype = ctypes.c_char_p
    L.iqmm_version.argtypes = []
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        msg = load().iqmm_last_error().decode() or f"unknown iqmm error (code {rc})"
        raise IqmmError(msg)


def opt_int(v) -> OptionalInt:
    return OptionalInt(0, False) if v is None else OptionalInt(int(v), True)


def empty_array() -> IqmmArray:
    return IqmmArray()
