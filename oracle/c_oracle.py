"""ctypes view of the C oracle (test infrastructure only).

Loads ``oracle/_build/liboracle_awq.so`` built by ``oracle/build.py``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build as _build

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_build.LIB):
            _build.build()
        L = ctypes.CDLL(_build.LIB)
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_mul.restype = ctypes.c_uint16
        L.oracle_f16_mul.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.oracle_unpack.restype = None
        L.oracle_unpack.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        L.oracle_dequant.restype = ctypes.c_int
        L.oracle_dequant.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
        L.oracle_gemm_f64.restype = ctypes.c_int
        L.oracle_gemm_f64.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                      ctypes.c_void_p, ctypes.c_void_p]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def unpack(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    rows, pn = packed.shape
    out = np.empty((rows, pn * 8), dtype=np.uint8)
    lib().oracle_unpack(_p(packed), rows, pn * 8, _p(out))
    return out


def dequant(qweight, qzeros, scales, group_size=128) -> np.ndarray:
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    qzeros = np.ascontiguousarray(qzeros, dtype=np.int32)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    k, pn = qweight.shape
    w = np.empty((k, pn * 8), dtype=np.float16)
    rc = lib().oracle_dequant(_p(qweight), _p(qzeros), _p(scales.view(np.uint16)), k, pn * 8,
                              group_size, _p(w.view(np.uint16)))
    if rc:
        raise ValueError("oracle_dequant rejected the shapes")
    return w


def gemm_f64(x, qweight, qzeros, scales, group_size=128) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    qzeros = np.ascontiguousarray(qzeros, dtype=np.int32)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    m, k = x.shape
    n = qweight.shape[1] * 8
    w = np.empty((k, n), dtype=np.uint16)
    y = np.empty((m, n), dtype=np.float64)
    rc = lib().oracle_gemm_f64(_p(x.view(np.uint16)), _p(qweight), _p(qzeros), _p(scales.view(np.uint16)),
                               m, n, k, group_size, _p(w), _p(y))
    if rc:
        raise ValueError("oracle_gemm_f64 rejected the shapes")
    return y


def f32_to_f16_bits(v: float) -> int:
    return int(lib().oracle_f32_to_f16(float(v)))


def f16_mul_bits(a_bits: int, b_bits: int) -> int:
    return int(lib().oracle_f16_mul(a_bits, b_bits))
