"""ctypes loader for oracle/_ref/libnative_quant_ref.so. TEST INFRASTRUCTURE ONLY.

The library is the reference's engine/native_quant.cpp compiled from source by
oracle/Makefile. Its ten exports and their argument order are those of
engine/native_quant.cpp:705-768; the Python-side shape rules and the
[rows, tokens] -> [tokens, rows] transpose follow engine/native_quant.py:102-156.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / '_ref' / 'libnative_quant_ref.so'
_SYMBOL = {2: 'q4_0', 8: 'q8_0', 12: 'q4k', 13: 'q5k', 14: 'q6k'}
_LIB = None


def available() -> bool:
    return LIB_PATH.exists()


def load():
    global _LIB
    if _LIB is None:
        lib = ctypes.CDLL(str(LIB_PATH))
        u8p, f32p = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_float)
        for name in _SYMBOL.values():
            fn = getattr(lib, f'localai_{name}_matvec')
            fn.argtypes = [u8p, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            fn.restype = None
            fn = getattr(lib, f'localai_{name}_matmul')
            fn.argtypes = [u8p, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            fn.restype = None
        _LIB = lib
    return _LIB


def matvec(raw, x, rows, cols, t, threads=4):
    lib = load()
    raw = np.frombuffer(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, dtype=np.float32)
    getattr(lib, f'localai_{_SYMBOL[t]}_matvec')(
        raw.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
        x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
        out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), rows, cols, threads)
    return out


def matmul(raw, xs, rows, cols, t, threads=4):
    """Returns [tokens, rows] like engine/native_quant.py:156."""
    lib = load()
    raw = np.frombuffer(raw, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    out = np.empty((rows, xs.shape[0]), dtype=np.float32)
    getattr(lib, f'localai_{_SYMBOL[t]}_matmul')(
        raw.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
        xs.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
        out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), rows, cols, xs.shape[0], threads)
    return out.T.copy()


def decode_rows(raw, t, rows, cols, threads=4):
    """The reference's exact row decoders (native_quant.cpp:543-618), observed
    through its batched matmul with one-hot vectors: out[r, j] = W[r, j]."""
    return matmul(raw, np.eye(cols, dtype=np.float32), rows, cols, t, threads).T
