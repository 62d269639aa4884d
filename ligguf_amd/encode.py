"""ctypes binding of libligguf_encode.so (include/ligguf_encode.h): weight
encoders and seeded synthetic tensors."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .lib import row_size

PKG = os.path.dirname(os.path.abspath(__file__))
ENC_SO = os.path.join(PKG, "libligguf_encode.so")
_enc = None


def load() -> C.CDLL:
    global _enc
    if _enc is None:
        if not os.path.exists(ENC_SO):
            raise RuntimeError(f"{ENC_SO} is not built: run `python -m ligguf_amd.build`")
        e = C.CDLL(ENC_SO)
        e.lge_row_size.restype = C.c_int64
        e.lge_row_size.argtypes = [C.c_int, C.c_int64]
        e.lge_fill_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p, C.c_int64, C.c_float]
        e.lge_quantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]
        e.lge_random_tensor.argtypes = [C.c_int, C.c_uint64, C.c_uint64, C.c_int64, C.c_int64, C.c_float, C.c_void_p]
        e.lge_random_q1.argtypes = [C.c_int, C.c_uint64, C.c_uint64, C.c_int64, C.c_int64, C.c_float, C.c_void_p]
        _enc = e
    return _enc


def normal(seed: int, stream: int, n: int, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().lge_fill_normal(seed, stream, out.ctypes.data, n, sigma)
    return out


def quantize(t: int, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == rows * cols
    out = np.empty(rows * row_size(t, cols), np.uint8)
    if load().lge_quantize(t, x.ctypes.data, rows, cols, out.ctypes.data) != 0:
        raise ValueError(f"cannot encode type {t} with {cols} columns")
    return out


def random_tensor(t: int, seed: int, stream: int, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    out = np.empty(rows * row_size(t, cols), np.uint8)
    if load().lge_random_tensor(t, seed, stream, rows, cols, sigma, out.ctypes.data) != 0:
        raise ValueError(f"cannot encode type {t} with {cols} columns")
    return out


def random_q1(t: int, seed: int, stream: int, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    out = np.empty(rows * row_size(t, cols), np.uint8)
    if load().lge_random_q1(t, seed, stream, rows, cols, sigma, out.ctypes.data) != 0:
        raise ValueError(f"cannot draw 1-bit type {t} with {cols} columns")
    return out
