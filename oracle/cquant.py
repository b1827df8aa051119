"""ctypes wrapper for oracle/quant_ref.c (TEST INFRASTRUCTURE ONLY)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_quant.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_quant.so"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        _lib.oracle_quantize_rows_f32.argtypes = [p, i64, i64, p, p]
        _lib.oracle_quantize_rows_f32.restype = None
        _lib.oracle_w8a16_gemm_f64.argtypes = [p, p, p, i64, i64, i64, p]
        _lib.oracle_w8a16_gemm_f64.restype = None
    return _lib


def quantize_rows_f32(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.int8)
    s = np.empty((rows,), dtype=np.float32)
    _load().oracle_quantize_rows_f32(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data)
    return q, s


def w8a16_gemm_f64(x: np.ndarray, q: np.ndarray, s: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    M, K = x.shape
    N = q.shape[0]
    assert q.shape == (N, K) and s.shape == (N,)
    y = np.empty((M, N), dtype=np.float64)
    _load().oracle_w8a16_gemm_f64(x.ctypes.data, q.ctypes.data, s.ctypes.data, M, N, K, y.ctypes.data)
    return y
