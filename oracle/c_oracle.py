"""ctypes loader for oracle/q4_0_ref.c -- TEST INFRASTRUCTURE ONLY (checker, never product)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libq4oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, p = ctypes.c_int64, ctypes.c_void_p
        for name in ("q4ref_quantize_ref", "q4ref_quantize_llama"):
            getattr(L, name).argtypes = [p, i64, i64, p]
        for name in ("q4ref_dequant_f32", "q4ref_dequant_f16"):
            getattr(L, name).argtypes = [p, i64, i64, p]
        L.q4ref_matmul_f64.argtypes = [p, i64, i64, p, i64, p]
        L.q4ref_f32_to_f16.argtypes = [ctypes.c_float]
        L.q4ref_f32_to_f16.restype = ctypes.c_uint16
        L.q4ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.q4ref_f16_to_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def quantize_ref_rule(W: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float32)
    K, N = W.shape
    out = np.empty((K // 32, N, 18), dtype=np.uint8)
    lib().q4ref_quantize_ref(_ptr(W), K, N, _ptr(out))
    return out


def quantize_llama_rule(W: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float32)
    K, N = W.shape
    out = np.empty((K // 32, N, 18), dtype=np.uint8)
    lib().q4ref_quantize_llama(_ptr(W), K, N, _ptr(out))
    return out


def dequantize(blocks: np.ndarray, dtype=np.float32) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb, N, _ = b.shape
    K = nb * 32
    if dtype == np.float32:
        out = np.empty((K, N), dtype=np.float32)
        lib().q4ref_dequant_f32(_ptr(b), K, N, _ptr(out))
        return out
    out = np.empty((K, N), dtype=np.uint16)
    lib().q4ref_dequant_f16(_ptr(b), K, N, _ptr(out))
    return out.view(np.float16)


def matmul_f64(X: np.ndarray, blocks: np.ndarray) -> np.ndarray:
    Xh = np.ascontiguousarray(X, dtype=np.float16).view(np.uint16)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    M, K = Xh.shape
    N = b.shape[1]
    Y = np.empty((M, N), dtype=np.float64)
    lib().q4ref_matmul_f64(_ptr(Xh), M, K, _ptr(b), N, _ptr(Y))
    return Y
