"""ctypes binding of the C ABI in ``include/mcq4.h`` (``_lib/libmcq4.so``).

The library is the only compute path: if it is missing the import fails loudly
(there is no CPU or pure-PyTorch fallback).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libmcq4.so")

MCQ4_OK = 0
MCQ4_ERR_INVALID_ARG = 1
MCQ4_ERR_SHAPE = 2
MCQ4_ERR_ALIGNMENT = 3
MCQ4_ERR_WORKSPACE = 4
MCQ4_ERR_HIP = 5
MCQ4_DTYPE_F32 = 0
MCQ4_DTYPE_F16 = 1
MCQ4_DTYPE_BF16 = 2

# Every symbol declared in include/mcq4.h with (restype, argtypes).
_i64, _p, _int, _sz = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "mcq4_version": (_int, []),
    "mcq4_status_string": (ctypes.c_char_p, [_int]),
    "mcq4_last_error": (ctypes.c_char_p, []),
    "mcq4_quantize_q4_0": (_int, [_p, _i64, _i64, _i64, _p, _p]),
    "mcq4_quantize_q4_0_typed": (_int, [_p, _int, _i64, _i64, _i64, _p, _p]),
    "mcq4_quantize_q4_0_llama": (_int, [_p, _i64, _i64, _i64, _p, _p]),
    "mcq4_dequantize_q4_0": (_int, [_p, _i64, _i64, _p, _i64, _int, _p]),
    "mcq4_matmul_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mcq4_matmul_q4_0_f16": (_int, [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "mcq4_matmul_q4_0": (_int, [_p, _int, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "mcq4_matmul_q4_0_f16_grouped": (_int, [_p, _i64, _int, _p, _p, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "mcq4_reload_options": (_int, []),
    "mcq4_matmul_q4_0_f16_noalloc": (_int, [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "mcq4_matmul_noalloc_max_workspace_bytes": (_sz, []),
    "mcq4_reset_workspace": (_int, [_p, _sz, _p]),
    "mcq4_split_fallback_count": (_int, [ctypes.POINTER(ctypes.c_uint64), _int]),
    "mcq4_quantize_int4": (_int, [_p, _int, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "mcq4_dequantize_int4": (_int, [_p, _p, _p, _int, _i64, _i64, _i64, _p, _i64, _int, _p]),
    "mcq4_matmul_int4_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _int]),
    "mcq4_matmul_int4": (_int, [_p, _int, _i64, _p, _p, _p, _int, _p, _i64, _i64, _i64, _i64,
                                _i64, _p, _sz, _p]),
    "mcq4_matmul_int4_silu": (_int, [_p, _int, _i64, _p, _p, _p, _int, _p, _i64, _i64, _i64,
                                     _i64, _i64, _p, _sz, _p]),
    "mcq4_matmul_int4_gelu": (_int, [_p, _int, _i64, _p, _p, _p, _int, _p, _i64, _i64, _i64,
                                     _i64, _i64, _p, _sz, _p]),
    "mcq4_quantize_to_int4": (_int, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "mcq4_matmul_int8_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _int]),
    "mcq4_matmul_int8": (_int, [_p, _int, _i64, _p, _p, _p, _int, _p, _i64, _i64, _i64, _i64,
                                _i64, _p, _sz, _p]),
    "mcq4_fused_rmsnorm_linear_int4_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "mcq4_fused_rmsnorm_linear_int4": (_int, [_p, _i64, _p, ctypes.c_float, _p, _p, _p, _int, _p,
                                              _i64, _i64, _i64, _i64, _i64, _p, _sz, _p]),
}


class Mcq4Error(RuntimeError):
    """A non-OK status returned by the C ABI (subclass of RuntimeError, like TORCH_CHECK)."""

    def __init__(self, status: int, func: str, message: str):
        self.status = status
        super().__init__(f"{func} failed ({status_string(status)}): {message}")


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"metalops_amd: native library {LIB_PATH} is not built; "
            "run `python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def status_string(status: int) -> str:
    return lib.mcq4_status_string(status).decode()


def reload_options() -> None:
    """Re-read the library's MCQ4_* test switches from the environment.

    The library reads them once, at its first launch, and again only here.
    """
    check(lib.mcq4_reload_options(), "mcq4_reload_options")


def split_fallback_count(reset: bool = False) -> int:
    """Split-K tiles recomputed because a split ran on another XCD (current device)."""
    v = ctypes.c_uint64(0)
    check(lib.mcq4_split_fallback_count(ctypes.byref(v), int(reset)), "mcq4_split_fallback_count")
    return int(v.value)


def check(status: int, func: str) -> None:
    if status != MCQ4_OK:
        raise Mcq4Error(status, func, lib.mcq4_last_error().decode())
