"""CPU tests of the C ABI surface (include/mcq4.h <-> metalops_amd/_lib/libmcq4.so).

No kernel is launched: every call here fails validation before touching the GPU.
"""
import ctypes
import os
import re

import pytest

from metalops_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mcq4.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mcq4_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_what_binding_knows():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name


def test_version_and_status_strings():
    L = _lib.lib
    assert L.mcq4_version() >= 10000
    assert _lib.status_string(_lib.MCQ4_OK) == "ok"
    assert "workspace" in _lib.status_string(_lib.MCQ4_ERR_WORKSPACE)
    assert _lib.status_string(99) == "unknown status"


def _err():
    return _lib.lib.mcq4_last_error().decode()


def test_matmul_validation_codes():
    L = _lib.lib
    X, W, Y = 0x10000, 0x20000, 0x30000   # never dereferenced: validation fails first
    assert L.mcq4_matmul_q4_0_f16(None, 32, W, Y, 8, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert "null" in _err()
    assert L.mcq4_matmul_q4_0_f16(X, 48, W, Y, 8, 1, 48, 8, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert "divisible by 32" in _err()
    assert L.mcq4_matmul_q4_0_f16(X, 32, W, Y, 8, 0, 32, 8, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert L.mcq4_matmul_q4_0_f16(X, 16, W, Y, 8, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert L.mcq4_matmul_q4_0_f16(X, 32, W, Y, 4, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert L.mcq4_matmul_q4_0_f16(X + 8, 32, W, Y, 8, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert L.mcq4_matmul_q4_0_f16(X, 36, W, Y, 8, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert L.mcq4_matmul_q4_0_f16(X, 32, W + 1, Y, 8, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert L.mcq4_matmul_q4_0_f16(X, 32, W, Y + 1, 8, 1, 32, 8, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT


def test_workspace_query_and_check():
    L = _lib.lib
    assert L.mcq4_matmul_workspace_bytes(1, 4096, 4096) == 0   # decode: no split-K
    need = L.mcq4_matmul_workspace_bytes(128, 8192, 128)       # one GEMM tile: split-K
    assert need >= 256 * 1024                                  # counter area + partials
    assert L.mcq4_matmul_workspace_bytes(1, 48, 8) == 0        # invalid K
    assert L.mcq4_matmul_workspace_bytes(0, 4096, 8) == 0
    rc = L.mcq4_matmul_q4_0_f16(0x10000, 8192, 0x20000, 0x30000, 128, 128, 8192, 128, None, 0, None)
    assert rc == _lib.MCQ4_ERR_WORKSPACE and "required" in _err()
    rc = L.mcq4_matmul_q4_0_f16(0x10000, 8192, 0x20000, 0x30000, 128, 128, 8192, 128,
                                0x40000, need - 1, None)
    assert rc == _lib.MCQ4_ERR_WORKSPACE


def test_quantize_dequant_validation_codes():
    L = _lib.lib
    assert L.mcq4_quantize_q4_0(None, 8, 32, 8, 0x20000, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert L.mcq4_quantize_q4_0(0x10000, 8, 33, 8, 0x20000, None) == _lib.MCQ4_ERR_SHAPE
    assert L.mcq4_quantize_q4_0(0x10000, 4, 32, 8, 0x20000, None) == _lib.MCQ4_ERR_SHAPE
    assert L.mcq4_quantize_q4_0_llama(0x10002, 8, 32, 8, 0x20000, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert L.mcq4_quantize_q4_0(0x10000, 8, 32, 8, 0x20001, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert L.mcq4_dequantize_q4_0(0x20000, 32, 8, 0x30000, 8, 7, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert L.mcq4_dequantize_q4_0(0x20000, 32, 8, 0x30002, 8, _lib.MCQ4_DTYPE_F32, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert L.mcq4_dequantize_q4_0(0x20000, 32, 8, 0x30000, 4, _lib.MCQ4_DTYPE_F16, None) == _lib.MCQ4_ERR_SHAPE
    assert L.mcq4_dequantize_q4_0(0x20000, 32 * 70000, 8, 0x30000, 8, 0, None) == _lib.MCQ4_ERR_SHAPE


def test_error_raises_runtime_error_subclass():
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(_lib.lib.mcq4_quantize_q4_0(None, 8, 32, 8, None, None), "mcq4_quantize_q4_0")


def test_int4_validation_codes():
    """Per-group INT4 entry points reject bad arguments before any launch."""
    L = _lib.lib
    F32, F16, BF16 = _lib.MCQ4_DTYPE_F32, _lib.MCQ4_DTYPE_F16, _lib.MCQ4_DTYPE_BF16
    X, P, S, Z, Y = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    mm = L.mcq4_matmul_int4
    assert mm(None, F16, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert mm(X, 7, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert mm(X, F16, 64, P, S, Z, 9, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert mm(X, F16, 64, P, S, Z, F32, Y, 8, 1, 63, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert "even" in _err()
    assert mm(X, F16, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 0, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert "group_size" in _err()
    assert mm(X, F16, 64, P, S, Z, F32, Y, 8, 0, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert mm(X, F16, 32, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert mm(X, F16, 64, P, S, Z, F32, Y, 4, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert mm(X + 1, F16, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert mm(X, F32, 64, P, S, Z, F32, Y + 2, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert mm(X, F16, 64, P, S + 2, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    # The decode kernel with a split K (long K, small groups) needs the workspace it reports.
    need = L.mcq4_matmul_int4_workspace_bytes(1, 16384, 4096, 32, F16)
    assert need > 0
    assert mm(X, F16, 16384, P, S, Z, F16, Y, 4096, 1, 16384, 4096, 32, None, 0, None) == _lib.MCQ4_ERR_WORKSPACE
    assert L.mcq4_matmul_int4_silu(None, F16, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert L.mcq4_matmul_int4_gelu(X, F16, 64, P, S, Z, F32, Y, 8, 1, 63, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    # quantize / dequantize
    q = L.mcq4_quantize_int4
    assert q(None, F32, 8, 64, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert q(X, 5, 8, 64, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert q(X, F32, 8, 63, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_SHAPE
    assert q(X, F32, 4, 64, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_SHAPE
    assert q(X + 2, F32, 8, 64, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_ALIGNMENT
    assert q(X, BF16, 8, 64, 8, 32, P, S + 1, Z, None) == _lib.MCQ4_ERR_ALIGNMENT
    d = L.mcq4_dequantize_int4
    assert d(None, S, Z, F32, 64, 8, 32, Y, 8, F16, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert d(P, S, Z, F32, 64, 8, 32, Y, 8, 3, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert d(P, S, Z, F32, 64, 8, 32, Y, 4, F16, None) == _lib.MCQ4_ERR_SHAPE
    assert d(P, S, Z, F32, 64, 8, -1, Y, 8, F16, None) == _lib.MCQ4_ERR_SHAPE
    assert d(P, S, Z, F32, 64, 8, 32, Y + 2, 8, F32, None) == _lib.MCQ4_ERR_ALIGNMENT


def test_int4_workspace_sizes():
    L = _lib.lib
    F16, F32 = _lib.MCQ4_DTYPE_F16, _lib.MCQ4_DTYPE_F32
    # fp32 activations and odd group sizes run the general kernel: no workspace
    assert L.mcq4_matmul_int4_workspace_bytes(1, 4096, 4096, 128, F32) == 0
    assert L.mcq4_matmul_int4_workspace_bytes(1, 4096, 4096, 100, F16) == 0
    # wide-N decode keeps K in one workgroup: no workspace
    assert L.mcq4_matmul_int4_workspace_bytes(1, 4096, 128256, 128, F16) == 0
    # split-K layouts start with the 256 KiB counter area
    for M, K, N in ((1, 4096, 4096), (16, 14336, 4096), (128, 4096, 4096)):
        ws = L.mcq4_matmul_int4_workspace_bytes(M, K, N, 128, F16)
        assert ws == 0 or ws > 256 * 1024


def test_int8_and_fused_validation_codes():
    L = _lib.lib
    F32, F16 = _lib.MCQ4_DTYPE_F32, _lib.MCQ4_DTYPE_F16
    X, P, S, Z, Y, W = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000
    m8 = L.mcq4_matmul_int8
    assert m8(None, F16, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert m8(X, F16, 64, P, S, Z, F32, Y, 8, 1, 0, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert m8(X, F16, 32, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert m8(X + 1, F16, 64, P, S, Z, F32, Y, 8, 1, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_ALIGNMENT
    q = L.mcq4_quantize_to_int4
    assert q(None, 8, 64, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert q(X, 8, 64, 8, 33, P, S, Z, None) == _lib.MCQ4_ERR_SHAPE
    assert q(X + 2, 8, 64, 8, 32, P, S, Z, None) == _lib.MCQ4_ERR_ALIGNMENT
    f = L.mcq4_fused_rmsnorm_linear_int4
    need = L.mcq4_fused_rmsnorm_linear_int4_workspace_bytes(4, 64, 8, 32)
    assert need >= 256 * 1024 + 4 * 64 * 2
    assert f(None, 64, W, 1e-6, P, S, Z, F16, Y, 8, 4, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert f(X, 64, W, 1e-6, P, S, Z, F16, Y, 8, 4, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_WORKSPACE
    assert f(X, 32, W, 1e-6, P, S, Z, F16, Y, 8, 4, 64, 8, 32, None, 0, None) == _lib.MCQ4_ERR_SHAPE
    assert f(X, 64, W, 1e-6, P, S, Z, F16, Y, 8, 4, 64, 8, 32, 0x70080, need, None) == _lib.MCQ4_ERR_ALIGNMENT  # 128-, not 256-aligned


def test_grouped_validation():
    """The grouped entry point's argument checks need no GPU: no weights, a null
    weight or output pointer, and ldy < N are rejected on either path."""
    f = _lib.lib.mcq4_matmul_q4_0_f16_grouped
    w = (ctypes.c_void_p * 2)(256, 512)
    y = (ctypes.c_void_p * 2)(1024, 2048)
    x = ctypes.c_void_p(4096)
    assert f(x, 64, 0, w, y, 64, 1, 64, 64, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    assert f(x, 64, 2, None, y, 64, 1, 64, 64, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    wn = (ctypes.c_void_p * 2)(256, None)
    assert f(x, 64, 2, wn, y, 64, 1, 64, 64, None, 0, None) == _lib.MCQ4_ERR_INVALID_ARG
    for m in (1, 3):                              # one-launch form and per-weight form
        assert f(x, 64, 2, w, y, 32, m, 64, 64, None, 0, None) == _lib.MCQ4_ERR_SHAPE
        assert b"ldy" in _lib.lib.mcq4_last_error()


