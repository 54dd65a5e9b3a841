"""GGML block_q4_0 quantize / dequantize / matmul on MI355X.

Mirrors metalcore's q4_0 API (``packages/metalcore/src/metalcore/quantization.py``):

* ``quantize_ggml_q4_0(weight)``            -- quantization.py:307-371
* ``dequantize_ggml_q4_0(blocks, dtype)``   -- quantization.py:374-419
* ``matmul_ggml_q4_0(X, W_blocks)``         -- quantization.py:422-454

Same names, argument order, defaults (dequant defaults to float16), block tensor
``[K/32, N, 18]`` uint8 and ``AssertionError`` messages for the K checks
(quantization.py:329, :443).  Every computation runs in the HIP kernels of
``libmcq4.so``; tensors must live on a ROCm device (``device.type == "cuda"``) --
there is deliberately no CPU fallback.  Work is enqueued on the current stream
and returns without synchronising, like the reference's Metal binding
(core_mps.mm:5947-5971).
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from typing import List, Optional, Sequence

import torch

from . import _lib

QK4_0 = 32                         # quantization.py:303
BLOCK_Q4_0_SIZE = 2 + QK4_0 // 2   # quantization.py:304 (18 bytes)

__all__ = [
    "QK4_0",
    "BLOCK_Q4_0_SIZE",
    "quantize_ggml_q4_0",
    "quantize_ggml_q4_0_llama",
    "dequantize_ggml_q4_0",
    "matmul_ggml_q4_0",
]


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "metalops_amd q4_0 ops run only on a ROCm GPU (torch device 'cuda'); "
                f"got a tensor on '{t.device}'. There is no CPU fallback.")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on one device, got {dev} and {t.device}")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_DTYPE_CODES = {torch.float32: _lib.MCQ4_DTYPE_F32, torch.float16: _lib.MCQ4_DTYPE_F16,
                torch.bfloat16: _lib.MCQ4_DTYPE_BF16}


def _quantize(weight: torch.Tensor, llama_rule: bool) -> torch.Tensor:
    K, N = weight.shape
    assert K % QK4_0 == 0, f"K ({K}) must be divisible by {QK4_0}"   # quantization.py:329
    _require_device(weight)
    # The reference rule rounds every step in the weight's dtype (fp32, fp16 and
    # bf16 run natively); other float dtypes are quantized from fp32, and the
    # llama.cpp rule (a benchmark generator) always runs in fp32.
    if llama_rule or weight.dtype not in _DTYPE_CODES:
        w = weight.float()
    else:
        w = weight
    esz = w.element_size()
    if w.stride(1) != 1 or w.stride(0) < N or w.data_ptr() % esz:
        w = w.contiguous()
    blocks = torch.empty((K // QK4_0, N, BLOCK_Q4_0_SIZE), dtype=torch.uint8, device=w.device)
    if K == 0 or N == 0:
        return blocks
    with torch.cuda.device(w.device):
        if llama_rule:
            _lib.check(_lib.lib.mcq4_quantize_q4_0_llama(w.data_ptr(), w.stride(0), K, N,
                                                         blocks.data_ptr(), _stream(w.device)),
                       "mcq4_quantize_q4_0_llama")
        else:
            _lib.check(_lib.lib.mcq4_quantize_q4_0_typed(w.data_ptr(), _DTYPE_CODES[w.dtype],
                                                         w.stride(0), K, N, blocks.data_ptr(),
                                                         _stream(w.device)),
                       "mcq4_quantize_q4_0_typed")
    return blocks


def quantize_ggml_q4_0(weight: torch.Tensor) -> torch.Tensor:
    """Quantize ``weight[K, N]`` to ``[K/32, N, 18]`` uint8 blocks (reference rule).

    Per block of 32 rows of a column: ``d = amax/7`` (1 when amax is 0),
    ``q = round_half_even(x/d + 8)`` clamped to [0, 15]; bytes 0..1 hold fp16(d),
    byte ``2+i`` holds ``q[2i] | q[2i+1] << 4`` (quantization.py:333-369).
    As in the reference, every step is rounded to the weight's own dtype (fp32,
    fp16 or bf16), so the bytes match the reference's for each of them.
    """
    return _quantize(weight, llama_rule=False)


def quantize_ggml_q4_0_llama(weight: torch.Tensor) -> torch.Tensor:
    """llama.cpp ``quantize_row_q4_0_ref`` rule in metalcore's layout (benchmark generator).

    ``d = max_signed/-8``, ``q = min(15, trunc(x/d + 8.5))``; produces negative
    scales and ``q = 0``, which the reference rule never does.  Not part of the
    reference API.
    """
    return _quantize(weight, llama_rule=True)


def dequantize_ggml_q4_0(blocks: torch.Tensor, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``[K/32, N, 18]`` blocks -> ``W[K, N] = (q - 8) * d`` in ``dtype`` (default float16).

    The product is exact in fp32; other dtypes receive one rounding of it, as
    the reference's ``.to(dtype)`` does (quantization.py:414-419).
    """
    if dtype is None:
        dtype = torch.float16
    num_blocks, N, bs = blocks.shape
    assert bs == BLOCK_Q4_0_SIZE, f"blocks last dim must be {BLOCK_Q4_0_SIZE}"
    K = num_blocks * QK4_0
    _require_device(blocks)
    if blocks.dtype != torch.uint8:
        raise RuntimeError("blocks must be uint8")
    b = blocks if (blocks.is_contiguous() and blocks.data_ptr() % 2 == 0) else blocks.contiguous()
    if b.data_ptr() % 2:
        b = b.clone()
    kernel_dtype = torch.float16 if dtype == torch.float16 else torch.float32
    out = torch.empty((K, N), dtype=kernel_dtype, device=b.device)
    if K and N:
        code = _lib.MCQ4_DTYPE_F16 if kernel_dtype == torch.float16 else _lib.MCQ4_DTYPE_F32
        with torch.cuda.device(b.device):
            _lib.check(_lib.lib.mcq4_dequantize_q4_0(b.data_ptr(), K, N, out.data_ptr(), N, code,
                                                     _stream(b.device)),
                       "mcq4_dequantize_q4_0")
    return out if out.dtype == dtype else out.to(dtype)


class _Workspace:
    """Per-device, zero-initialised split-K workspace reused across calls.

    The kernels leave the arrival counters at zero after every call, so the
    buffer is zero-filled once when (re)allocated; a call that fails is
    followed by a reset of its counter area on the same stream (``guard``),
    so an interrupted call cannot poison later ones.
    One buffer per (device, stream), so concurrent streams never share one; a
    larger request allocates a new buffer through PyTorch's stream-ordered
    caching allocator.
    """

    def __init__(self):
        self._bufs: dict = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        key = (device, stream)   # one buffer per stream: calls on one stream never overlap
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20)
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf

    @contextlib.contextmanager
    def guard(self, buf: Optional[torch.Tensor], stream: int, base: Optional[int] = None):
        """Resets the counter area at ``base`` (default: the buffer's start) if the body raises."""
        try:
            yield
        except Exception:
            if buf is not None:
                ptr = buf.data_ptr() if base is None else base
                _lib.lib.mcq4_reset_workspace(ptr, buf.numel() - (ptr - buf.data_ptr()), stream)
            raise


_workspace = _Workspace()


def matmul_ggml_q4_0(X: torch.Tensor, W_blocks: torch.Tensor) -> torch.Tensor:
    """``Y[M, N] = X[M, K] @ dequant(W_blocks)``, returned in ``X.dtype``.

    fp16 X runs the MFMA kernels: fp16 weights ``(q-8)*d`` (one rounding),
    fp32 accumulation, fp16 result (the reference's GPU kernel,
    native/quant_kernels.metal:1738-1886).  bf16 and fp32 X follow the
    reference's own path for those dtypes (quantization.py:452-454): the
    weight dequantized to X's dtype, fp32 accumulation, the result in X's
    dtype -- so bf16 activations beyond the fp16 range stay finite.  M <= 64
    runs the decode kernels, larger M the prefill GEMM.
    """
    num_blocks_per_col, N, _ = W_blocks.shape
    K = num_blocks_per_col * QK4_0
    assert X.shape[1] == K, f"X K dim ({X.shape[1]}) must match weight K ({K})"  # :443
    _require_device(X, W_blocks)
    if X.dim() != 2:
        raise RuntimeError(f"X must be 2-D [M, K], got shape {tuple(X.shape)}")
    if W_blocks.dtype != torch.uint8 or W_blocks.shape[2] != BLOCK_Q4_0_SIZE:
        raise RuntimeError("W_blocks must be uint8 [K/32, N, 18]")
    if X.dtype not in _DTYPE_CODES:
        raise RuntimeError(f"X must be float16, bfloat16 or float32, got {X.dtype}")
    M = X.shape[0]
    w = W_blocks if W_blocks.is_contiguous() else W_blocks.contiguous()
    if w.data_ptr() % 2:
        w = w.clone()
    Y = torch.empty((M, N), dtype=X.dtype, device=X.device)
    if M == 0 or N == 0:
        return Y
    if K == 0:
        return Y.zero_()
    stream = _stream(X.device)
    if X.dtype != torch.float16:
        x = X if (X.stride(1) == 1 and X.stride(0) >= K) else X.contiguous()
        with torch.cuda.device(x.device):
            _lib.check(_lib.lib.mcq4_matmul_q4_0(x.data_ptr(), _DTYPE_CODES[x.dtype], x.stride(0),
                                                 w.data_ptr(), Y.data_ptr(), N, M, K, N, None, 0,
                                                 stream),
                       "mcq4_matmul_q4_0")
        return Y
    x = X
    if x.stride(1) != 1 or x.stride(0) % 8 or x.stride(0) < K or x.data_ptr() % 16:
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()
    need = int(_lib.lib.mcq4_matmul_workspace_bytes(M, K, N))
    ws, ws_ptr, ws_bytes = None, None, 0
    if need:
        ws = _workspace.get(x.device, stream, need)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    with torch.cuda.device(x.device), _workspace.guard(ws, stream):
        _lib.check(_lib.lib.mcq4_matmul_q4_0_f16(x.data_ptr(), x.stride(0), w.data_ptr(),
                                                 Y.data_ptr(), N, M, K, N, ws_ptr, ws_bytes,
                                                 stream),
                   "mcq4_matmul_q4_0_f16")
    return Y


def matmul_ggml_q4_0_grouped(X: torch.Tensor, weights: Sequence[torch.Tensor]) -> List[torch.Tensor]:
    """``[X @ dequant(W) for W in weights]`` -- several q4_0 weights of one shape
    that share the activations (an MLP's gate and up), returned in ``X.dtype``.

    No counterpart in the reference, whose API takes one weight per call; the
    results are those of ``matmul_ggml_q4_0`` per weight (the same kernels'
    arithmetic).  For one fp16 activation row and up to four weights with N a
    multiple of 16 it is a single launch of the M == 1 kernel over all of their
    columns, which saves a launch and a kernel tail per extra weight.
    """
    weights = list(weights)
    if not weights:
        return []
    shape = tuple(weights[0].shape)
    for w in weights:
        if tuple(w.shape) != shape:
            raise RuntimeError(f"grouped weights must share one shape, got {tuple(w.shape)} and {shape}")
    num_blocks_per_col, N, _ = shape
    K = num_blocks_per_col * QK4_0
    assert X.shape[1] == K, f"X K dim ({X.shape[1]}) must match weight K ({K})"
    _require_device(X, *weights)
    if (X.dim() != 2 or X.dtype != torch.float16 or X.shape[0] != 1 or N % 16 or N == 0 or K == 0
            or len(weights) > 4):
        return [matmul_ggml_q4_0(X, w) for w in weights]
    for w in weights:
        if w.dtype != torch.uint8 or w.shape[2] != BLOCK_Q4_0_SIZE:
            raise RuntimeError("W_blocks must be uint8 [K/32, N, 18]")
    ws = []
    for w in weights:
        w = w if w.is_contiguous() else w.contiguous()
        ws.append(w.clone() if w.data_ptr() % 16 else w)
    x = X
    if x.stride(1) != 1 or x.stride(0) % 8 or x.stride(0) < K or x.data_ptr() % 16:
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()
    Ys = [torch.empty((1, N), dtype=X.dtype, device=X.device) for _ in ws]
    wp = (ctypes.c_void_p * len(ws))(*[w.data_ptr() for w in ws])
    yp = (ctypes.c_void_p * len(Ys))(*[y.data_ptr() for y in Ys])
    stream = _stream(X.device)
    # Shapes the one launch does not cover run per weight inside the library,
    # with the workspace a single-weight call would get.
    need = int(_lib.lib.mcq4_matmul_workspace_bytes(1, K, N))
    ws_buf, ws_ptr, ws_bytes = None, None, 0
    if need:
        ws_buf = _workspace.get(x.device, stream, need)
        ws_ptr, ws_bytes = ws_buf.data_ptr(), ws_buf.numel()
    with torch.cuda.device(x.device), _workspace.guard(ws_buf, stream):
        _lib.check(_lib.lib.mcq4_matmul_q4_0_f16_grouped(x.data_ptr(), x.stride(0), len(ws), wp, yp, N, 1, K, N,
                                                         ws_ptr, ws_bytes, stream),
                   "mcq4_matmul_q4_0_f16_grouped")
    return Ys
