"""Per-group INT4 quantize / dequantize / matmul and ``Int4Linear`` on MI355X.

Mirrors metalcore's per-group INT4 API
(``packages/metalcore/src/metalcore/quantization.py``):

* ``quantize_int4(weight, group_size=128)``                       -- :26-92
* ``dequantize_int4(W_packed, scales, zeros, group_size, dtype)`` -- :95-153
* ``matmul_int4(X, W_packed, scales, zeros, group_size=128)``     -- :156-239
* ``matmul_int4_silu`` / ``matmul_int4_gelu`` (the native bindings of
  ``native/core_mps.mm:5780-5914``, registered at :6936-6937)
* ``fused_rmsnorm_linear_int4`` (native binding ``core_mps.mm:3017-3103``,
  registered at :6885)
* ``quantize_to_int4(weight, group_size)`` (GPU-side quantizer binding,
  ``native/core_mps.mm:4655-4700``, registered at :6887)
* ``matmul_int8(X, W_packed, scales, zeros, group_size=128)``     -- :242-286
* ``Int4Linear``                                                  -- :457-613

Same names, argument order, defaults, layouts (``W_packed [K/2, N]`` uint8,
``scales``/``zeros`` ``[ceil(K/group_size), N]`` in the weight's dtype) and
result dtypes.  The computation runs in the HIP kernels of ``libmcq4.so``;
tensors must live on a ROCm device and there is no CPU fallback.  Work is
enqueued on the current stream without synchronising.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from .quantization import _workspace   # split-K workspace shared with the q4_0 path

__all__ = [
    "quantize_int4",
    "dequantize_int4",
    "matmul_int4",
    "matmul_int4_silu",
    "matmul_int4_gelu",
    "fused_rmsnorm_linear_int4",
    "quantize_to_int4",
    "matmul_int8",
    "Int4Linear",
]

_DT = {torch.float32: _lib.MCQ4_DTYPE_F32, torch.float16: _lib.MCQ4_DTYPE_F16,
       torch.bfloat16: _lib.MCQ4_DTYPE_BF16}


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "metalops_amd int4 ops run only on a ROCm GPU (torch device 'cuda'); "
                f"got a tensor on '{t.device}'. There is no CPU fallback.")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on one device, got {dev} and {t.device}")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dense(t: torch.Tensor, align: int) -> torch.Tensor:
    t = t.contiguous()
    if t.data_ptr() % align:
        t = t.clone()
    return t


def quantize_int4(
    weight: torch.Tensor,
    group_size: int = 128,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Quantize ``weight[K, N]`` to INT4 with a scale and zero point per group of rows.

    Returns ``(weight_packed [K/2, N] uint8, scales [G, N], zeros [G, N])`` with
    ``G = ceil(K / group_size)`` and scales/zeros in ``weight.dtype``.  Per group
    and column: ``scale = (max - min) / 15`` (at least 1e-8), ``zero = -min / scale``,
    ``q = round_half_even(w / scale + zero)`` clamped to [0, 15]; row ``k`` is
    the low nibble of byte row ``k // 2`` for even ``k``, the high nibble for
    odd ``k`` (quantization.py:62-90).  Each step is rounded to the weight's
    dtype as the reference's torch ops are.  float32, float16 and bfloat16
    weights are supported.
    """
    K, N = weight.shape
    if K % 2:
        # The reference indexes byte row K // 2 of a [K // 2, N] tensor here.
        raise IndexError(f"K ({K}) must be even: two rows share each packed byte")
    _require_device(weight)
    if weight.dtype not in _DT:
        raise RuntimeError(f"quantize_int4: unsupported weight dtype {weight.dtype}")
    w = weight
    es = w.element_size()
    if w.stride(1) != 1 or w.stride(0) < N or w.data_ptr() % es:
        w = w.contiguous()
    G = (K + group_size - 1) // group_size
    packed = torch.empty((K // 2, N), dtype=torch.uint8, device=w.device)
    scales = torch.empty((G, N), dtype=w.dtype, device=w.device)
    zeros = torch.empty((G, N), dtype=w.dtype, device=w.device)
    if K == 0 or N == 0:
        return packed, scales, zeros
    with torch.cuda.device(w.device):
        _lib.check(_lib.lib.mcq4_quantize_int4(w.data_ptr(), _DT[w.dtype], w.stride(0), K, N,
                                               group_size, packed.data_ptr(), scales.data_ptr(),
                                               zeros.data_ptr(), _stream(w.device)),
                   "mcq4_quantize_int4")
    return packed, scales, zeros


def quantize_to_int4(weight: torch.Tensor, group_size: int = 128):
    """GPU-side INT4 quantization (the reference's native ``quantize_to_int4``).

    The ``quantize_int4`` computation in fp32 with Metal's ``round`` (half away
    from zero), as quant_kernels.metal:634-686; scales and zeros are fp32.  The
    reference kernel reads the weight as fp32 (core_mps.mm:4671-4677), so other
    dtypes are upcast first.  K and the group size must be even.
    """
    if weight.dim() != 2:
        raise RuntimeError("weight must be 2D [K, N]")
    K, N = weight.shape
    if K % 2:
        raise RuntimeError("K must be even for INT4 packing")
    if group_size % 2:
        raise RuntimeError(f"group_size ({group_size}) must be even")
    _require_device(weight)
    w = weight.float()
    if w.stride(1) != 1 or w.stride(0) < N or w.data_ptr() % 4:
        w = w.contiguous()
    G = (K + group_size - 1) // group_size
    packed = torch.empty((K // 2, N), dtype=torch.uint8, device=w.device)
    scales = torch.empty((G, N), dtype=torch.float32, device=w.device)
    zeros = torch.empty((G, N), dtype=torch.float32, device=w.device)
    if K and N:
        with torch.cuda.device(w.device):
            _lib.check(_lib.lib.mcq4_quantize_to_int4(w.data_ptr(), w.stride(0), K, N, group_size,
                                                      packed.data_ptr(), scales.data_ptr(),
                                                      zeros.data_ptr(), _stream(w.device)),
                       "mcq4_quantize_to_int4")
    return packed, scales, zeros


def _sz_pair(scales: torch.Tensor, zeros: torch.Tensor):
    """Scales and zeros in one kernel dtype (exact upcast to fp32 when they differ)."""
    if scales.dtype != zeros.dtype or scales.dtype not in _DT:
        scales, zeros = scales.float(), zeros.float()
    return _dense(scales, 16), _dense(zeros, 16)


def _check_shapes(W_packed, scales, zeros, group_size):
    Kh, N = W_packed.shape
    K = Kh * 2
    G = (K + group_size - 1) // group_size
    if W_packed.dtype != torch.uint8:
        raise RuntimeError("W_packed must be uint8 [K/2, N]")
    if tuple(scales.shape) != (G, N) or tuple(zeros.shape) != (G, N):
        raise RuntimeError(
            f"scales/zeros must be [{G}, {N}] for K={K}, group_size={group_size}; got "
            f"{tuple(scales.shape)} and {tuple(zeros.shape)}")
    return K, N


def dequantize_int4(
    W_packed: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    group_size: int = 128,
    dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """``W[k, n] = ((q - zero) * scale)`` computed in fp32, returned in ``dtype`` (default fp16).

    Zero and scale are upcast exactly, the subtraction and the product are two
    fp32 roundings, and the result is rounded once to ``dtype`` -- bit for bit
    what quantization.py:144-151 computes.
    """
    if dtype is None:
        dtype = torch.float16
    _require_device(W_packed, scales, zeros)
    K, N = _check_shapes(W_packed, scales, zeros, group_size)
    s, z = _sz_pair(scales, zeros)
    p = _dense(W_packed, 1)
    kernel_dtype = dtype if dtype in _DT else torch.float32
    out = torch.empty((K, N), dtype=kernel_dtype, device=p.device)
    if K and N:
        with torch.cuda.device(p.device):
            _lib.check(_lib.lib.mcq4_dequantize_int4(p.data_ptr(), s.data_ptr(), z.data_ptr(),
                                                     _DT[s.dtype], K, N, group_size,
                                                     out.data_ptr(), N, _DT[kernel_dtype],
                                                     _stream(p.device)),
                       "mcq4_dequantize_int4")
    return out if out.dtype == dtype else out.to(dtype)


_FN = {0: "mcq4_matmul_int4", 1: "mcq4_matmul_int4_silu", 2: "mcq4_matmul_int4_gelu"}


def _matmul(X, W_packed, scales, zeros, group_size, act):
    _require_device(X, W_packed, scales, zeros)
    K, N = _check_shapes(W_packed, scales, zeros, group_size)
    batched = X.dim() == 3                                   # quantization.py:185-192
    if X.dim() not in (2, 3):
        raise RuntimeError(f"X must be [M, K] or [B, M, K], got shape {tuple(X.shape)}")
    if X.shape[-1] != K:
        raise RuntimeError(f"X K dim ({X.shape[-1]}) must match weight K ({K})")
    lead = X.shape[:-1]
    x = X.reshape(-1, K)
    out_dtype = X.dtype
    if x.dtype not in _DT:
        x = x.float()
    if x.stride(1) != 1 or x.stride(0) < K or x.stride(0) % 8 or x.data_ptr() % 16:
        x = _dense(x, 16)
    M = x.shape[0]
    s, z = _sz_pair(scales, zeros)
    p = _dense(W_packed, 16)
    Y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    if M and N:
        if K == 0:
            Y.zero_()
        else:
            xdt = _DT[x.dtype]
            need = int(_lib.lib.mcq4_matmul_int4_workspace_bytes(M, K, N, group_size, xdt))
            stream = _stream(x.device)
            ws, ws_ptr, ws_bytes = None, None, 0
            if need:
                ws = _workspace.get(x.device, stream, need)
                ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
            fn = getattr(_lib.lib, _FN[act])
            with torch.cuda.device(x.device), _workspace.guard(ws, stream):
                _lib.check(fn(x.data_ptr(), xdt, x.stride(0), p.data_ptr(), s.data_ptr(),
                              z.data_ptr(), _DT[s.dtype], Y.data_ptr(), N, M, K, N, group_size,
                              ws_ptr, ws_bytes, stream),
                           _FN[act])
    Y = Y if Y.dtype == out_dtype else Y.to(out_dtype)
    return Y.reshape(*lead, N) if batched else Y


def matmul_int4(
    X: torch.Tensor,
    W_packed: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    group_size: int = 128,
) -> torch.Tensor:
    """``Y = X @ dequant(W_packed, scales, zeros)`` for ``X`` ``[M, K]`` or ``[B, M, K]``.

    fp32 accumulation; the result has ``X``'s dtype.  fp16 activations run the
    MFMA kernels (decode GEMV for M <= 16 rows, and up to 32 rows when N is a
    multiple of 128; prefill GEMM above); fp32 and
    bf16 activations run the general fp32 kernel with the weight rounded to
    ``X``'s dtype first, as the reference builds ``W`` in ``X.dtype``
    (quantization.py:220-239).
    """
    return _matmul(X, W_packed, scales, zeros, group_size, 0)


def _fused(X, W_packed, scales, zeros, group_size, act):
    if X.dtype != torch.float16:
        raise RuntimeError("Fused kernel requires half precision")   # core_mps.mm:5795
    if X.dim() != 2:
        raise RuntimeError(f"X must be [M, K], got shape {tuple(X.shape)}")
    return _matmul(X, W_packed, scales, zeros, group_size, act)


def matmul_int4_silu(X, W_packed, scales, zeros, group_size: int = 128) -> torch.Tensor:
    """``silu(X @ dequant(W))`` with the activation fused into the matmul store (fp16 X)."""
    return _fused(X, W_packed, scales, zeros, group_size, 1)


def matmul_int4_gelu(X, W_packed, scales, zeros, group_size: int = 128) -> torch.Tensor:
    """``gelu(X @ dequant(W))`` (tanh form, as the fused reference kernel) fused into the store."""
    return _fused(X, W_packed, scales, zeros, group_size, 2)


def fused_rmsnorm_linear_int4(X, W_norm, W_packed, scales, zeros, eps, group_size):
    """``matmul_int4(rmsnorm(X, W_norm, eps), W_packed, scales, zeros, group_size)`` (fp16).

    RMSNorm as the reference's half kernel (training_kernels.metal:425-488):
    ``rstd = 1/sqrt(mean(x^2) + eps)`` in fp32, ``X_norm = fp16(x * rstd * w)``;
    the normalization kernel and the INT4 matmul run back to back on the current
    stream with ``X_norm`` in the shared workspace.  ``X`` is ``[B, K]`` fp16 and
    ``W_norm`` ``[K]`` fp16, as the reference binding requires (core_mps.mm:3029).
    """
    if X.dtype != torch.float16:
        raise RuntimeError("Fused kernel requires half precision")
    if X.dim() != 2:
        raise RuntimeError(f"X must be [B, K], got shape {tuple(X.shape)}")
    _require_device(X, W_norm, W_packed, scales, zeros)
    K, N = _check_shapes(W_packed, scales, zeros, group_size)
    if X.shape[1] != K or W_norm.numel() != K:
        raise RuntimeError(f"X [B, {X.shape[1]}] and W_norm [{W_norm.numel()}] must match K={K}")
    x = X if (X.stride(1) == 1 and X.data_ptr() % 2 == 0) else X.contiguous()
    wn = W_norm.to(torch.float16).contiguous()
    s, z = _sz_pair(scales, zeros)
    p = _dense(W_packed, 16)
    M = x.shape[0]
    Y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    if M == 0:
        return Y
    need = int(_lib.lib.mcq4_fused_rmsnorm_linear_int4_workspace_bytes(M, K, N, group_size))
    stream = _stream(x.device)
    ws = _workspace.get(x.device, stream, need + 256)
    base = (ws.data_ptr() + 255) // 256 * 256
    with torch.cuda.device(x.device), _workspace.guard(ws, stream, base):
        _lib.check(_lib.lib.mcq4_fused_rmsnorm_linear_int4(
            x.data_ptr(), x.stride(0), wn.data_ptr(), float(eps), p.data_ptr(), s.data_ptr(),
            z.data_ptr(), _DT[s.dtype], Y.data_ptr(), N, M, K, N, group_size, base,
            ws.numel() - (base - ws.data_ptr()), stream),
            "mcq4_fused_rmsnorm_linear_int4")
    return Y


def matmul_int8(
    X: torch.Tensor,
    W_packed: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    group_size: int = 128,
) -> torch.Tensor:
    """``Y = X @ dequant(W)`` with int8 weights ``W_packed [K, N]`` (quantization.py:242-286).

    ``W[k, n] = (q - zero) * scale`` per group of ``group_size`` rows; fp32
    accumulation, result in ``X``'s dtype.  fp16 activations run the MFMA
    kernels, other dtypes the general kernel (weights rounded to ``X``'s dtype
    as the reference's fallback builds ``W`` in ``X.dtype``).
    """
    _require_device(X, W_packed, scales, zeros)
    if X.dim() != 2:
        raise RuntimeError(f"X must be [M, K], got shape {tuple(X.shape)}")
    if W_packed.dtype not in (torch.int8, torch.uint8):
        raise RuntimeError("W_packed must be int8 [K, N]")
    K, N = W_packed.shape
    G = (K + group_size - 1) // group_size
    if tuple(scales.shape) != (G, N) or tuple(zeros.shape) != (G, N):
        raise RuntimeError(f"scales/zeros must be [{G}, {N}] for K={K}, group_size={group_size}")
    if X.shape[1] != K:
        raise RuntimeError(f"X K dim ({X.shape[1]}) must match weight K ({K})")
    out_dtype = X.dtype
    x = X if X.dtype in _DT else X.float()
    if x.stride(1) != 1 or x.stride(0) < K or x.stride(0) % 8 or x.data_ptr() % 16:
        x = _dense(x, 16)
    M = x.shape[0]
    s, z = _sz_pair(scales, zeros)
    w = _dense(W_packed.view(torch.int8), 16)
    Y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    if M and N:
        if K == 0:
            Y.zero_()
        else:
            xdt = _DT[x.dtype]
            need = int(_lib.lib.mcq4_matmul_int8_workspace_bytes(M, K, N, group_size, xdt))
            stream = _stream(x.device)
            ws, ws_ptr, ws_bytes = None, None, 0
            if need:
                ws = _workspace.get(x.device, stream, need)
                ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
            with torch.cuda.device(x.device), _workspace.guard(ws, stream):
                _lib.check(_lib.lib.mcq4_matmul_int8(x.data_ptr(), xdt, x.stride(0), w.data_ptr(),
                                                     s.data_ptr(), z.data_ptr(), _DT[s.dtype],
                                                     Y.data_ptr(), N, M, K, N, group_size, ws_ptr,
                                                     ws_bytes, stream),
                           "mcq4_matmul_int8")
    return Y if Y.dtype == out_dtype else Y.to(out_dtype)


class Int4Linear(nn.Module):
    """Linear layer over per-group INT4 weights (API of quantization.py:457-613).

    State (the serialized format, kept as in the reference): buffers
    ``weight_packed [in/2, out]`` uint8, ``scales`` / ``zeros [G, out]`` in the
    layer's dtype (fp32 when none is given) and ``bias [out]`` (or a ``None``
    parameter).

    Two execution modes:

    * dense (``dequantize()``, the default after ``from_float``): a dequantized
      copy of the weight, never serialized, feeds a plain GEMM; activations are
      cast to that copy's dtype (fp16 by default) and the result back;
    * quantized (``keep_quantized()``): every forward runs the INT4 kernels of
      ``matmul_int4`` on the packed weight -- 4x less weight traffic, which is
      what a memory-bound decode step wants.

    Inputs of any rank ``[..., in]`` are flattened to 2-D for the kernels.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        group_size: int = 128,
        bias: bool = True,
        device: Optional[torch.device] = None,
        dtype: Optional[torch.dtype] = None,
        dequant_on_load: bool = True,
    ):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self._dequant_on_load = dequant_on_load
        self._weight_dequant: Optional[torch.Tensor] = None
        param_dtype = dtype if dtype is not None else torch.float32
        groups = -(-in_features // group_size)
        factory = {"device": device}
        self.register_buffer("weight_packed",
                             torch.zeros(in_features // 2, out_features, dtype=torch.uint8, **factory))
        self.register_buffer("scales", torch.ones(groups, out_features, dtype=param_dtype, **factory))
        self.register_buffer("zeros", torch.zeros(groups, out_features, dtype=param_dtype, **factory))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=param_dtype, **factory))
        else:
            self.register_parameter("bias", None)

    # -- mode switches -------------------------------------------------------
    def dequantize(self, dtype: Optional[torch.dtype] = None) -> None:
        """Switch to dense mode with a weight dequantized to ``dtype`` (fp16 by default)."""
        target = torch.float16 if dtype is None else dtype
        self._weight_dequant = dequantize_int4(self.weight_packed, self.scales, self.zeros,
                                               self.group_size, target)
        self._dequant_on_load = True

    def keep_quantized(self) -> None:
        """Switch to quantized mode: free the dense copy, run the INT4 kernels."""
        self._dequant_on_load = False
        self._weight_dequant = None

    # -- construction --------------------------------------------------------
    @torch.no_grad()
    def _load_from_dense(self, weight_in_out: torch.Tensor, bias: Optional[torch.Tensor]) -> None:
        packed, scales, zeros = quantize_int4(weight_in_out, self.group_size)
        for name, value in (("weight_packed", packed), ("scales", scales), ("zeros", zeros)):
            getattr(self, name).copy_(value)
        if bias is not None:
            self.bias.copy_(bias)

    @classmethod
    def from_float(
        cls,
        module: nn.Linear,
        group_size: int = 128,
        dequant_on_load: bool = True,
    ) -> "Int4Linear":
        """Quantize an ``nn.Linear``: its ``[out, in]`` weight is packed as ``[in, out]``."""
        w = module.weight
        layer = cls(module.in_features, module.out_features, group_size=group_size,
                    bias=module.bias is not None, device=w.device, dtype=w.dtype,
                    dequant_on_load=dequant_on_load)
        layer._load_from_dense(w.detach().t().contiguous(),
                               None if module.bias is None else module.bias.detach())
        if dequant_on_load:
            layer.dequantize()
        return layer

    # -- compute -------------------------------------------------------------
    def _dense(self, x: torch.Tensor) -> torch.Tensor:
        w = self._weight_dequant
        return (x.to(w.dtype) @ w).to(x.dtype)

    def _quantized(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        y2 = matmul_int4(x.reshape(-1, x.shape[-1]), self.weight_packed, self.scales, self.zeros,
                         self.group_size)
        return y2.reshape(*lead, self.out_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self._dense(x) if self._weight_dequant is not None else self._quantized(x)
        return y if self.bias is None else y + self.bias

    def extra_repr(self) -> str:
        mode = "fast_fp16" if self._weight_dequant is not None else "int4_kernel"
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"group_size={self.group_size}, bias={self.bias is not None}, mode={mode}")
