"""CPU restatement of metalcore's per-group INT4 path -- TEST INFRASTRUCTURE ONLY.

Like ``q4_0_ref``, this module is the parity oracle: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` may import it,
and only as the checker.  The product path never calls it.

Reference: ``packages/metalcore/src/metalcore/quantization.py``

* ``:26-92``    ``quantize_int4(weight, group_size=128)`` -> ``(W_packed [K/2, N] u8,
  scales [G, N], zeros [G, N])`` with ``G = ceil(K / group_size)`` and
  scales/zeros in ``weight.dtype`` (``:53-58``).  Per group and column
  (``:62-92``): ``scale = (max - min) / 15``, ``scale = scale.clamp(min=1e-8)``,
  ``zero = -min / scale``, ``q = (w / scale + zero).round().clamp(0, 15)``; row
  ``k`` goes to byte ``k // 2``, low nibble for even ``k``, high nibble for odd.
  Every step is a torch op in ``weight.dtype``: computed in fp32 and rounded to
  that dtype after each op (fp32 has enough precision that this equals the
  correctly rounded op in fp16/bf16).  ``round`` is half-to-even.
* ``:95-153``   ``dequantize_int4``: ``W[k, n] = ((q.float() - zero) * scale).to(dtype)``
  (``:151``): the stored zero and scale are upcast exactly, subtract and multiply
  are separate fp32 roundings, then one rounding to ``dtype`` (default fp16).
* ``:156-239``  ``matmul_int4``: ``X @ W`` with ``W`` the same dequantized values in
  ``X.dtype`` (``:236-239``); ``X`` 2-D or 3-D (``:185-204``).

Parity status (how each function is pinned; the CPU tests hold the checks):

* ``dequantize``: closed form; known-answer tables with hand-computed values
  (q = 0..15 against chosen scale/zero), and the invariant that dequantizing a
  fresh quantization of a ladder ``min + i*step`` returns the ladder.
* ``quantize``: known answers (a group's min -> q 0 and max -> q 15; an exact
  ladder ``min + i*step`` -> q = i; constant groups; the fp16 clamp constant 1e-8
  rounding to 0), the bound ``|w - dequant| <= scale/2 + rounding`` for every
  element, per-op-rounding emulation checked against torch's own CPU fp16/bf16
  ops on the same inputs, and nibble order by single-row probes.
* ``matmul_f64``: float64 brute force over explicit loops on tiny shapes.
"""
from __future__ import annotations

import numpy as np

DEFAULT_GROUP = 128

# dtype codes shared with the C ABI (include/mcq4.h)
F32, F16, BF16 = "f32", "f16", "bf16"


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bf16, returned as fp32 values (NaN kept quiet)."""
    x = np.asarray(x, dtype=np.float32)
    shape = x.shape
    x = x.reshape(-1)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    out[np.isnan(x)] = np.float32(np.nan)
    return out.reshape(shape)


def round_to(x, dtype: str) -> np.ndarray:
    """Round fp32 values to ``dtype`` and return them as fp32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == F32:
        return x.copy()
    if dtype == F16:
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(np.float32)
    if dtype == BF16:
        return round_bf16(x)
    raise ValueError(dtype)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16-representable fp32 values -> uint16 bit patterns."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize(weight: np.ndarray, group_size: int = DEFAULT_GROUP, dtype: str = F32,
             rounding: str = "even"):
    """Restates quantization.py:49-92 (``rounding="even"``: torch.round).

    ``rounding="away"`` with fp32 gives the GPU-side quantizer quantize_to_int4
    (quant_kernels.metal:634-686: the same fp32 steps, Metal round() = half
    away from zero; even group sizes).

    ``weight`` holds values representable in ``dtype`` (as fp32).  Returns
    ``(packed uint8 [K/2, N], scales fp32 [G, N], zeros fp32 [G, N])``; scales
    and zeros hold ``dtype`` values.
    """
    w = round_to(weight, dtype)
    K, N = w.shape
    assert K % 2 == 0, "K must be even (two rows per byte)"
    G = (K + group_size - 1) // group_size
    R = lambda v: round_to(v, dtype)
    clamp_min = R(np.float32(1e-8))                                       # :75 scalar in dtype
    scales = np.zeros((G, N), dtype=np.float32)
    zeros = np.zeros((G, N), dtype=np.float32)
    q_all = np.zeros((K, N), dtype=np.uint8)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        for g in range(G):                                                # :62
            k0, k1 = g * group_size, min((g + 1) * group_size, K)
            grp = w[k0:k1]
            mn = grp.min(axis=0)                                          # :69-70
            mx = grp.max(axis=0)
            scale = R(R(mx - mn) / np.float32(15.0))                      # :74
            scale = np.maximum(scale, clamp_min)                          # :75
            zero = R(-mn / scale)                                         # :76
            scales[g], zeros[g] = scale, zero
            t = R(R(grp / scale) + zero)                                  # :83
            r = np.round(t) if rounding == "even" else np.sign(t) * np.floor(np.abs(t) + 0.5)
            q_all[k0:k1] = np.clip(np.nan_to_num(r, nan=0.0), 0, 15).astype(np.uint8)
    packed = (q_all[0::2] | (q_all[1::2] << 4)).astype(np.uint8)          # :85-90
    return packed, scales, zeros


def unpack(packed: np.ndarray) -> np.ndarray:
    """``[K/2, N]`` bytes -> ``q[K, N]`` (row 2i low nibble, 2i+1 high nibble)."""
    p = np.asarray(packed, dtype=np.uint8)
    q = np.empty((2 * p.shape[0], p.shape[1]), dtype=np.uint8)
    q[0::2] = p & 0x0F
    q[1::2] = p >> 4
    return q


def dequantize(packed, scales, zeros, group_size: int = DEFAULT_GROUP, out: str = F16):
    """Restates quantization.py:139-151; returns fp32 values of dtype ``out``."""
    q = unpack(packed).astype(np.float32)
    K = q.shape[0]
    g = np.arange(K) // group_size
    s = np.asarray(scales, dtype=np.float32)[g]
    z = np.asarray(zeros, dtype=np.float32)[g]
    with np.errstate(over="ignore", invalid="ignore"):
        w = ((q - z).astype(np.float32) * s).astype(np.float32)
    return round_to(w, out)


def matmul_f32(X, packed, scales, zeros, group_size: int = DEFAULT_GROUP):
    """``X.float() @ dequant_f32(W)``: the tolerance reference for the kernels."""
    X = np.asarray(X, dtype=np.float32)
    lead = X.shape[:-1]
    W = dequantize(packed, scales, zeros, group_size, F32)
    Y = X.reshape(-1, X.shape[-1]).astype(np.float64) @ W.astype(np.float64)
    return Y.astype(np.float32).reshape(*lead, -1)


def matmul_f64(X, packed, scales, zeros, group_size: int = DEFAULT_GROUP):
    """Brute-force float64 ``sum_k X[m,k] * (q[k,n] - z) * s`` with explicit loops."""
    q = unpack(packed)
    X = np.asarray(X, dtype=np.float64)
    M, K = X.shape
    N = q.shape[1]
    Y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                g = k // group_size
                w = (float(q[k, n]) - float(zeros[g, n])) * float(scales[g, n])
                acc += X[m, k] * w
            Y[m, n] = acc
    return Y


def fallback_torch_cpu(X, packed, scales, zeros, group_size: int = DEFAULT_GROUP):
    """The reference's CPU path for matmul_int4 (quantization.py:220-239): build
    W in X.dtype from ((q - zero) * scale) in fp32, then ``X @ W`` with torch on
    the CPU.  The row loop of the reference is vectorised here (same values);
    used as the CPU baseline of the benchmark."""
    import torch
    W = dequantize(packed, scales, zeros, group_size, F32)
    Wt = torch.from_numpy(W).to(X.dtype)
    return X @ Wt


def rmsnorm_f16(X, w, eps):
    """RMSNorm of fused_rmsnorm_linear_int4 (training_kernels.metal:425-488):
    rstd = 1/sqrt(sum(x^2)/K + eps) per row, X_norm = fp16((x * rstd) * w), with
    fp16 inputs.  The sum is taken in float64 here (the kernels' fp32 sums differ
    in the last bits, which can move an fp16 result by one ulp)."""
    x = np.asarray(X, dtype=np.float16).astype(np.float32)
    wf = np.asarray(w, dtype=np.float16).astype(np.float32)
    ss = (x.astype(np.float64) ** 2).sum(axis=1)
    rstd = (1.0 / np.sqrt(ss / x.shape[1] + eps)).astype(np.float32)
    return ((x * rstd[:, None]).astype(np.float32) * wf).astype(np.float16)


# ---- per-group INT8 (quantization.py:242-286) ----------------------------------

def dequantize_int8(W_q, scales, zeros, group_size: int = DEFAULT_GROUP, out: str = F32):
    """``W = (q.float() - zero) * scale`` per group of rows (quantization.py:276-284)."""
    q = np.asarray(W_q, dtype=np.int8).astype(np.float32)
    K = q.shape[0]
    g = np.arange(K) // group_size
    s = np.asarray(scales, dtype=np.float32)[g]
    z = np.asarray(zeros, dtype=np.float32)[g]
    with np.errstate(over="ignore", invalid="ignore"):
        w = ((q - z).astype(np.float32) * s).astype(np.float32)
    return round_to(w, out)


def matmul_int8_f32(X, W_q, scales, zeros, group_size: int = DEFAULT_GROUP):
    """``X.float() @ dequant_int8_f32(W)``: the tolerance reference."""
    X = np.asarray(X, dtype=np.float32)
    W = dequantize_int8(W_q, scales, zeros, group_size, F32)
    return (X.astype(np.float64) @ W.astype(np.float64)).astype(np.float32)


def matmul_int8_f64(X, W_q, scales, zeros, group_size: int = DEFAULT_GROUP):
    """Brute-force float64 loops on tiny shapes."""
    q = np.asarray(W_q, dtype=np.int8)
    X = np.asarray(X, dtype=np.float64)
    M, K = X.shape
    N = q.shape[1]
    Y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                g = k // group_size
                acc += X[m, k] * (float(q[k, n]) - float(zeros[g, n])) * float(scales[g, n])
            Y[m, n] = acc
    return Y
