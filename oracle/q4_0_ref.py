"""CPU restatement of metalcore's GGML block_q4_0 path -- TEST INFRASTRUCTURE ONLY.

This module is the parity oracle.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker (or, for the baseline, as the timed restatement of the reference's CPU
fallback).  The product path (``metalops_amd``) never imports it and has no CPU
fallback.

Reference (all paths under ``packages/metalcore/src/metalcore/``):

* ``quantization.py:303-304``  QK4_0 = 32, BLOCK_Q4_0_SIZE = 18.
* ``quantization.py:307-371``  ``quantize_ggml_q4_0`` (reference rule).
* ``quantization.py:374-419``  ``dequantize_ggml_q4_0``.
* ``quantization.py:422-454``  ``matmul_ggml_q4_0`` (fallback ``X @ dequant(W, X.dtype)``).
* ``native/quant_kernels.metal:1813-1830``  nibble order used by the Metal kernel
  (byte ``i`` of ``qs`` = element ``2i`` low nibble, ``2i+1`` high nibble).

Block layout: ``blocks[kb, n, 0:2]`` = fp16 ``d`` (little endian),
``blocks[kb, n, 2 + i]`` = ``q[2i] | q[2i+1] << 4`` for the 32 weights
``W[kb*32 : kb*32+32, n]``.  Dequant: ``W = (q - 8) * d``.

Two quantizer rules share that layout:

* ``quantize_ref_rule`` -- the reference's own rule: ``d = amax/7`` (0 -> 1),
  ``q = round_half_even(x/d + 8).clamp(0, 15)``.  The division ``amax / 7.0``
  follows torch's CPU semantics (a correctly rounded fp32 divide, verified in the
  CPU test-suite against torch itself).
* ``quantize_llama_rule`` -- the llama.cpp ``quantize_row_q4_0_ref`` rule used to
  generate the benchmark configurations: ``d = max_signed / -8``,
  ``id = 1/d`` (0 when ``d == 0``), ``q = min(15, trunc(x*id + 8.5))``.  It emits
  the same tensor layout and nibble order, so one kernel serves both.

Parity status of each function (how it is pinned):

* ``dequantize``: closed form ``(q - 8) * d`` exact in fp32; pinned by the
  exhaustive nibble x scale table test and the independent C restatement.
* ``quantize_ref_rule``: pinned by known-answer blocks (zero block, single-hot
  +a / -a at elements 0, 1, 16, 31, exact half-way ties resolved half-to-even),
  by the invariants ``q in [1, 15]`` and round-trip error ``<= d/2``, and by the
  independent C restatement (fp32).  Tie cases at inexact quotients, and the
  per-step rounding of fp16 / bf16 weights, are pinned by the torch-semantics
  tests (the reference's own torch ops run on CPU in each dtype).
* ``quantize_llama_rule``: known answers (max-signed element -> q = 0, zero
  block -> d = 0, q = 8) and the C restatement.
* ``matmul_f64`` / ``matmul_f32``: float64 brute force over explicit loops on
  tiny shapes.
"""
from __future__ import annotations

import numpy as np

QK4_0 = 32            # quantization.py:303
BLOCK_Q4_0_SIZE = 18  # quantization.py:304


def _check_weight(weight: np.ndarray) -> tuple[int, int, int]:
    K, N = weight.shape
    assert K % QK4_0 == 0, f"K ({K}) must be divisible by {QK4_0}"
    return K, N, K // QK4_0


def _pack(d32: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Pack fp32 scales ``d32[nb, N]`` and nibbles ``q[nb, 32, N]`` into ``[nb, N, 18]``.

    Follows quantization.py:351-369: d as fp16 bytes, then byte i = q[2i] | q[2i+1] << 4.
    """
    nb, _, N = q.shape
    out = np.zeros((nb, N, BLOCK_Q4_0_SIZE), dtype=np.uint8)
    with np.errstate(over="ignore"):
        out[:, :, 0:2] = d32.astype(np.float16).view(np.uint8).reshape(nb, N, 2)
    qt = np.ascontiguousarray(q.transpose(0, 2, 1))        # [nb, N, 32]
    out[:, :, 2:18] = qt[:, :, 0::2] | (qt[:, :, 1::2] << 4)
    return out


def quantize_ref_rule(weight: np.ndarray, dtype: str = "float32") -> np.ndarray:
    """Restates quantization.py:307-371 (``quantize_ggml_q4_0``).

    ``dtype`` is the weight's torch dtype ("float32", "float16" or "bfloat16";
    for bfloat16 pass fp32 values that are bf16-representable).  The reference
    runs each step as a torch op in that dtype (:338, :341, :342, :347), which
    on CPU is the fp32 operation rounded to the dtype; ``d.to(float16)`` (:352)
    is one more rounding for bf16.
    """
    from .int4_ref import round_to
    code = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}[dtype]
    if dtype == "float32":
        w = np.ascontiguousarray(weight, dtype=np.float32)
    else:
        w = round_to(np.asarray(weight, dtype=np.float32), code)
        assert np.array_equal(w, np.asarray(weight, dtype=np.float32)), "weight not representable in dtype"
    K, N, nb = _check_weight(w)
    rnd = (lambda v: v) if dtype == "float32" else (lambda v: round_to(v, code))
    wb = w.reshape(nb, QK4_0, N)                                  # :335
    amax = np.abs(wb).max(axis=1)                                 # :338, exact
    d = rnd(amax / np.float32(7.0))                               # :341
    d = np.where(d > 0, d, np.float32(1.0)).astype(np.float32)    # :342
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        t = rnd(rnd(wb / d[:, None, :]) + np.float32(8.0))        # :347, one op at a time
    q = np.clip(np.round(t), 0, 15).astype(np.uint8)              # round half to even
    return _pack(d, q)


def quantize_llama_rule(weight: np.ndarray) -> np.ndarray:
    """llama.cpp ``quantize_row_q4_0_ref`` scale/rounding rule in metalcore's layout.

    Rule: per block pick the element with the largest |x|
    (first one on ties), ``d = max / -8``, ``id = 1/d`` (0 if d == 0),
    ``q = min(15, (int8)(x*id + 8.5))``.
    """
    w = np.ascontiguousarray(weight, dtype=np.float32)
    K, N, nb = _check_weight(w)
    wb = w.reshape(nb, QK4_0, N)
    idx = np.abs(wb).argmax(axis=1)                               # first max on ties
    mx = np.take_along_axis(wb, idx[:, None, :], axis=1)[:, 0, :]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    t = wb * inv[:, None, :] + np.float32(8.5)
    q = np.minimum(np.trunc(t), 15).astype(np.int32)
    q = np.clip(q, 0, 15).astype(np.uint8)   # x*id >= -8 so trunc(t) >= 0 already
    return _pack(d, q)


def unpack_nibbles(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Return (q[nb, N, 32] uint8, d[nb, N] float16) from ``[nb, N, 18]`` blocks."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb, N, bs = b.shape
    assert bs == BLOCK_Q4_0_SIZE
    d = b[:, :, 0:2].copy().view(np.float16).reshape(nb, N)
    qs = b[:, :, 2:18]
    q = np.empty((nb, N, QK4_0), dtype=np.uint8)
    q[:, :, 0::2] = qs & 0x0F
    q[:, :, 1::2] = qs >> 4
    return q, d


def dequantize(blocks: np.ndarray, dtype=np.float16) -> np.ndarray:
    """Restates quantization.py:374-419: ``(q - 8) * d`` in fp32, then cast to ``dtype``."""
    q, d = unpack_nibbles(blocks)
    nb, N, _ = q.shape
    wq = (q.astype(np.float32) - np.float32(8.0)) * d.astype(np.float32)[:, :, None]
    with np.errstate(over="ignore"):   # |(q-8)*d| > 65504 -> inf in fp16, as torch's cast does
        return np.ascontiguousarray(wq.transpose(0, 2, 1).reshape(nb * QK4_0, N)).astype(dtype)


def matmul_f32(X: np.ndarray, blocks: np.ndarray) -> np.ndarray:
    """``X.float() @ dequant_f32(W)``: the tolerance reference for the kernels."""
    nb = blocks.shape[0]
    assert X.shape[1] == nb * QK4_0, f"X K dim ({X.shape[1]}) must match weight K ({nb * QK4_0})"
    return X.astype(np.float32) @ dequantize(blocks, np.float32)


def matmul_xdtype(X: np.ndarray, blocks: np.ndarray, dtype: str) -> np.ndarray:
    """The reference's path for non-fp16 activations (quantization.py:452-454):
    ``W = dequantize(blocks, X.dtype)`` (the exact fp32 product rounded once to
    ``dtype``), ``Y = X @ W`` summed in float64 here, then rounded to ``dtype``.
    ``X`` holds values representable in ``dtype`` ("float32" or "bfloat16")."""
    from .int4_ref import round_to
    code = {"float32": "f32", "bfloat16": "bf16"}[dtype]
    nb = blocks.shape[0]
    assert X.shape[1] == nb * QK4_0, f"X K dim ({X.shape[1]}) must match weight K ({nb * QK4_0})"
    W = round_to(dequantize(blocks, np.float32), code).astype(np.float64)
    return round_to((X.astype(np.float64) @ W).astype(np.float32), code)


def matmul_f64(X: np.ndarray, blocks: np.ndarray) -> np.ndarray:
    """Brute-force float64 ``sum_k X[m,k] * (q-8) * d`` with explicit loops (tiny shapes)."""
    q, d = unpack_nibbles(blocks)
    nb, N, _ = q.shape
    M, K = X.shape
    assert K == nb * QK4_0
    Xd = X.astype(np.float64)
    Y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for kb in range(nb):
                dd = float(d[kb, n])
                for j in range(QK4_0):
                    acc += Xd[m, kb * QK4_0 + j] * ((int(q[kb, n, j]) - 8) * dd)
            Y[m, n] = acc
    return Y


def fallback_torch_cpu(X, blocks):
    """Restates the reference's fallback (quantization.py:452-454) with torch CPU ops.

    ``W = dequantize_ggml_q4_0(W_blocks, X.dtype); return X @ W`` -- dequant is
    repeated on every call exactly as the reference does.  Used only as the timed
    CPU baseline in ``bench.py``.
    """
    import torch

    nb, N, _ = blocks.shape
    K = nb * QK4_0
    d = blocks[:, :, 0:2].contiguous().view(torch.float16).view(nb, N)
    packed = blocks[:, :, 2:18]
    q = torch.empty((nb, N, QK4_0), dtype=torch.int8)
    q[:, :, 0::2] = (packed & 0x0F).to(torch.int8)
    q[:, :, 1::2] = (packed >> 4).to(torch.int8)
    W = ((q.float() - 8.0) * d.unsqueeze(2).float()).permute(0, 2, 1).reshape(K, N).to(X.dtype)
    return X @ W
