"""Writes tests/golden/q4_0_golden.npz from the oracle (oracle/q4_0_ref.py).

The reference ships no q4_0 vectors (its tests cover no quantization), so these
fixtures freeze the pinned oracle's outputs on small seeded inputs that include
the edge cases (all-zero blocks, exact .5 ties, single-hot blocks, outliers,
negative and subnormal scales, ragged N).  The CPU suite checks that the oracle
still reproduces them; the GPU suite checks the HIP kernels against them.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import q4_0_ref as R  # noqa: E402


def build():
    rng = np.random.default_rng(20240601)
    K, N = 128, 37
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    mask = rng.random(W.shape) < 0.01
    W[mask] = (rng.standard_normal(int(mask.sum())) * 0.2).astype(np.float32)
    W[0:32, 0] = 0.0                                                  # zero block
    W[32:64, 1] = np.array([7.0, 0.5, 1.5, -0.5, -1.5, 2.5, -2.5, 6.5] + [0.0] * 24, np.float32)
    W[64:96, 2] = 0.0
    W[64 + 17, 2] = -0.3                                              # single-hot negative
    W[96:128, 3] = np.float32(1e-6) * rng.standard_normal(32).astype(np.float32)  # subnormal fp16 d

    blocks_ref = R.quantize_ref_rule(W)
    blocks_llama = R.quantize_llama_rule(W)

    braw = rng.integers(0, 256, (6, 29, 18), dtype=np.uint8)
    d = (rng.standard_normal((6, 29)) * 0.05).astype(np.float16)
    d.reshape(-1)[:4] = np.array([0.0, -0.0, 6e-8, -65504.0], np.float16)
    braw[:, :, 0:2] = d.view(np.uint8).reshape(6, 29, 2)

    X = rng.standard_normal((5, K)).astype(np.float16)
    return dict(
        W=W, blocks_ref=blocks_ref, blocks_llama=blocks_llama,
        blocks_raw=braw,
        deq_raw_f32=R.dequantize(braw, np.float32),
        deq_raw_f16=R.dequantize(braw, np.float16),
        X=X,
        Y_ref_f64=R.matmul_f64(X, blocks_ref),
        Y_llama_f64=R.matmul_f64(X, blocks_llama),
    )


if __name__ == "__main__":
    out = os.path.join(HERE, "q4_0_golden.npz")
    np.savez_compressed(out, **build())
    print("wrote", out, os.path.getsize(out), "bytes")
