"""Committed golden fixtures (tests/golden/q4_0_golden.npz) vs the oracle (CPU)
and vs the HIP kernels (GPU)."""
import os

import numpy as np
import pytest

from oracle import c_oracle as C
from oracle import q4_0_ref as R

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "q4_0_golden.npz"))


def test_oracle_reproduces_golden():
    np.testing.assert_array_equal(R.quantize_ref_rule(G["W"]), G["blocks_ref"])
    np.testing.assert_array_equal(C.quantize_ref_rule(G["W"]), G["blocks_ref"])
    np.testing.assert_array_equal(R.quantize_llama_rule(G["W"]), G["blocks_llama"])
    np.testing.assert_array_equal(C.quantize_llama_rule(G["W"]), G["blocks_llama"])
    np.testing.assert_array_equal(R.dequantize(G["blocks_raw"], np.float32).view(np.uint32),
                                  G["deq_raw_f32"].view(np.uint32))
    np.testing.assert_array_equal(C.dequantize(G["blocks_raw"], np.float16).view(np.uint16),
                                  G["deq_raw_f16"].view(np.uint16))
    np.testing.assert_allclose(C.matmul_f64(G["X"], G["blocks_ref"]), G["Y_ref_f64"], rtol=1e-12, atol=1e-15)


def test_golden_known_answers():
    q, d = R.unpack_nibbles(G["blocks_ref"])
    assert list(G["blocks_ref"][0, 0]) == [0x00, 0x3C] + [0x88] * 16
    assert list(q[1, 1, :8]) == [15, 8, 10, 8, 6, 10, 6, 14]
    assert q[2, 2, 17] == 1 and (np.delete(q[2, 2], 17) == 8).all()
    assert d[3, 3] != 0 and abs(float(d[3, 3])) < 6.2e-5       # subnormal fp16 scale


@pytest.mark.gpu
def test_kernels_reproduce_golden(dev):
    import torch

    import metalops_amd as mo
    W = torch.from_numpy(G["W"]).to(dev)
    np.testing.assert_array_equal(mo.quantize_ggml_q4_0(W).cpu().numpy(), G["blocks_ref"])
    np.testing.assert_array_equal(mo.quantize_ggml_q4_0_llama(W).cpu().numpy(), G["blocks_llama"])
    braw = torch.from_numpy(G["blocks_raw"]).to(dev)
    np.testing.assert_array_equal(mo.dequantize_ggml_q4_0(braw, torch.float32).cpu().numpy().view(np.uint32),
                                  G["deq_raw_f32"].view(np.uint32))
    np.testing.assert_array_equal(mo.dequantize_ggml_q4_0(braw).cpu().numpy().view(np.uint16),
                                  G["deq_raw_f16"].view(np.uint16))
    X = torch.from_numpy(G["X"]).to(dev)
    for key, yk in (("blocks_ref", "Y_ref_f64"), ("blocks_llama", "Y_llama_f64")):
        Y = mo.matmul_ggml_q4_0(X, torch.from_numpy(G[key]).to(dev)).float().cpu().numpy()
        Yr = G[yk]
        assert (np.abs(Y - Yr).max(axis=1) <= 1e-2 * np.abs(Yr).max(axis=1)).all()
