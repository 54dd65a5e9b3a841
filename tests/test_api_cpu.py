"""Host-side behaviour of the Python drop-in (no GPU needed).

Mirrors the reference's checks (quantization.py:329, :443): AssertionError with
the same message for K mismatches, checked before anything touches a device.
The product path has no CPU fallback: CPU tensors are rejected loudly.
"""
import pytest
import torch

import metalops_amd as mo


def test_exports_match_reference_names():
    for name in ("quantize_ggml_q4_0", "dequantize_ggml_q4_0", "matmul_ggml_q4_0"):
        assert callable(getattr(mo, name))
    assert mo.QK4_0 == 32 and mo.BLOCK_Q4_0_SIZE == 18


def test_matmul_k_mismatch_assertion():
    blocks = torch.zeros(4, 8, 18, dtype=torch.uint8)
    with pytest.raises(AssertionError, match=r"X K dim \(96\) must match weight K \(128\)"):
        mo.matmul_ggml_q4_0(torch.zeros(2, 96, dtype=torch.float16), blocks)


def test_quantize_k_assertion():
    with pytest.raises(AssertionError, match=r"K \(33\) must be divisible by 32"):
        mo.quantize_ggml_q4_0(torch.zeros(33, 4))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_cpu_tensors_rejected_no_fallback():
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mo.matmul_ggml_q4_0(torch.zeros(2, 64, dtype=torch.float16), torch.zeros(2, 8, 18, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mo.quantize_ggml_q4_0(torch.zeros(64, 4))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mo.dequantize_ggml_q4_0(torch.zeros(2, 8, 18, dtype=torch.uint8))


def test_int4_exports_match_reference_names():
    for name in ("quantize_int4", "dequantize_int4", "matmul_int4", "matmul_int4_silu",
                 "matmul_int4_gelu"):
        assert callable(getattr(mo, name))
    lin = mo.Int4Linear(64, 16, group_size=32)
    assert tuple(lin.weight_packed.shape) == (32, 16) and lin.weight_packed.dtype == torch.uint8
    assert tuple(lin.scales.shape) == (2, 16) and lin.scales.dtype == torch.float32
    assert lin.bias is not None and "mode=int4_kernel" in lin.extra_repr()
    assert mo.Int4Linear(64, 16, bias=False).bias is None


def test_int4_odd_k_rejected():
    with pytest.raises(IndexError):
        mo.quantize_int4(torch.zeros(33, 4))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_int4_cpu_tensors_rejected_no_fallback():
    W = torch.zeros(32, 8, dtype=torch.uint8)
    s = torch.ones(1, 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mo.quantize_int4(torch.zeros(64, 8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mo.dequantize_int4(W, s, s)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mo.matmul_int4(torch.zeros(2, 64, dtype=torch.float16), W, s, s)
