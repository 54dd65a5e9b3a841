"""The PyTorch-ROCm extension binding (metalops_amd/csrc/torch_ext/mcq4_torch.cpp),
which mirrors metalcore's matmul_ggml_q4_0_metal (native/core_mps.mm:5917-5975,
registered at :6938).  CPU: it loads and exports the binding, and rejects CPU
tensors with RuntimeError (TORCH_CHECK).  GPU: its results equal the C-ABI path
bit for bit and meet the oracle's tolerance."""
import numpy as np
import pytest
import torch

from oracle import q4_0_ref as ref


def test_extension_loads_and_checks():
    from metalops_amd import torch_ext
    assert callable(torch_ext.matmul_ggml_q4_0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        torch_ext.matmul_ggml_q4_0(torch.zeros(1, 32, dtype=torch.float16),
                                   torch.zeros(1, 8, 18, dtype=torch.uint8))


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (7, 1024, 520), (300, 2048, 1024), (2048, 4096, 512)])
def test_extension_matmul_vs_oracle(dev, M, K, N):
    import metalops_amd as mo
    from metalops_amd import torch_ext
    g = torch.Generator().manual_seed(M + K + N)
    W = torch.randn(K, N, generator=g) * 0.02
    X = torch.randn(M, K, generator=g).half()
    blocks = ref.quantize_llama_rule(W.numpy())
    b = torch.from_numpy(blocks).to(dev)
    Y = torch_ext.matmul_ggml_q4_0(X.to(dev), b)
    assert Y.dtype == torch.float16 and Y.shape == (M, N)
    assert torch.equal(Y, mo.matmul_ggml_q4_0(X.to(dev), b))
    Yr = ref.matmul_f32(X.numpy(), blocks)
    Yg = Y.float().cpu().numpy()
    assert np.isfinite(Yg).all()
    assert (np.abs(Yg - Yr).max(axis=1) <= 1e-2 * np.abs(Yr).max(axis=1)).all()
    with pytest.raises(RuntimeError, match="float16"):
        torch_ext.matmul_ggml_q4_0(X.float().to(dev), b)
    with pytest.raises(RuntimeError, match="K dimension"):
        torch_ext.matmul_ggml_q4_0(X[:, :K - 32].contiguous().to(dev), b)
