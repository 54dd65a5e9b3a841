"""The allocation-free entry point mcq4_matmul_q4_0_f16_noalloc (library-owned
scratch, no caller workspace) against mcq4_matmul_q4_0_f16 with a caller
workspace, both called through the C ABI: identical bits on two calls in a row,
the second with a smaller input, on shapes that use the split-K workspace."""
import ctypes

import pytest
import torch

from oracle import q4_0_ref as ref

pytestmark = pytest.mark.gpu


def _run_pair(dev, M, K, N, seed):
    from metalops_amd import _lib
    L = _lib.lib
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(K, N, generator=g) * 0.02
    X = torch.randn(M, K, generator=g).half().to(dev)
    b = torch.from_numpy(ref.quantize_llama_rule(W.numpy())).to(dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    need = int(L.mcq4_matmul_workspace_bytes(M, K, N))
    assert need <= int(L.mcq4_matmul_noalloc_max_workspace_bytes())
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)
    Y_ref = torch.empty(M, N, dtype=torch.float16, device=dev)
    Y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    _lib.check(L.mcq4_matmul_q4_0_f16(X.data_ptr(), K, b.data_ptr(), Y_ref.data_ptr(), N, M, K, N,
                                      ws.data_ptr() if need else None, need, stream), "workspace call")
    _lib.check(L.mcq4_matmul_q4_0_f16_noalloc(X.data_ptr(), K, b.data_ptr(), Y.data_ptr(), N, M, K, N, stream),
               "noalloc call")
    torch.cuda.synchronize(dev)
    assert torch.equal(Y.view(torch.int16), Y_ref.view(torch.int16)), f"M={M} K={K} N={N}"
    return need


@pytest.mark.parametrize("first,second", [
    ((200, 11008, 1024), (16, 14336, 4096)),      # prefill split-K (16 MiB) then decode split-K (span split form)
    ((16, 14336, 4096), (8, 4096, 1040)),         # decode split-K then a smaller decode
    ((128, 11008, 1024), (130, 1024, 384)),       # prefill split-K then a small prefill
])
def test_noalloc_matches_workspace_entry(dev, monkeypatch, first, second):
    from metalops_amd import _lib
    for k in ("MCQ4_GEMVM_SPLIT", "MCQ4_GEMM6_SPLIT", "MCQ4_GEMM_PATH", "MCQ4_XCD_LOCAL", "MCQ4_SPLIT_FOREIGN",
              "MCQ4_GEMV_SPAN"):
        monkeypatch.delenv(k, raising=False)
    print(f"noalloc {first} then {second}", flush=True)
    assert _run_pair(dev, *first, seed=1) > 0        # the first call uses the scratch workspace
    _run_pair(dev, *second, seed=2)
    # the decode shape at M=8 uses a split only when forced
    monkeypatch.setenv("MCQ4_GEMVM_SPLIT", "4")
    assert _run_pair(dev, 8, 4096, 1040, seed=3) > 0


def test_noalloc_rejects_oversized_and_bad_args(dev):
    from metalops_amd import _lib
    L = _lib.lib
    cap = int(L.mcq4_matmul_noalloc_max_workspace_bytes())
    assert cap == 256 * 1024 + 16 * 1024 * 1024
    # a plan whose split-K workspace exceeds the scratch is refused with a clear error
    big = (2048, 14336, 4096)
    assert int(L.mcq4_matmul_workspace_bytes(*big)) > cap
    xb = torch.zeros(1, 16, dtype=torch.float16, device=dev)
    assert L.mcq4_matmul_q4_0_f16_noalloc(xb.data_ptr(), 14336, xb.data_ptr(), xb.data_ptr(), 4096,
                                          *big, None) == _lib.MCQ4_ERR_WORKSPACE
    assert b"allocation-free" in L.mcq4_last_error()
    # argument errors are reported as by the workspace entry point
    assert L.mcq4_matmul_q4_0_f16_noalloc(None, 32, None, None, 8, 1, 32, 8, None) == _lib.MCQ4_ERR_INVALID_ARG
    x = torch.zeros(1, 48, dtype=torch.float16, device=dev)
    assert L.mcq4_matmul_q4_0_f16_noalloc(x.data_ptr(), 48, x.data_ptr(), x.data_ptr(), 8, 1, 48, 8,
                                          None) == _lib.MCQ4_ERR_SHAPE
