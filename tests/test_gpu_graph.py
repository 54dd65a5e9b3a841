"""HIP-graph capture and replay of the matmul entry points.

The kernels allocate nothing, record no memset, and leave their split-K
counters at zero, so a captured call must give the eager result on every
replay -- including replays with other (eager) work and synchronisations in
between, and split-K shapes whose counters are reused across replays.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mo(dev):
    import metalops_amd
    return metalops_amd


def _replay_check(dev, fn, out_ref, reps=4):
    s = torch.cuda.Stream(dev)
    with torch.cuda.stream(s):
        fn()                     # warm-up: per-stream workspace allocated before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = fn()
    for r in range(reps):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.float().cpu().numpy(), out_ref, err_msg=f"replay {r}")
        # unrelated eager work between replays
        (torch.randn(1024, 1024, device=dev) @ torch.randn(1024, 1024, device=dev)).sum().item()


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (1, 4096, 128256 // 16), (8, 4096, 2048),
                                   (16, 14336, 4096), (128, 4096, 1024), (512, 11008, 512), (384, 4096, 4096),
                                   (512, 11008, 4096), (1024, 4096, 4096), (2048, 4096, 14336), (2048, 14336, 4096)])
def test_q4_0_graph_replay(mo, dev, M, K, N):
    g = torch.Generator(device=dev).manual_seed(M + N)
    W = torch.randn(K, N, generator=g, device=dev) * 0.02
    blocks = mo.quantize_ggml_q4_0_llama(W)
    X = torch.randn(M, K, generator=g, device=dev).half()
    ref = mo.matmul_ggml_q4_0(X, blocks).float().cpu().numpy()
    _replay_check(dev, lambda: mo.matmul_ggml_q4_0(X, blocks), ref)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (16, 14336, 512), (1, 16384, 1024),
                                   (256, 4096, 1024), (128, 4096, 512)])
def test_int4_graph_replay(mo, dev, M, K, N):
    g = torch.Generator(device=dev).manual_seed(M + N)
    W = (torch.randn(K, N, generator=g, device=dev) * 0.02).half()
    gs = 32 if K == 16384 else 128          # K = 16384 with group 32 forces a decode K split
    packed, s, z = mo.quantize_int4(W, gs)
    X = torch.randn(M, K, generator=g, device=dev).half()
    ref = mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy()
    _replay_check(dev, lambda: mo.matmul_int4(X, packed, s, z, gs), ref)


def test_q4_0_grouped_graph_replay(mo, dev):
    """Gate and up in one launch, captured: every replay equals the eager call."""
    g = torch.Generator(device=dev).manual_seed(5)
    K, N = 4096, 11008
    blocks = [mo.quantize_ggml_q4_0_llama(torch.randn(K, N, generator=g, device=dev) * 0.02) for _ in range(2)]
    X = torch.randn(1, K, generator=g, device=dev).half()
    refs = [y.float().cpu().numpy() for y in mo.matmul_ggml_q4_0_grouped(X, blocks)]
    ref = np.concatenate(refs, axis=1)
    _replay_check(dev, lambda: torch.cat(mo.matmul_ggml_q4_0_grouped(X, blocks), dim=1), ref)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (1, 11008, 4096), (4, 4096, 1024)])
def test_fused_rmsnorm_graph_replay(mo, dev, M, K, N):
    """The fused RMSNorm + INT4 linear (one launch at M = 1, two kernels above),
    captured: every replay equals the eager call."""
    g = torch.Generator(device=dev).manual_seed(M + K)
    W = (torch.randn(K, N, generator=g, device=dev) * 0.02).half()
    packed, s, z = mo.quantize_int4(W, 128)
    X = (torch.randn(M, K, generator=g, device=dev) * 2).half()
    wn = (1 + 0.1 * torch.randn(K, generator=g, device=dev)).half()
    ref = mo.fused_rmsnorm_linear_int4(X, wn, packed, s, z, 1e-5, 128).float().cpu().numpy()
    _replay_check(dev, lambda: mo.fused_rmsnorm_linear_int4(X, wn, packed, s, z, 1e-5, 128), ref)
