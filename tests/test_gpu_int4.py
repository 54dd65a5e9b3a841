"""GPU parity tests of the per-group INT4 path against the CPU oracle (oracle/int4_ref.py).

* quantize / dequantize: bit-exact (packed bytes, scales, zeros, outputs) for
  fp32 / fp16 / bf16, group sizes 128, 64, 32, 33 and 3, partial last groups;
* matmul (every kernel: decode GEMV M <= 16, prefill GEMM, general kernel; fp16,
  bf16 and fp32 activations; fp32 / fp16 / bf16 scales): per output row
  max|Y - Y_ref| <= 1e-2 * max|Y_ref[m, :]| against X.float() @ dequant_f32(W)
  (the tolerance of the fp16 matmul path; the dequant itself is pinned exactly);
* fused SiLU / GELU stores, 3-D activations, repeated split-K calls, Int4Linear.
"""
import os

import numpy as np
import pytest
import torch

from oracle import int4_ref as R

pytestmark = pytest.mark.gpu

TDT = {R.F32: torch.float32, R.F16: torch.float16, R.BF16: torch.bfloat16}


@pytest.fixture(scope="module")
def mo(dev):
    import metalops_amd
    return metalops_amd


def _weights(K, N, seed, dtype=R.F32):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(K, N, generator=g) * 0.02
    idx = torch.randperm(K * N, generator=g)[: max(1, K * N // 100)]
    w.view(-1)[idx] = torch.randn(idx.numel(), generator=g) * 0.2
    return R.round_to(w.numpy(), dtype)


def _quant(mo, dev, K, N, gs, dtype=R.F32, seed=0):
    w = _weights(K, N, seed, dtype)
    wt = torch.from_numpy(w).to(TDT[dtype]).to(dev)
    packed, s, z = mo.quantize_int4(wt, gs)
    return w, packed, s, z


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(a, b) or np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- quantize / dequantize ----------------------------------------------------

@pytest.mark.parametrize("dtype", [R.F32, R.F16, R.BF16])
@pytest.mark.parametrize("K,N,gs", [(256, 96, 128), (96, 40, 64), (24, 10, 3), (66, 9, 33),
                                    (4096, 512, 128)])
def test_quantize_bit_exact(mo, dev, dtype, K, N, gs):
    print(f"quantize {dtype} K={K} N={N} gs={gs}", flush=True)
    w, packed, s, z = _quant(mo, dev, K, N, gs, dtype, seed=K + N)
    rp, rs, rz = R.quantize(w, gs, dtype)
    assert s.dtype == TDT[dtype] and z.dtype == TDT[dtype]
    np.testing.assert_array_equal(packed.cpu().numpy(), rp)
    assert _bits_equal(s.float().cpu().numpy(), rs)
    assert _bits_equal(z.float().cpu().numpy(), rz)


def test_quantize_strided_input(mo, dev):
    w = _weights(128, 80, 5)
    big = torch.zeros(128, 96, device=dev)
    big[:, :80] = torch.from_numpy(w).to(dev)
    packed, s, z = mo.quantize_int4(big[:, :80], 64)
    rp, rs, rz = R.quantize(w, 64)
    np.testing.assert_array_equal(packed.cpu().numpy(), rp)
    assert _bits_equal(s.cpu().numpy(), rs) and _bits_equal(z.cpu().numpy(), rz)


@pytest.mark.parametrize("sz", [R.F32, R.F16, R.BF16])
@pytest.mark.parametrize("out", [torch.float32, torch.float16, torch.bfloat16])
def test_dequant_bit_exact(mo, dev, sz, out):
    K, N, gs = 192, 72, 64
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=3)
    got = mo.dequantize_int4(packed, s, z, gs, out)
    assert got.dtype == out and tuple(got.shape) == (K, N)
    name = {torch.float32: R.F32, torch.float16: R.F16, torch.bfloat16: R.BF16}[out]
    want = R.dequantize(packed.cpu().numpy(), s.float().cpu().numpy(), z.float().cpu().numpy(),
                        gs, name)
    assert _bits_equal(got.float().cpu().numpy(), want)
    # default dtype is fp16 (quantization.py:137-138)
    assert mo.dequantize_int4(packed, s, z, gs).dtype == torch.float16


def test_dequant_handmade_codes(mo, dev):
    """Every code 0..15 in both nibbles against chosen scales/zeros."""
    K, N, gs = 32, 16, 16
    q = np.array([[(k + 3 * n) % 16 for n in range(N)] for k in range(K)], np.uint8)
    packed = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    rng = np.random.default_rng(0)
    s = rng.normal(0, 1, (2, N)).astype(np.float32)
    z = rng.uniform(-2, 17, (2, N)).astype(np.float32)
    got = mo.dequantize_int4(torch.from_numpy(packed).to(dev), torch.from_numpy(s).to(dev),
                             torch.from_numpy(z).to(dev), gs, torch.float32)
    assert _bits_equal(got.cpu().numpy(), R.dequantize(packed, s, z, gs, R.F32))


# ---- matmul -------------------------------------------------------------------

def _check_rows(Y, Yref, tol=1e-2):
    Y = np.asarray(Y, np.float64)
    Yref = np.asarray(Yref, np.float64)
    assert np.all(np.isfinite(Y))
    scale = np.maximum(np.abs(Yref).max(axis=-1, keepdims=True), 1e-6)
    err = np.abs(Y - Yref) / scale
    assert err.max() <= tol, f"max row-relative error {err.max():.3e}"


def _ref(X, packed, s, z, gs):
    return R.matmul_f32(X.float().cpu().numpy(), packed.cpu().numpy(), s.float().cpu().numpy(),
                        z.float().cpu().numpy(), gs)


@pytest.fixture
def i4_path():
    old = os.environ.get("MCQ4_I4_PATH")

    def set_path(v):
        if v is None:
            os.environ.pop("MCQ4_I4_PATH", None)
        else:
            os.environ["MCQ4_I4_PATH"] = v
    yield set_path
    set_path(old)


MM_CASES = [
    # (M, K, N, gs): decode GEMV shapes (M <= 16)
    (1, 4096, 4096, 128), (1, 256, 136, 128), (2, 512, 256, 64), (5, 1024, 392, 32),
    (16, 2048, 1024, 128), (8, 96, 24, 64), (3, 4096, 11008, 128), (1, 14336, 512, 128),
    (1, 512, 2176, 256), (2, 512, 2004, 128),
    # prefill GEMM shapes (M > 16, N % 128 == 0)
    (17, 512, 256, 128), (64, 1024, 512, 64), (128, 4096, 1024, 128), (300, 2048, 768, 32),
    (512, 1024, 2048, 128), (33, 96, 128, 64),
    # group sizes of 3 and 5 K steps (the scale group index by multiply-high)
    (300, 1920, 768, 96), (129, 2080, 1024, 160),
    # general kernel (N % 128 != 0 with M > 16; N % 8 != 0)
    (40, 256, 200, 128), (3, 128, 21, 64),
]


@pytest.mark.parametrize("M,K,N,gs", MM_CASES)
@pytest.mark.parametrize("sz", [R.F32, R.F16])
def test_matmul_fp16(mo, dev, M, K, N, gs, sz):
    print(f"matmul_int4 fp16 M={M} K={K} N={N} gs={gs} sz={sz}", flush=True)
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=M + K + N)
    X = (torch.randn(M, K, generator=torch.Generator().manual_seed(M)) ).half().to(dev)
    Y = mo.matmul_int4(X, packed, s, z, gs)
    assert Y.dtype == torch.float16 and tuple(Y.shape) == (M, N)
    _check_rows(Y.float().cpu().numpy(), _ref(X, packed, s, z, gs))


@pytest.mark.parametrize("M,K,N,gs", [(1, 1024, 512, 128), (16, 512, 256, 64), (130, 512, 384, 128)])
def test_matmul_bf16_scales(mo, dev, M, K, N, gs):
    w, packed, s, z = _quant(mo, dev, K, N, gs, R.BF16, seed=11)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(1)).half().to(dev)
    Y = mo.matmul_int4(X, packed, s, z, gs)
    _check_rows(Y.float().cpu().numpy(), _ref(X, packed, s, z, gs))


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,K,N,gs", [(1, 4096, 512, 128), (8, 512, 100, 64), (128, 1024, 256, 128)])
def test_matmul_other_activation_dtypes(mo, dev, xdt, M, K, N, gs):
    """fp32 / bf16 activations run the general kernel; result in X.dtype."""
    w, packed, s, z = _quant(mo, dev, K, N, gs, R.F32, seed=2)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(4)).to(xdt).to(dev)
    Y = mo.matmul_int4(X, packed, s, z, gs)
    assert Y.dtype == xdt
    Yref = _ref(X, packed, s, z, gs)
    _check_rows(Y.float().cpu().numpy(), Yref, tol=1e-2)
    if xdt == torch.float32:
        # fp32 activations with fp32 weights: much tighter than the fp16 bar
        _check_rows(Y.cpu().numpy(), Yref, tol=1e-4)


@pytest.mark.parametrize("M,K,N,gs", [(1, 1024, 512, 128), (12, 512, 256, 64), (200, 1024, 512, 128)])
def test_matmul_kernels_agree_with_general(mo, dev, i4_path, M, K, N, gs):
    """The MFMA kernels and the general kernel agree within the same tolerance."""
    w, packed, s, z = _quant(mo, dev, K, N, gs, R.F32, seed=9)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(5)).half().to(dev)
    Y_fast = mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy()
    i4_path("generic")
    Y_gen = mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy()
    _check_rows(Y_fast, Y_gen)


def test_matmul_batched_and_strided(mo, dev):
    K, N, gs = 512, 256, 128
    w, packed, s, z = _quant(mo, dev, K, N, gs)
    X3 = torch.randn(3, 5, K, generator=torch.Generator().manual_seed(6)).half().to(dev)
    Y3 = mo.matmul_int4(X3, packed, s, z, gs)
    assert tuple(Y3.shape) == (3, 5, N)
    _check_rows(Y3.reshape(15, N).float().cpu().numpy(), _ref(X3.reshape(15, K), packed, s, z, gs))
    Xbig = torch.randn(40, K + 8, generator=torch.Generator().manual_seed(7)).half().to(dev)
    Xv = Xbig[:, 3:3 + K]                       # misaligned view: copied to a dense buffer
    _check_rows(mo.matmul_int4(Xv, packed, s, z, gs).float().cpu().numpy(),
                _ref(Xv, packed, s, z, gs))


def test_split_k_repeat_and_interleave(mo, dev):
    """Split-K counters are left at zero: repeated and interleaved shapes stay correct."""
    cases = [(1, 4096, 4096, 128), (16, 14336, 512, 128), (128, 4096, 512, 128)]
    data = []
    for i, (M, K, N, gs) in enumerate(cases):
        w, packed, s, z = _quant(mo, dev, K, N, gs, seed=20 + i)
        X = torch.randn(M, K, generator=torch.Generator().manual_seed(i)).half().to(dev)
        data.append((X, packed, s, z, gs, _ref(X, packed, s, z, gs)))
    for rep in range(3):
        for X, packed, s, z, gs, Yref in data:
            _check_rows(mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy(), Yref)


@pytest.mark.parametrize("wb,M,K,N,gs", [(4, 1, 4096, 4096, 128), (4, 4, 4096, 1040, 64), (4, 16, 14336, 512, 128),
                                         (4, 9, 2048, 4112, 32), (8, 1, 4096, 4096, 128), (8, 8, 11008, 200, 128)])
def test_xcd_local_exchange(mo, dev, monkeypatch, wb, M, K, N, gs):
    """The split-K GEMV's XCD-local exchange (default) and the agent-scope one sum
    the same partials in the same order: identical bits, and both match the oracle.
    Tile counts that are not a multiple of 8 exercise the padded grid."""
    print(f"xcd-local wb={wb} M={M} K={K} N={N} gs={gs}", flush=True)
    for k in ("MCQ4_I4_SPW1", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("MCQ4_I4_GEMV1", "0")         # the register-ring GEMV for M == 1 too
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(K + M)).half()
    if wb == 4:
        w, packed, s, z = _quant(mo, dev, K, N, gs, seed=K + N)
        fn = lambda: mo.matmul_int4(X.to(dev), packed, s, z, gs)
        Yref = _ref(X.to(dev), packed, s, z, gs)
    else:
        q, s8, z8 = _int8_weights(K, N, gs, R.F16, K + N)
        args = [torch.from_numpy(a).to(dev) for a in (q, s8.astype(np.float16), z8.astype(np.float16))]
        fn = lambda: mo.matmul_int8(X.to(dev), *args, gs)
        Yref = R.matmul_int8_f32(X.float().numpy(), q, s8, z8, gs)
    Y = fn()
    Y2 = fn()
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    Y0 = fn()
    _check_rows(Y.float().cpu().numpy(), Yref)
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))
    assert torch.equal(Y.view(torch.int16), Y0.view(torch.int16))


@pytest.mark.parametrize("M,K,N,act", [(2048, 14336, 4096, None), (1300, 2048, 5120, None),
                                       (1024, 2048, 6144, "silu")])
def test_gemm6_split2_exchange_matches_reduce(mo, dev, monkeypatch, M, K, N, act):
    """i4_gemm6 with two K splits: the in-kernel XCD-local sum (default) and the
    reduction kernel both compute act(p0 + p1): identical bits, and the oracle agrees."""
    print(f"i4_gemm6 split2 exchange M={M} K={K} N={N} act={act}", flush=True)
    for k in ("MCQ4_I4_GEMM6", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("MCQ4_I4_GEMM7", "0")      # the shapes that i4_gemm7 would take
    gs = 128
    w, packed, s, z = _quant(mo, dev, K, N, gs, seed=M + N)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half().to(dev)
    fn = (lambda: mo.matmul_int4_silu(X, packed, s, z, gs)) if act else (lambda: mo.matmul_int4(X, packed, s, z, gs))
    Y = fn()
    Y2 = fn()
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    Y0 = fn()
    assert torch.isfinite(Y.float()).all()
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))
    assert torch.equal(Y.view(torch.int16), Y0.view(torch.int16))
    if M * K * N <= 2048 * 2048 * 6144:
        base = _ref(X, packed, s, z, gs)
        if act:
            base = _silu(base.astype(np.float64))
        _check_rows(Y.float().cpu().numpy(), base)


# i4_gemm7 (256 x 256 tiles): grids of 160+ tiles, or 96+ with K >= 8192 (two
# K splits summed by the reduction kernel); ragged M, N % 256 == 128 (waves past
# N), group sizes 32..128, bf16 scales, fused activations.
GEMM7_CASES = [
    (2048, 512, 6144, 128, R.F16, None), (1800, 1024, 6400, 64, R.F16, None),
    (2048, 8192, 3200, 128, R.F16, None), (2048, 512, 6144, 32, R.BF16, None),
    (1793, 8448, 3072, 128, R.BF16, "silu"), (2048, 512, 6144, 128, R.F16, "gelu"),
]


@pytest.mark.parametrize("M,K,N,gs,sz,act", GEMM7_CASES)
def test_gemm7(mo, dev, monkeypatch, M, K, N, gs, sz, act):
    print(f"i4_gemm7 M={M} K={K} N={N} gs={gs} sz={sz} act={act}", flush=True)
    for k in ("MCQ4_I4_GEMM6", "MCQ4_I4_GEMM7", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=M + K)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half().to(dev)
    f = {None: mo.matmul_int4, "silu": mo.matmul_int4_silu, "gelu": mo.matmul_int4_gelu}[act]
    Y = f(X, packed, s, z, gs)
    Y2 = f(X, packed, s, z, gs)
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))
    base = _ref(X, packed, s, z, gs)
    if act == "silu":
        base = _silu(base.astype(np.float64))
    elif act == "gelu":
        base = _gelu_tanh(base.astype(np.float64))
    _check_rows(Y.float().cpu().numpy(), base)
    # the 128 x 256-tile kernel agrees within the same bar
    monkeypatch.setenv("MCQ4_I4_GEMM7", "0")
    Y6 = f(X, packed, s, z, gs)
    _check_rows(Y6.float().cpu().numpy(), base)


@pytest.mark.parametrize("M,K,N,gs", [(300, 1024, 768, 128), (129, 2048, 2560, 64), (1024, 4096, 2816, 128),
                                      (300, 1920, 768, 96), (257, 2080, 1280, 160)])
def test_gemm7_forced(mo, dev, monkeypatch, M, K, N, gs):
    """i4_gemm7 taken below its grid rule (MCQ4_I4_GEMM7=1): ragged M, a handful
    of tiles, N % 256 == 0 and == 128 (waves past N)."""
    print(f"i4_gemm7 forced M={M} K={K} N={N} gs={gs}", flush=True)
    for k in ("MCQ4_I4_GEMM6", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("MCQ4_I4_GEMM7", "1")
    w, packed, s, z = _quant(mo, dev, K, N, gs, R.F16, seed=M + N)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M + 1)).half().to(dev)
    Y = mo.matmul_int4(X, packed, s, z, gs)
    _check_rows(Y.float().cpu().numpy(), _ref(X, packed, s, z, gs))


def _silu(y):
    return y / (1.0 + np.exp(-y))


def _gelu_tanh(y):
    return 0.5 * y * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (y + 0.044715 * y ** 3)))


@pytest.mark.parametrize("M,K,N,gs", [(1, 1024, 512, 128), (16, 512, 256, 64), (256, 1024, 512, 128),
                                      (40, 256, 200, 128)])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_fused_activation(mo, dev, M, K, N, gs, act):
    w, packed, s, z = _quant(mo, dev, K, N, gs, seed=31)
    X = (torch.randn(M, K, generator=torch.Generator().manual_seed(8)) * 4).half().to(dev)
    fn = mo.matmul_int4_silu if act == "silu" else mo.matmul_int4_gelu
    Y = fn(X, packed, s, z, gs)
    base = _ref(X, packed, s, z, gs).astype(np.float64)
    want = _silu(base) if act == "silu" else _gelu_tanh(base)
    Y = Y.float().cpu().numpy().astype(np.float64)
    scale = np.maximum(np.abs(base).max(axis=-1, keepdims=True), 1e-6)
    assert (np.abs(Y - want) / scale).max() <= 1e-2


def test_fused_requires_half(mo, dev):
    w, packed, s, z = _quant(mo, dev, 64, 16, 32)
    with pytest.raises(RuntimeError, match="half precision"):
        mo.matmul_int4_silu(torch.zeros(2, 64, device=dev), packed, s, z, 32)


@pytest.mark.parametrize("dequant_on_load", [True, False])
def test_int4_linear(mo, dev, dequant_on_load):
    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 256).to(dev)
    q = mo.Int4Linear.from_float(lin, group_size=128, dequant_on_load=dequant_on_load)
    assert q.scales.dtype == torch.float32 and tuple(q.weight_packed.shape) == (256, 256)
    x = torch.randn(4, 7, 512, device=dev)
    y = q(x)
    assert y.dtype == torch.float32 and tuple(y.shape) == (4, 7, 256)
    ref = _ref(x.reshape(28, 512).half() if dequant_on_load else x.reshape(28, 512),
               q.weight_packed, q.scales, q.zeros, 128) + lin.bias.detach().cpu().numpy()
    _check_rows(y.reshape(28, 256).detach().cpu().numpy(), ref)
    q.keep_quantized()
    assert "int4_kernel" in q.extra_repr()
    y2 = q(x.half())
    assert y2.dtype == torch.float32      # fp16 product + fp32 bias buffer promotes (reference :604-605)
    _check_rows(y2.reshape(28, 256).float().detach().cpu().numpy(), ref)
    q.dequantize()
    assert "fast_fp16" in q.extra_repr()


@pytest.mark.parametrize("M,K,N,gs,sz", [(1, 4096, 4096, 128, R.F16), (4, 1024, 768, 64, R.F32),
                                         (16, 2048, 512, 128, R.F16), (64, 512, 256, 128, R.F16),
                                         (300, 1024, 512, 32, R.F32), (3, 256, 200, 128, R.F16)])
def test_fused_rmsnorm_linear_int4(mo, dev, M, K, N, gs, sz):
    """Y = matmul_int4(rmsnorm(X, w, eps)) against the oracle's fp16 X_norm and matmul."""
    print(f"fused rmsnorm+int4 M={M} K={K} N={N} gs={gs} sz={sz}", flush=True)
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=40 + M)
    g = torch.Generator().manual_seed(M)
    X = (torch.randn(M, K, generator=g) * 3).half()
    wn = (1 + 0.1 * torch.randn(K, generator=g)).half()
    Y = mo.fused_rmsnorm_linear_int4(X.to(dev), wn.to(dev), packed, s, z, 1e-5, gs)
    assert Y.dtype == torch.float16 and tuple(Y.shape) == (M, N)
    xn = R.rmsnorm_f16(X.numpy(), wn.numpy(), 1e-5)
    Yref = R.matmul_f32(xn.astype(np.float32), packed.cpu().numpy(), s.float().cpu().numpy(),
                        z.float().cpu().numpy(), gs)
    _check_rows(Y.float().cpu().numpy(), Yref)
    # the plain matmul afterwards still sees a clean workspace (split-K counters)
    X2 = torch.randn(1, K, generator=g).half().to(dev)
    _check_rows(mo.matmul_int4(X2, packed, s, z, gs).float().cpu().numpy(), _ref(X2, packed, s, z, gs))


@pytest.mark.parametrize("K,N,gs,sz", [(4096, 4096, 128, R.F16), (11008, 4096, 128, R.BF16),
                                       (4096, 1408, 64, R.F32), (512, 256, 32, R.F16),
                                       (1024, 12288, 128, R.F16)])
def test_fused_rmsnorm_one_launch_matches_two(mo, dev, monkeypatch, K, N, gs, sz):
    """M = 1 normalises inside the GEMV; its bits equal the two-kernel path's
    (norm kernel, then matmul) on the same inputs, with the XCD-local and the
    agent-scope split exchange, and it stays within tolerance of the oracle."""
    print(f"fused rmsnorm one launch K={K} N={N} gs={gs} sz={sz}", flush=True)
    for k in ("MCQ4_I4_RMS_FUSE", "MCQ4_XCD_LOCAL", "MCQ4_I4_GEMV1", "MCQ4_I4_SPW1"):
        monkeypatch.delenv(k, raising=False)
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=K + N)
    g = torch.Generator().manual_seed(K + gs)
    X = (torch.randn(1, K, generator=g) * 3).half()
    wn = (1 + 0.1 * torch.randn(K, generator=g)).half()
    Xd, wnd = X.to(dev), wn.to(dev)
    Y1 = mo.fused_rmsnorm_linear_int4(Xd, wnd, packed, s, z, 1e-5, gs)
    monkeypatch.setenv("MCQ4_I4_RMS_FUSE", "0")
    Y2 = mo.fused_rmsnorm_linear_int4(Xd, wnd, packed, s, z, 1e-5, gs)
    assert torch.equal(Y1.view(torch.int16), Y2.view(torch.int16))
    monkeypatch.delenv("MCQ4_I4_RMS_FUSE")
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    Y3 = mo.fused_rmsnorm_linear_int4(Xd, wnd, packed, s, z, 1e-5, gs)
    assert torch.equal(Y1.view(torch.int16), Y3.view(torch.int16))
    monkeypatch.delenv("MCQ4_XCD_LOCAL")
    xn = R.rmsnorm_f16(X.numpy(), wn.numpy(), 1e-5)
    Yref = R.matmul_f32(xn.astype(np.float32), packed.cpu().numpy(), s.float().cpu().numpy(),
                        z.float().cpu().numpy(), gs)
    _check_rows(Y1.float().cpu().numpy(), Yref)
    assert torch.equal(mo.fused_rmsnorm_linear_int4(Xd, wnd, packed, s, z, 1e-5, gs).view(torch.int16),
                       Y1.view(torch.int16))


@pytest.mark.parametrize("M,K,N,gs", [(1, 4096, 1024, 128), (1, 250, 96, 50), (5, 250, 96, 50),
                                      (2, 11008, 512, 128)])
def test_fused_rmsnorm_unaligned_row(mo, dev, M, K, N, gs):
    """A row that is not 16-byte aligned takes the two-kernel path with scalar
    loads (and K % 8 != 0 a tail): the same sum order, so the same bits as the
    aligned call, and within tolerance of the oracle."""
    print(f"fused rmsnorm unaligned M={M} K={K} N={N} gs={gs}", flush=True)
    w, packed, s, z = _quant(mo, dev, K, N, gs, R.F16, seed=K + 7)
    g = torch.Generator().manual_seed(K + M)
    X = (torch.randn(M, K, generator=g) * 2).half()
    wn = (1 + 0.1 * torch.randn(K, generator=g)).half()
    Xa = X.to(dev)
    big = torch.zeros(M, K + 8, dtype=torch.float16, device=dev)
    big[:, 1:K + 1] = Xa
    Xu = big[:, 1:K + 1]
    assert Xu.data_ptr() % 16 != 0
    Ya = mo.fused_rmsnorm_linear_int4(Xa, wn.to(dev), packed, s, z, 1e-6, gs)
    Yu = mo.fused_rmsnorm_linear_int4(Xu, wn.to(dev), packed, s, z, 1e-6, gs)
    assert torch.equal(Ya.view(torch.int16), Yu.view(torch.int16))
    xn = R.rmsnorm_f16(X.numpy(), wn.numpy(), 1e-6)
    Yref = R.matmul_f32(xn.astype(np.float32), packed.cpu().numpy(), s.float().cpu().numpy(),
                        z.float().cpu().numpy(), gs)
    _check_rows(Ya.float().cpu().numpy(), Yref)


def test_fused_rmsnorm_requires_half(mo, dev):
    w, packed, s, z = _quant(mo, dev, 64, 16, 32)
    with pytest.raises(RuntimeError, match="half precision"):
        mo.fused_rmsnorm_linear_int4(torch.zeros(2, 64, device=dev), torch.ones(64, device=dev),
                                     packed, s, z, 1e-6, 32)


# ---- GPU-side quantize_to_int4 and INT8 matmul ----------------------------------

@pytest.mark.parametrize("K,N,gs", [(256, 96, 128), (96, 40, 64), (4096, 512, 128), (24, 10, 2)])
def test_quantize_to_int4_bit_exact(mo, dev, K, N, gs):
    w = _weights(K, N, K + 3 * N)
    packed, s, z = mo.quantize_to_int4(torch.from_numpy(w).to(dev), gs)
    rp, rs, rz = R.quantize(w, gs, R.F32, rounding="away")
    assert s.dtype == torch.float32
    np.testing.assert_array_equal(packed.cpu().numpy(), rp)
    assert _bits_equal(s.cpu().numpy(), rs) and _bits_equal(z.cpu().numpy(), rz)


def _int8_weights(K, N, gs, sz, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(-128, 128, (K, N)).astype(np.int8)
    G = (K + gs - 1) // gs
    s = R.round_to(rng.uniform(0.0005, 0.005, (G, N)).astype(np.float32), sz)
    z = R.round_to(rng.uniform(-20, 20, (G, N)).astype(np.float32), sz)
    return q, s, z


I8_CASES = [
    (1, 4096, 4096, 128), (3, 1024, 392, 16), (16, 2048, 1024, 64), (8, 48, 24, 16),
    (1, 14336, 512, 128),
    (17, 512, 256, 128), (128, 4096, 1024, 128), (300, 1024, 768, 32), (512, 1024, 2048, 128),
    (40, 256, 200, 128), (5, 100, 21, 25),
]


@pytest.mark.parametrize("M,K,N,gs", I8_CASES)
@pytest.mark.parametrize("sz", [R.F32, R.F16])
def test_matmul_int8_fp16(mo, dev, M, K, N, gs, sz):
    print(f"matmul_int8 fp16 M={M} K={K} N={N} gs={gs} sz={sz}", flush=True)
    q, s, z = _int8_weights(K, N, gs, sz, M + K + N)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half()
    Y = mo.matmul_int8(X.to(dev), torch.from_numpy(q).to(dev),
                       torch.from_numpy(s).to(TDT[sz]).to(dev), torch.from_numpy(z).to(TDT[sz]).to(dev), gs)
    assert Y.dtype == torch.float16 and tuple(Y.shape) == (M, N)
    _check_rows(Y.float().cpu().numpy(), R.matmul_int8_f32(X.float().numpy(), q, s, z, gs))


GEMV1_I8_CASES = [
    # (M, K, N, gs, steps per wave or None): int8 weights on the async-copy GEMV
    (1, 4096, 4096, 128, None), (1, 4096, 14336, 128, None), (1, 14336, 4096, 128, None),
    (1, 4096, 32000, 128, None), (1, 160, 128, 32, 2), (1, 2048, 384, 64, 3),
    (2, 4096, 4096, 128, None), (5, 11008, 4096, 128, None), (8, 4096, 1024, 32, None),
    (16, 4096, 14336, 128, None), (16, 14336, 4096, 128, None), (11, 1024, 16384, 256, None),
]


@pytest.mark.parametrize("M,K,N,gs,spw", GEMV1_I8_CASES)
@pytest.mark.parametrize("sz", [R.F16, R.BF16, R.F32])
def test_gemv1_int8(mo, dev, monkeypatch, M, K, N, gs, spw, sz):
    """Int8 weights on the async-copy GEMV against the oracle, repeat calls and
    the agent-scope split exchange (identical bits), strided activations, and
    the register-ring int8 GEMV."""
    print(f"gemv1 int8 M={M} K={K} N={N} gs={gs} spw={spw} sz={sz}", flush=True)
    for k in ("MCQ4_I4_SPW1", "MCQ4_I4_GEMV1", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    if spw is not None:
        monkeypatch.setenv("MCQ4_I4_SPW1", str(spw))
    q, s, z = _int8_weights(K, N, gs, sz, M + K + N + gs)
    args = [torch.from_numpy(q).to(dev), torch.from_numpy(s).to(TDT[sz]).to(dev),
            torch.from_numpy(z).to(TDT[sz]).to(dev)]
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M * K + 1)).half().to(dev)
    Yref = R.matmul_int8_f32(X.float().cpu().numpy(), q, s, z, gs)
    Y = mo.matmul_int8(X, *args, gs)
    _check_rows(Y.float().cpu().numpy(), Yref)
    assert torch.equal(mo.matmul_int8(X, *args, gs).view(torch.int16), Y.view(torch.int16))
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    assert torch.equal(mo.matmul_int8(X, *args, gs).view(torch.int16), Y.view(torch.int16))
    monkeypatch.delenv("MCQ4_XCD_LOCAL")
    Xw = torch.zeros(M, K + 64, dtype=torch.float16, device=dev)
    Xw[:, :K] = X
    assert torch.equal(mo.matmul_int8(Xw[:, :K], *args, gs).view(torch.int16), Y.view(torch.int16))
    monkeypatch.setenv("MCQ4_I4_GEMV1", "4")            # async-copy GEMV for 4-bit weights only
    _check_rows(mo.matmul_int8(X, *args, gs).float().cpu().numpy(), Yref)


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_matmul_int8_other_dtypes(mo, dev, xdt):
    M, K, N, gs = 6, 512, 136, 64
    q, s, z = _int8_weights(K, N, gs, R.F32, 1)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(2)).to(xdt)
    Y = mo.matmul_int8(X.to(dev), torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev),
                       torch.from_numpy(z).to(dev), gs)
    assert Y.dtype == xdt
    _check_rows(Y.float().cpu().numpy(), R.matmul_int8_f32(X.float().numpy(), q, s, z, gs))


# ---- M == 1 async-copy GEMV (i4_gemv1.hip) ----------------------------------------

GEMV1_CASES = [
    # (K, N, gs, steps per wave of the split-K GEMV or None for its default plan)
    (4096, 4096, 128, None), (4096, 12288, 128, None), (11008, 4096, 128, None),
    (4096, 1024, 32, None), (2048, 512, 64, 3), (4096, 256, 128, 2), (4096, 384, 128, 16),
    (160, 128, 32, 2), (32, 128, 32, None), (14336, 512, 256, 5), (16384, 256, 512, None),
    (4096, 4112, 128, None), (11008, 1040, 64, None), (288, 144, 32, None), (1024, 16400, 128, None),
]


@pytest.mark.parametrize("K,N,gs,spw", GEMV1_CASES)
@pytest.mark.parametrize("sz", [R.F32, R.F16, R.BF16])
def test_gemv1_paths(mo, dev, monkeypatch, K, N, gs, spw, sz):
    """The M == 1 async-copy GEMV and the register-ring GEMV against the oracle:
    split and unsplit plans, ragged step ranges, group sizes 32..512, N not a
    multiple of 128 (register ring only), all scale dtypes."""
    print(f"gemv1 K={K} N={N} gs={gs} spw={spw} sz={sz}", flush=True)
    for k in ("MCQ4_I4_SPW1", "MCQ4_I4_GEMV1", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    if spw is not None:
        monkeypatch.setenv("MCQ4_I4_SPW1", str(spw))
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=K + N + gs)
    X = torch.randn(1, K, generator=torch.Generator().manual_seed(K)).half().to(dev)
    Yref = _ref(X, packed, s, z, gs)
    for rep in range(2):                       # split-K counters are left at zero
        Y = mo.matmul_int4(X, packed, s, z, gs)
        _check_rows(Y.float().cpu().numpy(), Yref)
    # the agent-scope split exchange sums the same partials in the same order
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    Y0 = mo.matmul_int4(X, packed, s, z, gs)
    assert torch.equal(Y0.view(torch.int16), Y.view(torch.int16))
    monkeypatch.delenv("MCQ4_XCD_LOCAL")
    # the register-ring GEMV
    monkeypatch.setenv("MCQ4_I4_GEMV1", "0")
    _check_rows(mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy(), Yref)


GEMV1_MR_CASES = [
    # (M, K, N, gs, steps per wave or None)
    (2, 4096, 4096, 128, None), (3, 4096, 14336, 128, None), (4, 14336, 4096, 128, None),
    (8, 4096, 1024, 32, None), (9, 2048, 512, 64, 3), (16, 4096, 14336, 128, None),
    (16, 11008, 4096, 128, None), (5, 160, 128, 32, 2), (16, 32, 256, 32, None), (7, 1024, 16384, 128, None),
    # two 16-row activation blocks (M = 17..32)
    (17, 4096, 4096, 128, None), (24, 14336, 4096, 128, None), (32, 4096, 14336, 128, None),
    (20, 2048, 512, 64, 3), (31, 1024, 16384, 128, None), (32, 160, 128, 32, 2), (29, 11008, 1024, 256, None),
]


@pytest.mark.parametrize("M,K,N,gs,spw", GEMV1_MR_CASES)
@pytest.mark.parametrize("sz", [R.F16, R.BF16, R.F32])
def test_gemv1_multirow(mo, dev, monkeypatch, M, K, N, gs, spw, sz):
    """The async-copy GEMV with 2..16 activation rows (each ring slot carries the
    step's activation block) against the oracle, the register-ring GEMV, and the
    agent-scope split exchange (identical bits)."""
    print(f"gemv1 multirow M={M} K={K} N={N} gs={gs} spw={spw} sz={sz}", flush=True)
    for k in ("MCQ4_I4_SPW1", "MCQ4_I4_GEMV1", "MCQ4_I4_PATH", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    if spw is not None:
        monkeypatch.setenv("MCQ4_I4_SPW1", str(spw))
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=M + K + N + gs)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M * K)).half().to(dev)
    Yref = _ref(X, packed, s, z, gs)
    Y = mo.matmul_int4(X, packed, s, z, gs)
    _check_rows(Y.float().cpu().numpy(), Yref)
    Y2 = mo.matmul_int4(X, packed, s, z, gs)                  # counters were left at zero
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    assert torch.equal(mo.matmul_int4(X, packed, s, z, gs).view(torch.int16), Y.view(torch.int16))
    monkeypatch.delenv("MCQ4_XCD_LOCAL")
    # row-strided activations: a view into a wider buffer
    Xw = torch.zeros(M, K + 64, dtype=torch.float16, device=dev)
    Xw[:, :K] = X
    assert torch.equal(mo.matmul_int4(Xw[:, :K], packed, s, z, gs).view(torch.int16), Y.view(torch.int16))
    # the register-ring GEMV (async-copy kernel limited to M == 1)
    monkeypatch.setenv("MCQ4_I4_GEMV1", "1")
    _check_rows(mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy(), Yref)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_gemv1_fused_activation(mo, dev, act):
    K, N, gs = 4096, 1024, 128
    w, packed, s, z = _quant(mo, dev, K, N, gs, seed=41)
    X = (torch.randn(1, K, generator=torch.Generator().manual_seed(9)) * 4).half().to(dev)
    fn = mo.matmul_int4_silu if act == "silu" else mo.matmul_int4_gelu
    Y = fn(X, packed, s, z, gs).float().cpu().numpy().astype(np.float64)
    base = _ref(X, packed, s, z, gs).astype(np.float64)
    want = _silu(base) if act == "silu" else _gelu_tanh(base)
    assert np.isfinite(Y).all()
    scale = np.maximum(np.abs(base).max(axis=-1, keepdims=True), 1e-6)
    assert (np.abs(Y - want) / scale).max() <= 1e-2


# ---- prefill GEMM with the activation tile in LDS (i4_gemm6.hip) --------------------

@pytest.mark.parametrize("M,K,N,gs", [(17, 512, 256, 128), (130, 96, 384, 32), (300, 2048, 768, 64),
                                      (512, 4096, 1024, 128), (2048, 1024, 512, 128), (129, 11008, 256, 128),
                                      (64, 160, 640, 32)])
@pytest.mark.parametrize("sz", [R.F16, R.BF16])
def test_gemm6_paths(mo, dev, monkeypatch, M, K, N, gs, sz):
    """i4_gemm6 and i4_gemm against the oracle: split K, odd step counts, ragged M."""
    print(f"gemm6 M={M} K={K} N={N} gs={gs} sz={sz}", flush=True)
    monkeypatch.delenv("MCQ4_I4_GEMM6", raising=False)
    monkeypatch.delenv("MCQ4_I4_PATH", raising=False)
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=M + K + gs)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half().to(dev)
    Yref = _ref(X, packed, s, z, gs)
    for rep in range(2):
        _check_rows(mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy(), Yref)
    monkeypatch.setenv("MCQ4_I4_GEMM6", "0")
    _check_rows(mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy(), Yref)


def _random_decode_shapes(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        gs = int(rng.choice([32, 64, 128, 256]))
        K = int(rng.integers(1, 64)) * gs
        N = int(rng.integers(1, 40)) * 128
        M = int(rng.integers(1, 17))
        out.append((M, K, N, gs))
    return out


@pytest.mark.parametrize("M,K,N,gs", _random_decode_shapes(16, 2024))
def test_decode_random_shapes(mo, dev, M, K, N, gs):
    """Seeded random decode shapes (M 1..16, any group size, tile counts that are
    not multiples of 8) through the default kernels, against the oracle."""
    print(f"random decode M={M} K={K} N={N} gs={gs}", flush=True)
    w, packed, s, z = _quant(mo, dev, K, N, gs, seed=M * 7 + K + N)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(K + M)).half().to(dev)
    _check_rows(mo.matmul_int4(X, packed, s, z, gs).float().cpu().numpy(), _ref(X, packed, s, z, gs))


@pytest.mark.parametrize("M,K,N,gs", _random_decode_shapes(12, 2025))
def test_decode_random_shapes_int8(mo, dev, monkeypatch, M, K, N, gs):
    """Seeded random int8 decode shapes on the default routing (the async-copy
    GEMV where it applies) and on the register-ring GEMV, against the oracle."""
    print(f"random int8 decode M={M} K={K} N={N} gs={gs}", flush=True)
    monkeypatch.delenv("MCQ4_I4_SPW1", raising=False)
    q, s, z = _int8_weights(K, N, gs, R.F16, M * 5 + K + N)
    args = [torch.from_numpy(q).to(dev), torch.from_numpy(s).half().to(dev), torch.from_numpy(z).half().to(dev)]
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(K * 3 + M)).half().to(dev)
    Yref = R.matmul_int8_f32(X.float().cpu().numpy(), q, s, z, gs)
    monkeypatch.delenv("MCQ4_I4_GEMV1", raising=False)
    _check_rows(mo.matmul_int8(X, *args, gs).float().cpu().numpy(), Yref)
    monkeypatch.setenv("MCQ4_I4_GEMV1", "4")
    _check_rows(mo.matmul_int8(X, *args, gs).float().cpu().numpy(), Yref)


def _random_i4_cases(n, seed):
    """Seeded random (M, K, N, gs, sz) over the decode GEMVs and the prefill GEMMs:
    group sizes 32..128, fp16/bf16/fp32 scales, ragged and aligned N."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.choice([1, 1, 2, 5, 8, 16, 17, 32, 33, 64, 130, 300, 520]))
        gs = int(rng.choice([32, 64, 128]))
        K = gs * int(rng.integers(1, max(2, 4096 // gs)))
        N = int(rng.choice([int(rng.integers(1, 300)), 128 * int(rng.integers(1, 20)), 8 * int(rng.integers(1, 200))]))
        sz = [R.F16, R.BF16, R.F32][int(rng.integers(0, 3))]
        out.append((M, K, N, gs, sz))
    return out


@pytest.mark.parametrize("M,K,N,gs,sz", _random_i4_cases(32, 4242))
def test_matmul_random_shapes(mo, dev, M, K, N, gs, sz):
    print(f"random matmul_int4 M={M} K={K} N={N} gs={gs} sz={sz}", flush=True)
    w, packed, s, z = _quant(mo, dev, K, N, gs, sz, seed=M + K + N)
    X = torch.randn(M, K, generator=torch.Generator().manual_seed(M + K)).half().to(dev)
    Y = mo.matmul_int4(X, packed, s, z, gs)
    _check_rows(Y.float().cpu().numpy(), _ref(X, packed, s, z, gs))
