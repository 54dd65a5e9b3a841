"""GPU parity: the HIP kernels of libmcq4.so against the CPU oracle.

Bars (from the reference semantics, quantization.py:307-454):
  * quantize (both rules): bit-exact bytes.
  * dequantize: bit-exact fp32 and fp16.
  * matmul: max|err| <= 1e-2 * ||Y_ref[m, :]||_inf per row, Y_ref = X.float() @ dequant_f32(W)
    (TOL below); in practice the kernels sit orders of magnitude inside it.
"""
import numpy as np
import pytest
import torch

from oracle import q4_0_ref as ref

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _mo():
    import metalops_amd as mo
    return mo


def _weights(K, N, seed, outliers=False):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(K, N, generator=g) * 0.02
    if outliers:
        n = max(1, W.numel() // 100)
        idx = torch.randperm(W.numel(), generator=g)[:n]
        W.view(-1)[idx] = torch.randn(n, generator=g) * 0.2
    return W


def _acts(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).half()


def _check_rows(Y, Yref, tol=TOL):
    Y = np.asarray(Y, dtype=np.float64)
    Yref = np.asarray(Yref, dtype=np.float64)
    assert np.isfinite(Y).all(), f"non-finite outputs at {np.argwhere(~np.isfinite(Y))[:4].tolist()}"
    err = np.abs(Y - Yref).max(axis=1)
    bound = tol * np.abs(Yref).max(axis=1)
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, f"rows {bad[:8]} exceed tolerance: err={err[bad[:4]]} bound={bound[bad[:4]]}"
    return float((err / np.maximum(bound, 1e-30)).max())


@pytest.mark.parametrize("K,N", [(32, 1), (32, 7), (64, 33), (352, 257), (4096, 96)])
@pytest.mark.parametrize("rule", ["ref", "ref_f16", "ref_bf16", "llama"])
def test_quantize_bit_exact(dev, K, N, rule):
    """Reference rule for fp32, fp16 and bf16 weights (every step rounded in the
    weight's dtype, quantization.py:335-347) and the llama.cpp generator rule."""
    mo = _mo()
    W = _weights(K, N, seed=K * 7 + N, outliers=True)
    W[:32, 0] = 0.0  # an all-zero block
    if K >= 64 and N >= 2:
        W[32:64, 1] = torch.randn(32) * 1e-7            # fp16 subnormal range: amax/7 -> 0 in fp16
    if rule.startswith("ref"):
        tdt, name = {"ref": (torch.float32, "float32"), "ref_f16": (torch.float16, "float16"),
                     "ref_bf16": (torch.bfloat16, "bfloat16")}[rule]
        Wd = W.to(tdt)
        got = mo.quantize_ggml_q4_0(Wd.to(dev)).cpu().numpy()
        want = ref.quantize_ref_rule(Wd.float().numpy(), name)
    else:
        got = mo.quantize_ggml_q4_0_llama(W.to(dev)).cpu().numpy()
        want = ref.quantize_llama_rule(W.numpy())
    assert got.shape == (K // 32, N, 18)
    np.testing.assert_array_equal(got, want)


def test_quantize_ties_and_specials(dev):
    mo = _mo()
    # Column 0: amax = 7 -> d = 1 exactly, so x + 8 lands on .5 ties: half-to-even.
    col = np.zeros(32, np.float32)
    col[:8] = [7.0, 0.5, 1.5, -0.5, -1.5, 2.5, -2.5, 6.5]
    W = np.zeros((32, 4), np.float32)
    W[:, 0] = col
    W[5, 1] = -3.0          # single-hot negative
    W[:, 2] = np.linspace(-1, 1, 32, dtype=np.float32)
    got = mo.quantize_ggml_q4_0(torch.from_numpy(W).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, ref.quantize_ref_rule(W))
    q, d = ref.unpack_nibbles(got)
    assert list(q[0, 0, :8]) == [15, 8, 10, 8, 6, 10, 6, 14]
    assert d[0, 3] == np.float16(1.0) and (q[0, 3] == 8).all()   # zero block: d = 1, q = 8


@pytest.mark.parametrize("K,N", [(32, 1), (64, 33), (352, 257), (1024, 640)])
def test_dequant_bit_exact(dev, K, N):
    mo = _mo()
    rng = np.random.default_rng(K + N)
    blocks = rng.integers(0, 256, size=(K // 32, N, 18), dtype=np.uint8)
    # keep scales finite: random fp16 in a sane exponent range, both signs, some subnormals
    d = (rng.standard_normal((K // 32, N)) * 0.01).astype(np.float16)
    d.reshape(-1)[:5] = np.array([0.0, -0.0, 6e-8, -6e-8, 65504.0], np.float16)[: min(5, d.size)]
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(K // 32, N, 2)
    tb = torch.from_numpy(blocks).to(dev)
    got32 = mo.dequantize_ggml_q4_0(tb, torch.float32).cpu().numpy()
    np.testing.assert_array_equal(got32.view(np.uint32), ref.dequantize(blocks, np.float32).view(np.uint32))
    got16 = mo.dequantize_ggml_q4_0(tb).cpu().numpy()
    assert got16.dtype == np.float16
    np.testing.assert_array_equal(got16.view(np.uint16), ref.dequantize(blocks, np.float16).view(np.uint16))


SMALL_SHAPES = [
    (1, 32, 1), (1, 64, 33), (1, 352, 257), (2, 256, 100), (5, 352, 33), (16, 1024, 48),
    (17, 352, 40), (33, 512, 130), (64, 256, 64), (1, 4096, 96), (4, 14336, 64),
    (65, 352, 70), (100, 512, 300), (128, 1024, 256), (257, 352, 130), (300, 2048, 520),
]


@pytest.mark.parametrize("M,K,N", SMALL_SHAPES)
def test_matmul_small_vs_oracle(dev, M, K, N):
    mo = _mo()
    W = _weights(K, N, seed=M + K + N, outliers=True)
    X = _acts(M, K, seed=M * 3 + 1)
    blocks = ref.quantize_llama_rule(W.numpy())
    Y = mo.matmul_ggml_q4_0(X.to(dev), torch.from_numpy(blocks).to(dev))
    assert Y.dtype == torch.float16 and Y.shape == (M, N)
    _check_rows(Y.float().cpu().numpy(), ref.matmul_f32(X.numpy(), blocks))


def test_matmul_matches_f64_bruteforce(dev):
    mo = _mo()
    W = _weights(96, 9, seed=5)
    X = _acts(3, 96, seed=6)
    blocks = ref.quantize_ref_rule(W.numpy())
    Y = mo.matmul_ggml_q4_0(X.to(dev), torch.from_numpy(blocks).to(dev)).float().cpu().numpy()
    _check_rows(Y, ref.matmul_f64(X.numpy(), blocks), tol=2e-3)


def test_matmul_deterministic(dev):
    mo = _mo()
    W = _weights(2048, 384, seed=1)
    X = _acts(8, 2048, seed=2)
    b = mo.quantize_ggml_q4_0(W.to(dev))
    y1 = mo.matmul_ggml_q4_0(X.to(dev), b)
    y2 = mo.matmul_ggml_q4_0(X.to(dev), b)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("tdtype,name", [(torch.float32, "float32"), (torch.bfloat16, "bfloat16")])
@pytest.mark.parametrize("M,K,N", [(1, 352, 257), (5, 1024, 96), (33, 512, 130), (130, 2048, 264)])
def test_matmul_activation_dtypes(dev, tdtype, name, M, K, N):
    """bf16 / fp32 activations follow the reference's path for them
    (quantization.py:452-454): W dequantized to X's dtype, the product in X's
    dtype, the result in X's dtype.  Oracle: the same rounding of W, float64
    sums; bar 1e-2 of the row's max (bf16 output rounding is 2^-9 relative) and
    1e-5 for fp32."""
    mo = _mo()
    W = _weights(K, N, seed=M + K, outliers=True)
    g = torch.Generator().manual_seed(M * 5 + N)
    X = torch.randn(M, K, generator=g).to(tdtype)
    blocks = ref.quantize_llama_rule(W.numpy())
    Y = mo.matmul_ggml_q4_0(X.to(dev), torch.from_numpy(blocks).to(dev))
    assert Y.dtype == tdtype and Y.shape == (M, N)
    Yref = ref.matmul_xdtype(X.float().numpy(), blocks, name)
    _check_rows(Y.float().cpu().numpy(), Yref, tol=TOL if tdtype == torch.bfloat16 else 1e-5)


def test_matmul_bf16_beyond_fp16_range(dev):
    """bf16 activations of magnitude 1e6 (inf in fp16): finite results equal to
    the reference's bf16 path, where an fp16 cast would give inf."""
    mo = _mo()
    W = _weights(256, 64, seed=3)
    X = (torch.randn(4, 256, generator=torch.Generator().manual_seed(4)) * 1e6).to(torch.bfloat16)
    blocks = ref.quantize_ref_rule(W.numpy())
    Y = mo.matmul_ggml_q4_0(X.to(dev), torch.from_numpy(blocks).to(dev))
    assert torch.isfinite(Y.float()).all()
    _check_rows(Y.float().cpu().numpy(), ref.matmul_xdtype(X.float().numpy(), blocks, "bfloat16"))


def _full_size_check(dev, M, K, N, outliers=False):
    """Full-size config: GPU quantize (llama rule), kernel vs fp32 torch GEMM of the
    bit-exact GPU dequant (dequant itself is pinned bit-exact against the oracle above)."""
    mo = _mo()
    g = torch.Generator(device=dev).manual_seed(M + K + N)
    W = torch.randn(K, N, generator=g, device=dev) * 0.02
    if outliers:
        n = W.numel() // 100
        idx = torch.randperm(W.numel(), generator=g, device=dev)[:n]
        W.view(-1)[idx] = torch.randn(n, generator=g, device=dev) * 0.2
    X = torch.randn(M, K, generator=g, device=dev).half()
    b = mo.quantize_ggml_q4_0_llama(W)
    del W
    Y = mo.matmul_ggml_q4_0(X, b).float()
    Yref = X.float() @ mo.dequantize_ggml_q4_0(b, torch.float32)
    err = (Y - Yref).abs().amax(dim=1)
    bound = TOL * Yref.abs().amax(dim=1)
    assert bool((err <= bound).all()), f"max err/bound {(err / bound).max().item()}"


@pytest.mark.parametrize("M,K,N", [
    (1, 4096, 12288), (1, 4096, 4096), (1, 4096, 11008), (1, 11008, 4096),
    (4, 4096, 14336), (8, 4096, 14336), (16, 4096, 14336),
    (4, 14336, 4096), (8, 14336, 4096), (16, 14336, 4096),
])
def test_matmul_decode_configs(dev, M, K, N):
    _full_size_check(dev, M, K, N)


@pytest.mark.parametrize("M,K,N", [(2048, 4096, 14336), (2048, 14336, 4096), (512, 11008, 4096)])
def test_matmul_prefill_configs(dev, M, K, N):
    _full_size_check(dev, M, K, N, outliers=True)


def test_matmul_lm_head(dev):
    _full_size_check(dev, 1, 4096, 128256)
    _full_size_check(dev, 512, 4096, 128256)


def test_matmul_ragged_down(dev):
    """K = 11008 (43 K blocks of 256, not a multiple of the K tile) at M = 1 and 512."""
    _full_size_check(dev, 1, 11008, 4096)
    _full_size_check(dev, 512, 11008, 4096, outliers=True)


# Every kernel variant on ragged and full shapes, pinned through the library's
# MCQ4_* switches (re-read on each environment write, tests/conftest.py).
PATHS = {
    "gemv_dma": {},
    "gemv_dma_wide": {},

    "decode_lds_m1": {"MCQ4_GEMV_PATH": "off"},
    "gemvm": {},
    "gemvm_nohoist": {"MCQ4_GEMVM_HOIST": "0"},
    "gemvm_split2": {"MCQ4_GEMVM_SPLIT": "2"},
    "gemvm_split8": {"MCQ4_GEMVM_SPLIT": "8"},
    "gemvm_split4": {"MCQ4_GEMVM_SPLIT": "4"},
    "gemvm_split2_reduce": {"MCQ4_GEMVM_SPLIT": "2", "MCQ4_XCD_LOCAL": "0"},
    "decode_lds": {},
    "gemvm_rb2": {},
    "gemvm_rb2_split2": {"MCQ4_GEMVM_SPLIT": "2"},
    "gemvm_rb2_split4_reduce": {"MCQ4_GEMVM_SPLIT": "4", "MCQ4_XCD_LOCAL": "0"},
    "gemm6_33_64": {},
    "decode_lds_small_m": {"MCQ4_GEMV_PATH": "off"},
    "decode_direct": {"MCQ4_DECODE_PATH": "direct"},
    "gemm_sync": {"MCQ4_GEMM_PATH": "sync"},
    "gemm_async_bm256": {"MCQ4_GEMM_PATH": "async", "MCQ4_GEMM2_BM": "256"},
    "gemm_async_bm128": {"MCQ4_GEMM_PATH": "async", "MCQ4_GEMM2_BM": "128"},
    "gemm6": {"MCQ4_GEMM_PATH": "6"},
    "gemm6_split3": {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "3"},
    "gemm6_split2": {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "2"},
    "gemm6_split2_reduce": {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "2", "MCQ4_XCD_LOCAL": "0"},
    "gemm6_split4": {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "4"},
    "gemm6_split8": {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "8"},
    "gemm6_split16": {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "16"},
    "gemm7": {"MCQ4_GEMM_PATH": "7"},
    "gemm7_split2": {"MCQ4_GEMM_PATH": "7", "MCQ4_GEMM6_SPLIT": "2"},
    "gemm7_split3": {"MCQ4_GEMM_PATH": "7", "MCQ4_GEMM6_SPLIT": "3"},
    "gemm8": {"MCQ4_GEMM_PATH": "8"},
    "gemm8_split1": {"MCQ4_GEMM_PATH": "8", "MCQ4_GEMM8_SPLIT": "1"},
    "gemm8_split2": {"MCQ4_GEMM_PATH": "8", "MCQ4_GEMM8_SPLIT": "2"},
    "gemv_span": {},
    "gemv_span_split": {"MCQ4_GEMV_SPAN": "1"},
    "gemv_span_split_off": {"MCQ4_GEMV_SPAN": "0"},
    "gemv_span_off": {"MCQ4_GEMV_SPAN": "0"},
    "skinny_tail": {},
}
PATH_SHAPES = {
    "gemv_dma": [(1, 32, 16), (1, 352, 264), (1, 1024, 4104), (1, 11008, 512), (1, 4096, 65536),
                 (1, 16384, 272), (1, 14336, 4096)],
    # 64-column tiles (N >= 65536, N % 64 == 0): one K block, odd block counts
    # (a last item of one row) and waves without batches.
    "gemv_dma_wide": [(1, 32, 65536), (1, 352, 65536), (1, 2080, 65600), (1, 4096, 70016)],

    # Contiguous spans of 16-column groups (M <= 16, 4096 < N <= 16384, K <= 4096):
    # one to four groups per workgroup, one K block, a partial last batch, the
    # largest K and N, ragged group counts (257, 513, 767 groups).
    "gemv_span": [(1, 32, 4112), (1, 352, 8208), (1, 4096, 12288), (1, 4064, 12272), (1, 2080, 6144),
                  (1, 96, 4128), (1, 4096, 8192), (1, 4096, 16384), (1, 1024, 14336),
                  # M = 2..16: 4, 8 and 16 distinct rows per MFMA A operand.
                  (2, 352, 8208), (3, 4096, 14336), (4, 4096, 14336), (5, 32, 4112), (8, 2080, 16384),
                  (9, 4096, 12288), (12, 96, 16368), (16, 4096, 14336), (16, 4064, 6144)],
    "gemv_span_off": [(1, 4096, 12288), (1, 352, 8208), (4, 4096, 14336), (16, 352, 8208)],
    # 64-column spans over K splits (2 <= M <= 16, N % 64 == 0, N <= 4096; forced,
    # since by default only splits of 64+ K blocks take it): 4, 8, 16 distinct rows
    # per MFMA; 2 to 8 splits; a last split shorter than the others, waves without
    # an item, partial last batches, grid padding.
    "gemv_span_split": [(2, 14336, 4096), (4, 14336, 4096), (8, 14336, 4096), (16, 14336, 4096),
                        (3, 11008, 4096), (7, 4096, 4096), (12, 4096, 2048), (16, 16384, 4096),
                        (5, 352, 1024), (9, 2080, 2048), (13, 1024, 64), (6, 4128, 3008)],
    "gemv_span_split_off": [(4, 14336, 4096), (16, 4096, 4096)],
    # N % 16 != 0 with K >= 2048: the columns past the last whole 16-column tile, K
    # split over workgroups whose partials a second kernel sums; after the M = 1
    # strip kernel, the small-batch strip kernel (one and two row blocks) and, at
    # N >= 8192, 32-column tail tiles.
    # (At M = 1 the strip kernel takes an 8-column last tile itself.)
    "skinny_tail": [(1, 4096, 4104), (1, 11008, 4104), (1, 2048, 2056), (1, 4096, 32008), (1, 32, 24),
                    (1, 4128, 40), (1, 352, 1048), (3, 2048, 2056),
                    (12, 11008, 8200), (20, 4096, 1032), (32, 14336, 520), (16, 4096, 8200)],
    "decode_lds_m1": [(1, 352, 264), (1, 4096, 1032)],
    "gemvm": [(2, 32, 16), (3, 352, 264), (4, 1024, 4104), (5, 11008, 512), (8, 4096, 14336),
              (11, 2048, 1040), (16, 14336, 4096), (16, 352, 8200)],
    # One batch per wave (the hoisted -S form by default) with it turned off.
    "gemvm_nohoist": [(16, 14336, 4096), (8, 4096, 14336), (3, 352, 264), (16, 352, 8200)],
    "gemvm_split2": [(2, 352, 264), (9, 4096, 1040), (16, 14336, 4096), (5, 11008, 512)],
    "gemvm_split8": [(16, 2048, 1032), (3, 14336, 512), (12, 512, 200)],
    "gemvm_split4": [(16, 4096, 1040), (6, 11008, 264), (13, 352, 8200)],
    "gemvm_split2_reduce": [(9, 4096, 1040), (16, 14336, 4096), (4, 4096, 1040), (8, 2048, 264)],
    "decode_lds": [(1, 352, 264), (40, 2048, 96), (64, 256, 64), (17, 1024, 520), (33, 4096, 1032)],
    "gemvm_rb2": [(17, 4096, 1024), (20, 2048, 4096), (32, 14336, 512), (31, 1024, 2048), (18, 352, 272),
                  (24, 4096, 1032), (29, 11008, 4096)],
    "gemvm_rb2_split2": [(32, 14336, 4096), (21, 4096, 1040), (17, 2048, 264)],
    "gemvm_rb2_split4_reduce": [(32, 4096, 1024), (25, 11008, 512)],
    "gemm6_33_64": [(33, 4096, 1024), (48, 2048, 768), (64, 11008, 512), (40, 352, 256)],
    "decode_lds_small_m": [(3, 1024, 520), (16, 4096, 1032)],
    "decode_direct": [(1, 352, 257), (7, 1024, 520), (16, 4096, 1000), (64, 512, 72)],
    "gemm_sync": [(65, 352, 70), (200, 1024, 264), (300, 2048, 520)],
    "gemm_async_bm256": [(65, 352, 72), (257, 1024, 264), (300, 2048, 520), (512, 4096, 776)],
    "gemm_async_bm128": [(65, 352, 72), (129, 1024, 264), (300, 2048, 520), (384, 4096, 776)],
    "gemm6": [(129, 352, 128), (257, 1024, 384), (300, 2048, 512), (512, 4096, 768), (2048, 4096, 1024),
              (200, 32, 256), (130, 64, 384), (513, 96, 256), (2048, 11008, 512)],
    "gemm6_split3": [(200, 352, 384), (300, 4096, 640)],
    "gemm6_split2": [(200, 352, 384), (300, 4096, 640), (512, 4096, 1024), (129, 1024, 2304)],
    "gemm6_split2_reduce": [(300, 4096, 640), (129, 1024, 2304)],
    "gemm6_split4": [(200, 2048, 384), (300, 4096, 640), (512, 11008, 1024)],
    "gemm6_split8": [(129, 4096, 256), (512, 11008, 512), (300, 8192, 768)],
    "gemm6_split16": [(200, 16384, 256), (130, 8192, 384)],
    "gemm7": [(129, 352, 128), (257, 1024, 384), (300, 2048, 512), (512, 4096, 768), (2048, 4096, 1024),
              (200, 32, 256), (130, 64, 384), (513, 96, 256), (2048, 11008, 512), (65, 4096, 4096)],
    "gemm7_split2": [(200, 352, 384), (300, 4096, 640), (512, 4096, 1024)],
    "gemm7_split3": [(300, 4096, 640), (129, 2048, 2304)],
    # K blocks per split below, at and past one four-block stage (1, 3, 5, 7 blocks:
    # phases idle in the last stage), and the plan's two splits.
    "gemm8": [(129, 352, 128), (257, 1024, 384), (300, 2048, 512), (512, 4096, 768), (2048, 4096, 1024),
              (200, 32, 256), (513, 96, 256), (100, 160, 128), (200, 224, 256), (512, 11008, 4096),
              (2048, 11008, 512)],
    "gemm8_split1": [(512, 4096, 768), (300, 2048, 512), (130, 4128, 256), (65, 1024, 128)],
    "gemm8_split2": [(600, 1056, 640), (2048, 4096, 1024), (129, 1024, 2304)],
}


@pytest.mark.parametrize("path,M,K,N", [(p, *s) for p, shapes in PATH_SHAPES.items() for s in shapes])
def test_matmul_each_kernel(dev, monkeypatch, path, M, K, N):
    for k in ("MCQ4_DECODE_PATH", "MCQ4_GEMM_PATH", "MCQ4_GEMM2_BM", "MCQ4_GEMV_PATH",
              "MCQ4_GEMM6_SPLIT", "MCQ4_GEMM8_SPLIT", "MCQ4_GEMVM_SPLIT", "MCQ4_GEMVM_HOIST", "MCQ4_XCD_LOCAL",
              "MCQ4_GEMV_SPAN"):
        monkeypatch.delenv(k, raising=False)
    for k, v in PATHS[path].items():
        monkeypatch.setenv(k, v)
    mo = _mo()
    W = _weights(K, N, seed=M * 7 + K + N, outliers=True)
    X = _acts(M, K, seed=M + 11)
    blocks = ref.quantize_llama_rule(W.numpy())
    Y = mo.matmul_ggml_q4_0(X.to(dev), torch.from_numpy(blocks).to(dev))
    _check_rows(Y.float().cpu().numpy(), ref.matmul_f32(X.numpy(), blocks))


@pytest.mark.parametrize("M,K,N,split", [(2048, 14336, 4096, "gemm2"), (300, 4096, 640, "gemm2"),
                                         (1000, 2048, 1280, "gemm2"), (512, 11008, 4096, "gemm4"),
                                         (300, 4096, 640, "gemm3"), (384, 4096, 4096, "gemm4"),
                                         (16, 14336, 4096, "gemvm2"),
                                         (9, 4096, 1040, "gemvm2"), (12, 11008, 8200, "gemvm4"),
                                         (16, 2048, 1032, "gemvm8"), (512, 11008, 4096, "few8"),
                                         (600, 1056, 640, "few8")])
def test_split_exchange_matches_reduce(dev, monkeypatch, M, K, N, split):
    """K split over workgroups: the in-kernel XCD-local sum (default) and the
    reduction kernel add the same partials in the same order (two splits of the
    GEMM: p0 + p1, which commutes; three or four splits go to the reduction
    kernel either way), so the outputs are identical bits.  The few-tile GEMM
    (q4_gemm8, two splits) has no reduction-kernel form: its runs must repeat
    bit for bit."""
    print(f"split exchange {split} M={M} K={K} N={N}", flush=True)
    for k in ("MCQ4_GEMM_PATH", "MCQ4_XCD_LOCAL", "MCQ4_GEMM6_SPLIT", "MCQ4_GEMM8_SPLIT", "MCQ4_GEMVM_SPLIT",
              "MCQ4_GEMV_PATH"):
        monkeypatch.delenv(k, raising=False)
    if split == "few8":
        monkeypatch.setenv("MCQ4_GEMM_PATH", "8")
    elif split.startswith("gemm"):
        monkeypatch.setenv("MCQ4_GEMM_PATH", "6")
        monkeypatch.setenv("MCQ4_GEMM6_SPLIT", split[-1])
    else:
        monkeypatch.setenv("MCQ4_GEMVM_SPLIT", split[-1])
    mo = _mo()
    g = torch.Generator().manual_seed(M + K)
    blocks = torch.randint(0, 256, (K // 32, N, 18), generator=g, dtype=torch.uint8)
    blocks[:, :, 0:2] = torch.tensor([0x1f, 0x21], dtype=torch.uint8)   # d = 0.0101 (fp16 0x211f)
    blocks = blocks.to(dev)
    X = torch.randn(M, K, generator=g).half().to(dev)
    Y = mo.matmul_ggml_q4_0(X, blocks)
    Y2 = mo.matmul_ggml_q4_0(X, blocks)
    assert torch.isfinite(Y.float()).all()
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))
    if split == "few8":
        return
    monkeypatch.setenv("MCQ4_XCD_LOCAL", "0")
    Y0 = mo.matmul_ggml_q4_0(X, blocks)
    assert torch.equal(Y.view(torch.int16), Y0.view(torch.int16))



def _random_cases(n, seed):
    """Seeded random (M, K, N, pad) shapes over every dispatch region: M from 1 to
    600 (decode kernels, the small- and large-grid GEMMs), K any multiple of 32 up
    to 4096, N ragged or aligned, and row strides past K (pad halves)."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        M = int(rng.choice([1, 1, 2, 3, 4, 7, 8, 12, 16, 17, 24, 32, 33, 48, 64, 65, 96, 130, 257, 384, 600]))
        K = 32 * int(rng.integers(1, 129))
        N = int(rng.choice([int(rng.integers(1, 400)), 8 * int(rng.integers(1, 300)),
                            128 * int(rng.integers(1, 24))]))
        pad = int(rng.choice([0, 0, 8, 40]))
        cases.append((M, K, N, pad))
    return cases


# The span kernel's region (M <= 16, 4096 < N <= 16384, K <= 4096) with row strides
# past K, which the random draw above never reaches.
SPAN_STRIDE_CASES = [(1, 2048, 8208, 8), (3, 4096, 8192, 40), (6, 352, 16384, 40), (16, 1024, 12288, 8),
                     (11, 4096, 14336, 40)]


@pytest.mark.parametrize("M,K,N,pad", _random_cases(48, 20261202) + SPAN_STRIDE_CASES)
def test_matmul_random_shapes(dev, M, K, N, pad):
    """Random shapes and strides against the oracle's fp32 product, with the
    reference-rule quantizer; the row stride of X is K + pad."""
    print(f"random matmul M={M} K={K} N={N} pad={pad}", flush=True)
    mo = _mo()
    W = _weights(K, N, seed=M * 131 + K + N, outliers=True)
    blocks = ref.quantize_ref_rule(W.numpy())
    Xw = _acts(M, K + pad, seed=M + K + pad)
    X = Xw[:, :K]
    Y = mo.matmul_ggml_q4_0(Xw.to(dev)[:, :K], torch.from_numpy(blocks).to(dev))
    assert Y.shape == (M, N) and Y.dtype == torch.float16
    _check_rows(Y.float().cpu().numpy(), ref.matmul_f32(X.contiguous().numpy(), blocks))


def _few_tile_cases(n, seed):
    """Seeded random shapes for the few-tile GEMM forced (MCQ4_GEMM_PATH=8): M 65..700,
    K any multiple of 32 up to 4096, N a multiple of 128 up to 2048, split plan 1 or 2."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(65, 701)), 32 * int(rng.integers(1, 129)), 128 * int(rng.integers(1, 17)),
             int(rng.choice([8, 40])), str(rng.choice(["1", "2"]))) for _ in range(n)]


@pytest.mark.parametrize("M,K,N,pad,split", _few_tile_cases(16, 20261203))
def test_matmul_few_tile_random(dev, monkeypatch, M, K, N, pad, split):
    """q4_gemm8 on random shapes and strides (row stride K + pad) with one or two K
    splits: against the oracle's fp32 product."""
    print(f"few-tile random M={M} K={K} N={N} pad={pad} split={split}", flush=True)
    for k in ("MCQ4_GEMM_PATH", "MCQ4_GEMM8_SPLIT", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("MCQ4_GEMM_PATH", "8")
    monkeypatch.setenv("MCQ4_GEMM8_SPLIT", split)
    mo = _mo()
    W = _weights(K, N, seed=M * 17 + K + N, outliers=True)
    blocks = ref.quantize_llama_rule(W.numpy())
    Xw = _acts(M, K + pad, seed=M + 2 * K + pad)
    Y = mo.matmul_ggml_q4_0(Xw.to(dev)[:, :K], torch.from_numpy(blocks).to(dev))
    _check_rows(Y.float().cpu().numpy(), ref.matmul_f32(Xw[:, :K].contiguous().numpy(), blocks))


@pytest.mark.parametrize("K,N,count", [(4096, 11008, 2), (4096, 4096, 3), (352, 64, 4), (11008, 4096, 2),
                                       (4096, 32768, 2), (2080, 65536, 2), (32, 16, 2)])
def test_matmul_grouped(dev, K, N, count):
    """Weights sharing one activation row in one launch (gate and up): every output
    within the bar of the oracle, and of the single-weight calls."""
    print(f"grouped matmul K={K} N={N} count={count}", flush=True)
    mo = _mo()
    Ws = [_weights(K, N, seed=K + N + 17 * g, outliers=True) for g in range(count)]
    blocks = [ref.quantize_llama_rule(W.numpy()) for W in Ws]
    X = _acts(1, K, seed=K + count)
    bd = [torch.from_numpy(b).to(dev) for b in blocks]
    Ys = mo.matmul_ggml_q4_0_grouped(X.to(dev), bd)
    assert len(Ys) == count
    for g in range(count):
        assert Ys[g].shape == (1, N) and Ys[g].dtype == torch.float16
        _check_rows(Ys[g].float().cpu().numpy(), ref.matmul_f32(X.numpy(), blocks[g]))
        _check_rows(Ys[g].float().cpu().numpy(), mo.matmul_ggml_q4_0(X.to(dev), bd[g]).float().cpu().numpy())


def _random_grouped_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        K = 32 * int(rng.integers(1, 200))
        N = 16 * int(rng.integers(1, 700))
        cases.append((K, N, int(rng.integers(2, 5))))
    return cases


@pytest.mark.parametrize("K,N,count", _random_grouped_cases(16, 20261203))
def test_matmul_grouped_random_shapes(dev, K, N, count):
    """Random grouped shapes (16-column multiples, 2..4 weights): each output within
    the bar of the oracle."""
    print(f"random grouped matmul K={K} N={N} count={count}", flush=True)
    mo = _mo()
    blocks = [ref.quantize_ref_rule(_weights(K, N, seed=K * 7 + N + g).numpy()) for g in range(count)]
    X = _acts(1, K, seed=K + N)
    Ys = mo.matmul_ggml_q4_0_grouped(X.to(dev), [torch.from_numpy(b).to(dev) for b in blocks])
    for g in range(count):
        _check_rows(Ys[g].float().cpu().numpy(), ref.matmul_f32(X.numpy(), blocks[g]))


def test_matmul_grouped_other_cases(dev):
    """Rows > 1, more than four weights and N % 16 != 0 take the per-weight path
    (the same results bit for bit); mismatched shapes are rejected."""
    mo = _mo()
    K, N = 256, 72
    blocks = [torch.from_numpy(ref.quantize_llama_rule(_weights(K, N, seed=g).numpy())).to(dev) for g in range(5)]
    for X in (_acts(3, K, seed=1).to(dev), _acts(1, K, seed=2).to(dev)):
        Ys = mo.matmul_ggml_q4_0_grouped(X, blocks)
        for g in range(5):
            assert torch.equal(Ys[g].view(torch.int16), mo.matmul_ggml_q4_0(X, blocks[g]).view(torch.int16))
    other = torch.from_numpy(ref.quantize_llama_rule(_weights(K, 64, seed=9).numpy())).to(dev)
    with pytest.raises(RuntimeError):
        mo.matmul_ggml_q4_0_grouped(_acts(1, K, seed=3).to(dev), [blocks[0], other])
    # K above the one-launch kernel's limit: per weight inside the library, same results.
    K2, N2 = 16416, 64
    big = [torch.from_numpy(ref.quantize_llama_rule(_weights(K2, N2, seed=20 + g).numpy())).to(dev)
           for g in range(2)]
    X2 = _acts(1, K2, seed=4).to(dev)
    for y, b in zip(mo.matmul_ggml_q4_0_grouped(X2, big), big):
        assert torch.equal(y.view(torch.int16), mo.matmul_ggml_q4_0(X2, b).view(torch.int16))
    # N == 0: empty outputs, as for one weight.
    empty = [torch.zeros((K // 32, 0, 18), dtype=torch.uint8, device=dev) for _ in range(2)]
    assert [tuple(y.shape) for y in mo.matmul_ggml_q4_0_grouped(_acts(1, K, seed=5).to(dev), empty)] == [(1, 0)] * 2


@pytest.mark.parametrize("M,K,N", [(1, 4096, 8192), (3, 2048, 8208), (6, 1024, 12288), (12, 4096, 16384),
                                   (4, 16384, 1024), (16, 8192, 4096), (1, 4096, 4096), (5, 4096, 4096),
                                   (24, 2048, 1024), (40, 1024, 2048), (300, 2048, 512), (512, 4096, 4096),
                                   (1024, 2048, 4096), (256, 1024, 40960)])
def test_matmul_capi_row_strides(dev, M, K, N):
    """The C entry point with row strides past K and N on both sides (ldx = K + 40,
    ldy = N + 24) across the decode and prefill kernels: outputs match the oracle
    and the padding columns of Y keep what was there."""
    from metalops_amd import _lib
    print(f"capi strided M={M} K={K} N={N}", flush=True)
    W = _weights(K, N, seed=M + K + 3 * N, outliers=True)
    blocks = ref.quantize_llama_rule(W.numpy())
    Xw = _acts(M, K + 40, seed=M + 5)
    Xd = Xw.to(dev)
    bd = torch.from_numpy(blocks).to(dev)
    ldy = N + 24
    Y = torch.full((M, ldy), 7.0, dtype=torch.float16, device=dev)
    need = _lib.lib.mcq4_matmul_workspace_bytes(M, K, N)
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)
    st = _lib.lib.mcq4_matmul_q4_0_f16(Xd.data_ptr(), K + 40, bd.data_ptr(), Y.data_ptr(), ldy, M, K, N,
                                       ws.data_ptr() if need else None, need,
                                       torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.lib.mcq4_last_error()
    torch.cuda.synchronize()
    Yc = Y.float().cpu().numpy()
    assert (Yc[:, N:] == 7.0).all()
    _check_rows(Yc[:, :N], ref.matmul_f32(Xw[:, :K].contiguous().numpy(), blocks))


@pytest.mark.parametrize("path", ["6", "7", "8"])
@pytest.mark.parametrize("M,K,N", [(300, 1056, 1024), (129, 2080, 2304)])
def test_prefill_tight_activation_storage(dev, monkeypatch, path, M, K, N):
    """Prefill kernels on activations whose storage ends at the last row's K-th
    element (row stride K + 40, no padding after the last row): the copies past a
    split's K range must stay inside that storage (reads past it return zero and
    feed no MFMA), and the outputs match the oracle."""
    from metalops_amd import _lib
    print(f"tight activations path={path} M={M} K={K} N={N}", flush=True)
    for k in ("MCQ4_GEMM_PATH", "MCQ4_GEMM6_SPLIT", "MCQ4_GEMM8_SPLIT", "MCQ4_XCD_LOCAL"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("MCQ4_GEMM_PATH", path)
    ldx = K + 40
    W = _weights(K, N, seed=M + K + N, outliers=True)
    blocks = ref.quantize_llama_rule(W.numpy())
    X = _acts(M, K, seed=M + 9)
    flat = torch.zeros((M - 1) * ldx + K, dtype=torch.float16)
    flat.as_strided((M, K), (ldx, 1)).copy_(X)
    Xd = flat.to(dev)
    bd = torch.from_numpy(blocks).to(dev)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    need = _lib.lib.mcq4_matmul_workspace_bytes(M, K, N)
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)
    st = _lib.lib.mcq4_matmul_q4_0_f16(Xd.data_ptr(), ldx, bd.data_ptr(), Y.data_ptr(), N, M, K, N,
                                       ws.data_ptr() if need else None, need,
                                       torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.lib.mcq4_last_error()
    torch.cuda.synchronize()
    _check_rows(Y.float().cpu().numpy(), ref.matmul_f32(X.numpy(), blocks))
