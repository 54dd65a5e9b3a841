"""CPU tests that pin the oracle (oracle/q4_0_ref.py and oracle/q4_0_ref.c).

The reference (packages/metalcore) ships no q4_0 tests or golden vectors, so the
oracle is pinned by what the mathematics and torch's documented semantics fix:
closed forms, known-answer blocks, invariants, an independent C restatement,
float64 brute force, and torch's own CPU arithmetic for the steps the reference
delegates to torch (divide, round, fp16 cast; quantization.py:338-352).
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import q4_0_ref as R


def _block_bytes(d: float, q):
    q = list(q)
    out = np.zeros(18, np.uint8)
    out[0:2] = np.array([d], np.float16).view(np.uint8)
    for i in range(16):
        out[2 + i] = q[2 * i] | (q[2 * i + 1] << 4)
    return out


# ---- dequantize ---------------------------------------------------------------

def test_dequant_exhaustive_nibble_scale_table():
    """Every nibble value 0..15 at every element position x a table of scales:
    W = (q - 8) * d exactly (closed form, quantization.py:412)."""
    scales = np.array([0.0, -0.0, 6e-8, -6e-8, 1.0, -1.0, 65504.0, -65504.0, 0.0123, -3.5],
                      np.float16)
    nb = 16
    blocks = np.zeros((nb, len(scales), 18), np.uint8)
    for kb in range(nb):
        for n, d in enumerate(scales):
            q = [(kb + j) % 16 for j in range(32)]
            blocks[kb, n] = _block_bytes(float(d), q)
    for deq in (R.dequantize, C.dequantize):
        W = deq(blocks, np.float32)
        for kb in range(nb):
            for n, d in enumerate(scales):
                for j in range(32):
                    want = np.float32(((kb + j) % 16) - 8) * np.float32(d)
                    assert W[kb * 32 + j, n].view(np.uint32) == np.float32(want).view(np.uint32)


def test_dequant_nibble_order_single_hot():
    """byte i = element 2i (low) | element 2i+1 (high) (quantization.py:364-367,
    quant_kernels.metal:1826-1829) -- not llama.cpp's j / j+16 order."""
    for j in (0, 1, 2, 15, 16, 17, 30, 31):
        q = [8] * 32
        q[j] = 15
        blk = _block_bytes(1.0, q)[None, None, :]
        W = R.dequantize(blk, np.float32)[:, 0]
        assert W[j] == 7.0 and np.count_nonzero(W) == 1
        byte = blk[0, 0, 2 + j // 2]
        assert (byte >> 4 if j % 2 else byte & 0xF) == 15


def test_dequant_fp16_is_one_rounding_of_exact_product():
    rng = np.random.default_rng(3)
    blocks = rng.integers(0, 256, (8, 50, 18), dtype=np.uint8)
    d = (rng.standard_normal((8, 50)) * 1e3).astype(np.float16)
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(8, 50, 2)
    w32 = R.dequantize(blocks, np.float32)
    w16 = R.dequantize(blocks, np.float16)
    np.testing.assert_array_equal(w16.view(np.uint16), w32.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(w16.view(np.uint16), C.dequantize(blocks, np.float16).view(np.uint16))


# ---- quantize (reference rule) ----------------------------------------------------

def test_quantize_ref_zero_block():
    """amax = 0 -> d = 1 (quantization.py:342): bytes 00 3C then 0x88 x16."""
    out = R.quantize_ref_rule(np.zeros((32, 1), np.float32))
    assert list(out[0, 0]) == [0x00, 0x3C] + [0x88] * 16
    np.testing.assert_array_equal(C.quantize_ref_rule(np.zeros((32, 1), np.float32)), out)


@pytest.mark.parametrize("j", [0, 1, 16, 31])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_quantize_ref_single_hot(j, sign):
    """One nonzero +a / -a: d = a/7, that element -> q = 15 / 1, all others 8."""
    a = np.float32(0.37)
    W = np.zeros((32, 1), np.float32)
    W[j, 0] = sign * a
    for quant in (R.quantize_ref_rule, C.quantize_ref_rule):
        out = quant(W)
        q, d = R.unpack_nibbles(out)
        assert d[0, 0] == np.float16(a / np.float32(7.0))
        want = np.full(32, 8)
        want[j] = 15 if sign > 0 else 1
        np.testing.assert_array_equal(q[0, 0], want)


def test_quantize_ref_ties_round_half_to_even():
    """amax = 7 makes d = 1 exactly, so x + 8 hits exact .5 ties; torch.round
    rounds them to even (8.5 -> 8, 9.5 -> 10, 6.5 -> 6, 14.5 -> 14)."""
    x = np.array([7.0, 0.5, 1.5, -0.5, -1.5, 2.5, -2.5, 6.5] + [0.0] * 24, np.float32)
    want = [15, 8, 10, 8, 6, 10, 6, 14] + [8] * 24
    for quant in (R.quantize_ref_rule, C.quantize_ref_rule):
        q, d = R.unpack_nibbles(quant(x[:, None]))
        assert d[0, 0] == 1.0
        assert list(q[0, 0]) == want


def test_quantize_ref_invariants_random():
    """q in [1, 15] for finite input, |x - deq| <= d/2 + |q-8|*|d - fp16(d)|."""
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((1024, 67)) * 0.02).astype(np.float32)
    W[rng.random(W.shape) < 0.01] *= 10
    out = R.quantize_ref_rule(W)
    q, dh = R.unpack_nibbles(out)
    assert q.min() >= 1 and q.max() <= 15
    amax = np.abs(W.reshape(32, 32, 67)).max(axis=1)
    d32 = amax / np.float32(7.0)
    deq = R.dequantize(out, np.float32).astype(np.float64)
    qq = q.transpose(0, 2, 1).reshape(1024, 67).astype(np.float64)
    d32e = np.repeat(d32, 32, axis=0).astype(np.float64)
    dhe = np.repeat(dh.astype(np.float64), 32, axis=0)
    bound = d32e / 2 + np.abs(qq - 8) * np.abs(d32e - dhe) + 1e-12
    assert (np.abs(W - deq) <= bound * (1 + 1e-6)).all()


def test_quantize_ref_matches_torch_cpu_semantics():
    """The steps the reference hands to torch (quantization.py:338-352) evaluated by
    torch itself on CPU agree with the numpy and C restatements bit for bit."""
    g = torch.Generator().manual_seed(11)
    W = torch.randn(512, 129, generator=g) * 0.02
    W[torch.rand(W.shape, generator=g) < 0.02] *= 10
    nb = 512 // 32
    wb = W.view(nb, 32, 129)
    d = wb.abs().amax(dim=1) / 7.0
    d = torch.where(d > 0, d, torch.ones_like(d))
    q = ((wb / d.unsqueeze(1)) + 8.0).round().clamp(0, 15).to(torch.uint8)
    q_t = q.permute(0, 2, 1)
    packed = (q_t[:, :, 0::2] | (q_t[:, :, 1::2] << 4)).numpy()
    dbytes = d.to(torch.float16).view(torch.uint8).view(nb, 129, 2).numpy()
    out = R.quantize_ref_rule(W.numpy())
    np.testing.assert_array_equal(out[:, :, 0:2], dbytes)
    np.testing.assert_array_equal(out[:, :, 2:], packed)
    np.testing.assert_array_equal(C.quantize_ref_rule(W.numpy()), out)


def _torch_reference_quantize(W: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """The reference's own steps (quantization.py:335-369) run by torch on CPU in
    W's dtype; returns (d bytes [nb, N, 2], packed nibbles [nb, N, 16])."""
    K, N = W.shape
    nb = K // 32
    wb = W.view(nb, 32, N)
    d = wb.abs().amax(dim=1) / 7.0
    d = torch.where(d > 0, d, torch.ones_like(d))
    q = ((wb / d.unsqueeze(1)) + 8.0).round().clamp(0, 15).to(torch.uint8)
    q_t = q.permute(0, 2, 1)
    packed = (q_t[:, :, 0::2] | (q_t[:, :, 1::2] << 4)).numpy()
    dbytes = d.to(torch.float16).contiguous().view(torch.uint8).view(nb, N, 2).numpy()
    return dbytes, packed


@pytest.mark.parametrize("tdtype,name", [(torch.float16, "float16"), (torch.bfloat16, "bfloat16")])
def test_quantize_ref_half_dtypes_match_torch(tdtype, name):
    """fp16 / bf16 weights: the reference rounds amax/7, x/d and +8 in the
    weight's dtype.  The oracle's per-step rounding equals torch's CPU ops in
    that dtype bit for bit -- on random data, on outliers, on tiny (subnormal
    range) blocks where amax/7 rounds to zero in fp16, and on blocks built so
    that x/d + 8 lands on exact half-way points in the dtype."""
    g = torch.Generator().manual_seed(23)
    K, N = 512, 67
    W = torch.randn(K, N, generator=g) * 0.02
    W[torch.rand(W.shape, generator=g) < 0.02] *= 10
    W[0:32, 0] = torch.randn(32, generator=g) * 1e-7          # fp16 subnormal range
    W[32:64, 1] = 0.0                                          # zero block -> d = 1
    # exact ties: amax = 7 * 2^-3 -> d = 2^-3, x = (k + 0.5) d -> x/d + 8 = k + 8.5
    W[64:96, 2] = torch.tensor([(k % 7 + 0.5) * 0.125 * (1 if k % 2 else -1) for k in range(32)])
    W[64, 2] = 0.875
    Wd = W.to(tdtype)
    dbytes, packed = _torch_reference_quantize(Wd)
    out = R.quantize_ref_rule(Wd.float().numpy(), name)
    np.testing.assert_array_equal(out[:, :, 0:2], dbytes)
    np.testing.assert_array_equal(out[:, :, 2:], packed)
    # and the dtype matters: the fp32 rule gives other bytes on this data
    assert not np.array_equal(R.quantize_ref_rule(Wd.float().numpy()), out)


def test_quantize_ref_bf16_scale_overflows_fp16():
    """A bf16 block with amax/7 beyond the fp16 range stores d = inf (the
    reference's d.to(float16)) while q is still computed with the finite bf16 d."""
    W = torch.zeros(32, 2, dtype=torch.bfloat16)
    W[:, 0] = 1e6
    W[3, 0] = -1e6
    W[:, 1] = torch.linspace(-3, 3, 32).to(torch.bfloat16)
    dbytes, packed = _torch_reference_quantize(W)
    out = R.quantize_ref_rule(W.float().numpy(), "bfloat16")
    np.testing.assert_array_equal(out[:, :, 0:2], dbytes)
    np.testing.assert_array_equal(out[:, :, 2:], packed)
    assert np.isinf(out[0, 0, 0:2].copy().view(np.float16)[0])


def test_quantize_rejects_bad_k():
    with pytest.raises(AssertionError, match="divisible by 32"):
        R.quantize_ref_rule(np.zeros((33, 2), np.float32))


# ---- quantize (llama.cpp rule, benchmark generator) -----------------------------

def test_quantize_llama_known_answers():
    x = np.zeros((32, 3), np.float32)
    x[4, 0] = -2.0      # max-signed element negative -> d = +0.25, that element -> q = 0
    x[7, 0] = 1.0
    x[9, 1] = 2.0       # positive max -> d = -0.25, element -> q = 0 as well
    for quant in (R.quantize_llama_rule, C.quantize_llama_rule):
        q, d = R.unpack_nibbles(quant(x))
        assert d[0, 0] == np.float16(0.25) and q[0, 0, 4] == 0 and q[0, 0, 7] == 12
        assert d[0, 1] == np.float16(-0.25) and q[0, 1, 9] == 0
        assert d[0, 2] == 0.0 and (q[0, 2] == 8).all()        # zero block: d = 0, q = 8
        assert q[0, 0, 0] == 8


def test_quantize_llama_first_max_wins_on_ties():
    x = np.zeros((32, 1), np.float32)
    x[3, 0] = 1.0
    x[10, 0] = -1.0     # same |x|, later: the first (+1) sets d = -1/8
    q, d = R.unpack_nibbles(R.quantize_llama_rule(x))
    assert d[0, 0] == np.float16(-0.125) and q[0, 0, 3] == 0 and q[0, 0, 10] == 15
    np.testing.assert_array_equal(C.quantize_llama_rule(x), R.quantize_llama_rule(x))


def test_quantize_llama_numpy_vs_c_random():
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((2048, 41)) * 0.02).astype(np.float32)
    mask = rng.random(W.shape) < 0.01
    W[mask] = (rng.standard_normal(int(mask.sum())) * 0.2).astype(np.float32)
    np.testing.assert_array_equal(R.quantize_llama_rule(W), C.quantize_llama_rule(W))
    np.testing.assert_array_equal(R.quantize_ref_rule(W), C.quantize_ref_rule(W))


# ---- matmul ---------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(1, 32, 1), (5, 64, 3), (17, 352, 33)])
def test_matmul_f32_vs_f64_bruteforce(M, K, N):
    rng = np.random.default_rng(M * K + N)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float16)
    blocks = R.quantize_ref_rule(W)
    y64 = R.matmul_f64(X, blocks)
    np.testing.assert_allclose(C.matmul_f64(X, blocks), y64, rtol=1e-12, atol=1e-12)
    y32 = R.matmul_f32(X, blocks)
    assert (np.abs(y32 - y64).max(axis=1) <= 1e-5 * np.abs(y64).max(axis=1) + 1e-12).all()


def test_matmul_linearity_in_x():
    rng = np.random.default_rng(1)
    blocks = R.quantize_llama_rule((rng.standard_normal((64, 5)) * 0.1).astype(np.float32))
    X1 = rng.integers(-4, 4, (2, 64)).astype(np.float16)
    X2 = rng.integers(-4, 4, (2, 64)).astype(np.float16)
    y = R.matmul_f64(X1, blocks) + R.matmul_f64(X2, blocks)
    np.testing.assert_allclose(R.matmul_f64((X1 + X2).astype(np.float16), blocks), y, rtol=1e-12)


def test_fallback_torch_cpu_matches_dequant_then_matmul():
    rng = np.random.default_rng(2)
    blocks = R.quantize_ref_rule((rng.standard_normal((128, 24)) * 0.02).astype(np.float32))
    X = rng.standard_normal((3, 128)).astype(np.float32)
    Y = R.fallback_torch_cpu(torch.from_numpy(X), torch.from_numpy(blocks)).numpy()
    np.testing.assert_allclose(Y, X @ R.dequantize(blocks, np.float32), rtol=1e-5, atol=1e-6)


def test_matmul_xdtype_against_torch_fallback():
    """The oracle's bf16 / fp32 path equals the reference fallback's steps run by
    torch on CPU (dequantize to X.dtype, then X @ W) within the output rounding."""
    g = torch.Generator().manual_seed(5)
    W = torch.randn(256, 40, generator=g) * 0.02
    blocks = R.quantize_ref_rule(W.numpy())
    for tdt, name, tol in ((torch.bfloat16, "bfloat16", 1e-2), (torch.float32, "float32", 1e-6)):
        X = torch.randn(3, 256, generator=g).to(tdt)
        want = R.fallback_torch_cpu(X, torch.from_numpy(blocks)).float().numpy()
        got = R.matmul_xdtype(X.float().numpy(), blocks, name)
        err = np.abs(got - want).max(axis=1)
        assert (err <= tol * np.abs(want).max(axis=1)).all()
    # a wrong weight rounding (fp32 W with bf16 X) is caught at a tighter bar than the output rounding
    X = torch.randn(2, 256, generator=g).to(torch.bfloat16)
    Wb = R.dequantize(blocks, np.float32)
    exact = X.float().numpy().astype(np.float64) @ Wb.astype(np.float64)
    ref_w = R.matmul_xdtype(X.float().numpy(), blocks, "bfloat16")
    assert np.abs(ref_w - exact).max() > 0
