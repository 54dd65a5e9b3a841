"""CPU tests that pin the per-group INT4 oracle (oracle/int4_ref.py).

The reference ships no INT4 tests or golden vectors, so the oracle is pinned
by what the mathematics fixes: hand-computed dequant tables (with exact
rational arithmetic for the rounding order), exact ladders, ties, the
min -> 0 / max -> 15 property, the round-trip bound, float64 brute force for
the matmul, and torch's own CPU fp16/bf16 ops for the per-op rounding that
the reference inherits from running each step as a torch op
(quantization.py:69-83).
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import int4_ref as R


def _pack(q):
    q = np.asarray(q, np.uint8)
    return (q[0::2] | (q[1::2] << 4)).astype(np.uint8)


def _f32(x) -> float:
    """Round an exact rational to fp32 (via the correctly rounded double; f64 -> f32
    double rounding is harmless for one + or x of fp32 operands)."""
    return float(np.float32(float(x)))


# ---- dequantize ---------------------------------------------------------------

def test_dequant_exact_table():
    """Power-of-two scales and half-integer zeros: (q - z) * s exactly (quantization.py:151)."""
    K, N, gs = 32, 3, 16
    q = np.array([[(k + n) % 16 for n in range(N)] for k in range(K)], np.uint8)
    s = np.array([[0.25, 0.5, 2.0], [1.0, -0.125, 3.0]], np.float32)
    z = np.array([[2.5, 0.0, 7.0], [15.0, 1.5, -3.0]], np.float32)
    for out in (R.F32, R.F16, R.BF16):
        W = R.dequantize(_pack(q), s, z, gs, out)
        for k in range(K):
            for n in range(N):
                g = k // gs
                want = (Fraction(int(q[k, n])) - Fraction(float(z[g, n]))) * Fraction(float(s[g, n]))
                assert W[k, n] == float(want), (out, k, n)


def test_dequant_rounding_order():
    """fl(fl(q - z) * s): two fp32 roundings, subtraction first, then the cast.

    The expected values come from exact rationals rounded at the two points the
    reference rounds; at least one element differs from the q*s - z*s ordering,
    so the test sees a swapped formula.
    """
    K, N, gs = 16, 2, 16
    q = np.array([[k, 15 - k] for k in range(K)], np.uint8)
    s = np.array([[0.1, 3.3]], np.float32)
    z = np.array([[1.0 / 3.0, 7.77]], np.float32)
    W32 = R.dequantize(_pack(q), s, z, gs, R.F32)
    W16 = R.dequantize(_pack(q), s, z, gs, R.F16)
    differs = False
    for k in range(K):
        for n in range(N):
            d = _f32(Fraction(int(q[k, n])) - Fraction(float(z[0, n])))
            want = _f32(Fraction(d) * Fraction(float(s[0, n])))
            assert W32[k, n] == want
            assert W16[k, n] == float(np.float16(want))
            alt = np.float32(np.float32(q[k, n]) * s[0, n]) - np.float32(z[0, n] * s[0, n])
            differs |= bool(np.float32(alt) != np.float32(want))
    assert differs


def test_nibble_order_single_row():
    """Row k is byte row k // 2, low nibble for even k (quantization.py:85-90)."""
    for hot in range(4):
        w = np.zeros((4, 1), np.float32)
        w[hot, 0] = 1.0
        packed, s, z = R.quantize(w, 4)
        assert s[0, 0] == np.float32(1.0) / np.float32(15.0)
        expect = np.zeros((2, 1), np.uint8)
        expect[hot // 2, 0] = 0x0F if hot % 2 == 0 else 0xF0
        np.testing.assert_array_equal(packed, expect)
        assert R.unpack(packed)[hot, 0] == 15


# ---- quantize -----------------------------------------------------------------

@pytest.mark.parametrize("dtype", [R.F32, R.F16, R.BF16])
def test_quantize_exact_ladder(dtype):
    """min + i*step with power-of-two step: scale = step, zero = -min/step, q = i."""
    gs, N = 32, 5
    rng = np.random.default_rng(1)
    w = np.zeros((2 * gs, N), np.float32)
    qs = np.zeros_like(w, dtype=np.uint8)
    for g in range(2):
        for n in range(N):
            idx = rng.permutation(np.r_[np.arange(16), rng.integers(0, 16, gs - 16)])
            step = 2.0 ** -(3 + n)
            mn = -step * (2 + g + n)
            w[g * gs:(g + 1) * gs, n] = mn + idx * step
            qs[g * gs:(g + 1) * gs, n] = idx
    packed, s, z = R.quantize(w, gs, dtype)
    np.testing.assert_array_equal(R.unpack(packed), qs)
    for g in range(2):
        for n in range(N):
            assert s[g, n] == 2.0 ** -(3 + n)
            assert z[g, n] == 2 + g + n
    np.testing.assert_array_equal(R.dequantize(packed, s, z, gs, R.F32), w)


def test_quantize_ties_half_to_even():
    """w/scale + zero = k + 0.5 exactly rounds to the even neighbour (torch.round)."""
    w = np.array([0.0, 1.875, 0.0625, 0.1875, 0.3125, 0.4375, 0.5625, 1.8125], np.float32)
    packed, s, z = R.quantize(w[:, None], 8)
    assert s[0, 0] == 0.125 and z[0, 0] == 0.0
    np.testing.assert_array_equal(R.unpack(packed)[:, 0], [0, 15, 0, 2, 2, 4, 4, 14])


@pytest.mark.parametrize("dtype", [R.F32, R.F16, R.BF16])
@pytest.mark.parametrize("gs", [128, 64, 33, 3])
def test_quantize_min_max_and_bound(dtype, gs):
    """Every group's minimum quantizes to 0 and maximum to 15; every element
    dequantizes within scale/2 (+ a few ulps of the dtype's rounding steps)."""
    rng = np.random.default_rng(gs)
    K, N = 2 * 3 * gs if gs > 8 else 24, 7
    w = R.round_to(rng.normal(0, 1, (K, N)).astype(np.float32) * rng.uniform(0.01, 5, N), dtype)
    packed, s, z = R.quantize(w, gs, dtype)
    q = R.unpack(packed)
    deq = R.dequantize(packed, s, z, gs, R.F32)
    eps = {R.F32: 2.0 ** -23, R.F16: 2.0 ** -10, R.BF16: 2.0 ** -7}[dtype]
    for g in range(s.shape[0]):
        rows = slice(g * gs, min((g + 1) * gs, K))
        grp, qg = w[rows], q[rows]
        for n in range(N):
            assert qg[np.argmin(grp[:, n]), n] == 0
            assert qg[np.argmax(grp[:, n]), n] == 15
        err = np.abs(grp - deq[rows])
        bound = 0.5 * s[g] + 4 * eps * (np.abs(grp) + np.abs(z[g] * s[g]) + s[g])
        assert np.all(err <= bound)


def test_quantize_constant_group():
    """A constant group: scale clamps to fp32(1e-8), q = 0, dequant returns the value."""
    w = np.full((8, 2), 0.3, np.float32)
    w[:, 1] = 0.0
    packed, s, z = R.quantize(w, 8)
    assert np.all(s == np.float32(1e-8))
    np.testing.assert_array_equal(R.unpack(packed), 0)
    deq = R.dequantize(packed, s, z, 8, R.F32)
    np.testing.assert_allclose(deq[:, 0], 0.3, rtol=1e-6)
    np.testing.assert_array_equal(deq[:, 1], 0.0)
    # The clamp bound rounds to 0 in fp16 (below half the smallest subnormal),
    # to a nonzero value in bf16.
    assert R.round_to(np.float32(1e-8), R.F16) == 0.0
    assert 0.9e-8 < R.round_to(np.float32(1e-8), R.BF16) < 1.1e-8


def test_round_bf16_known_values():
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, 1.01171875, -2.5], np.float32)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7 (even: 1); 1 + 3*2^-8 is a tie
    # between 1 + 2^-7 and 1 + 2^-6 (even: 1 + 2^-6).
    np.testing.assert_array_equal(R.round_bf16(x), [1.0, 1.0, 1.0078125, 1.0078125, 1.015625, -2.5])
    # and agrees with torch's fp32 -> bf16 conversion on random bit patterns
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) < 3.0e38)]
    np.testing.assert_array_equal(R.round_bf16(v), torch.from_numpy(v).bfloat16().float().numpy())


@pytest.mark.parametrize("tdtype,dtype", [(torch.float16, R.F16), (torch.bfloat16, R.BF16),
                                          (torch.float32, R.F32)])
def test_quantize_per_op_rounding_matches_torch(tdtype, dtype):
    """The reference runs each step as a torch op in the weight dtype; torch's CPU
    ops on the same inputs give the oracle's scales, zeros and codes bit for bit."""
    gs, K, N = 32, 96, 33
    g = torch.Generator().manual_seed(7)
    wt = (torch.randn(K, N, generator=g) * torch.rand(N, generator=g) * 3).to(tdtype)
    ref_s, ref_z, ref_q = [], [], []
    for gi in range(K // gs):
        grp = wt[gi * gs:(gi + 1) * gs]
        mn, mx = grp.min(dim=0).values, grp.max(dim=0).values
        sc = ((mx - mn) / 15.0).clamp(min=1e-8)
        zr = -mn / sc
        ref_s.append(sc)
        ref_z.append(zr)
        ref_q.append((grp / sc + zr).round().clamp(0, 15).to(torch.uint8))
    packed, s, z = R.quantize(wt.float().numpy(), gs, dtype)
    np.testing.assert_array_equal(s, torch.stack(ref_s).float().numpy())
    np.testing.assert_array_equal(z, torch.stack(ref_z).float().numpy())
    np.testing.assert_array_equal(R.unpack(packed), torch.cat(ref_q).numpy())


# ---- matmul -------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N,gs", [(1, 32, 3, 16), (5, 96, 7, 64), (3, 24, 4, 3), (2, 64, 9, 128)])
def test_matmul_bruteforce(M, K, N, gs):
    rng = np.random.default_rng(M * K + N)
    w = rng.normal(0, 1, (K, N)).astype(np.float32)
    packed, s, z = R.quantize(w, gs)
    X = rng.normal(0, 1, (M, K)).astype(np.float32)
    np.testing.assert_allclose(R.matmul_f32(X, packed, s, z, gs),
                               R.matmul_f64(X, packed, s, z, gs), rtol=1e-5, atol=1e-5)


def test_matmul_batched_shape():
    rng = np.random.default_rng(3)
    packed, s, z = R.quantize(rng.normal(0, 1, (64, 8)).astype(np.float32), 32)
    X = rng.normal(0, 1, (2, 3, 64)).astype(np.float32)
    Y = R.matmul_f32(X, packed, s, z, 32)
    assert Y.shape == (2, 3, 8)
    np.testing.assert_allclose(Y[1], R.matmul_f64(X[1], packed, s, z, 32), rtol=1e-5, atol=1e-5)


# ---- RMSNorm prologue of fused_rmsnorm_linear_int4 ------------------------------

def test_rmsnorm_closed_forms():
    """Constant rows: x * rstd = c / sqrt(c^2 + eps); a zero row stays zero."""
    K = 64
    X = np.zeros((3, K), np.float16)
    X[0] = 2.0
    X[1] = -0.5
    w = np.full(K, 1.5, np.float16)
    got = R.rmsnorm_f16(X, w, 1e-6)
    assert np.all(got[2] == 0)
    for r, c in ((0, 2.0), (1, -0.5)):
        want = np.float16(c / np.sqrt(c * c + 1e-6) * 1.5)
        assert np.all(np.abs(got[r].astype(np.float32) - np.float32(want)) <= 2 ** -10 * 1.5)


def test_rmsnorm_matches_torch_functional():
    """torch.nn.functional.rms_norm in float64 (an independent implementation),
    rounded to fp16 once, agrees within one fp16 ulp."""
    rng = np.random.default_rng(0)
    X = (rng.normal(0, 1, (5, 256)) * rng.uniform(0.1, 10, (5, 1))).astype(np.float16)
    w = rng.normal(1, 0.1, 256).astype(np.float16)
    got = R.rmsnorm_f16(X, w, 1e-5).astype(np.float64)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(X.astype(np.float64)), (256,),
                                       torch.from_numpy(w.astype(np.float64)), eps=1e-5)
    ref = ref.numpy()
    ulp = np.abs(ref.astype(np.float16).astype(np.float64)) * 2.0 ** -10 + 2.0 ** -24
    assert np.all(np.abs(got - ref) <= ulp)


# ---- GPU-side quantizer rounding (quantize_to_int4) and INT8 --------------------

def test_quantize_away_rounding_ties():
    """quantize_to_int4 rounds half away from zero (Metal round()): with scale 0.125
    and zero 0 the codes of 0.5, 1.5, 2.5, 3.5 are 1, 2, 3, 4 (torch.round: 0, 2, 2, 4)."""
    w = np.array([0.0, 1.875, 0.0625, 0.1875, 0.3125, 0.4375, 0.5625, 1.8125], np.float32)
    packed, s, z = R.quantize(w[:, None], 8, rounding="away")
    np.testing.assert_array_equal(R.unpack(packed)[:, 0], [0, 15, 1, 2, 3, 4, 5, 15])
    # away and even agree everywhere except on exact ties
    rng = np.random.default_rng(2)
    w2 = rng.normal(0, 1, (256, 9)).astype(np.float32)
    pa = R.unpack(R.quantize(w2, 64, rounding="away")[0]).astype(int)
    pe = R.unpack(R.quantize(w2, 64)[0]).astype(int)
    assert np.all(np.abs(pa - pe) <= 1) and np.mean(pa != pe) < 0.01


def test_int8_dequant_known_answers():
    q = np.array([[-128, 127], [0, -1], [5, 100]], np.int8)
    s = np.array([[0.5, 2.0]], np.float32)
    z = np.array([[-2.0, 1.5]], np.float32)
    W = R.dequantize_int8(q, s, z, 4)
    np.testing.assert_array_equal(W, [[-63.0, 251.0], [1.0, -5.0], [3.5, 197.0]])


@pytest.mark.parametrize("M,K,N,gs", [(1, 32, 3, 16), (4, 48, 5, 32), (2, 20, 7, 3)])
def test_int8_matmul_bruteforce(M, K, N, gs):
    rng = np.random.default_rng(K + N)
    q = rng.integers(-128, 128, (K, N)).astype(np.int8)
    G = (K + gs - 1) // gs
    s = rng.uniform(0.001, 0.02, (G, N)).astype(np.float32)
    z = rng.uniform(-3, 3, (G, N)).astype(np.float32)
    X = rng.normal(0, 1, (M, K)).astype(np.float32)
    np.testing.assert_allclose(R.matmul_int8_f32(X, q, s, z, gs), R.matmul_int8_f64(X, q, s, z, gs),
                               rtol=1e-5, atol=1e-5)
