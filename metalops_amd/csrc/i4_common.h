// Shared definitions for the gfx950 per-group INT4 kernels.
//
// Format (metalcore quantization.py:26-92): packed[K/2][N] uint8 with row k in
// byte row k/2 (even k in the low nibble, odd k in the high nibble);
// scales[G][N], zeros[G][N] (G = ceil(K/group)) in one float dtype;
// W[k][n] = (q - zeros[k/group][n]) * scales[k/group][n].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q4_common.h"

namespace mcq4 {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// dtype codes of the C ABI (MCQ4_DTYPE_*)
enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };
// fused activations of the matmul store
enum : int { ACT_NONE = 0, ACT_SILU = 1, ACT_GELU = 2 };

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Element i of a float array of dtype dt, upcast exactly to fp32.
__device__ __forceinline__ float load_dt(const void *p, int64_t i, int dt) {
    if (dt == DT_F32) return ((const float *)p)[i];
    if (dt == DT_F16) return (float)((const _Float16 *)p)[i];
    return bf16_bits_to_f32(((const uint16_t *)p)[i]);
}

// fp32 value rounded (nearest even) to dtype dt and returned as fp32.
__device__ __forceinline__ float round_dt(float x, int dt) {
    if (dt == DT_F32) return x;
    if (dt == DT_F16) return (float)(_Float16)x;
    return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

__device__ __forceinline__ void store_dt(void *p, int64_t i, float v, int dt) {
    if (dt == DT_F32) ((float *)p)[i] = v;
    else if (dt == DT_F16) ((_Float16 *)p)[i] = (_Float16)v;
    else ((uint16_t *)p)[i] = f32_to_bf16_bits(v);
}

// One output of the per-group INT4 (WB = 4, packed[K/2][N]) or INT8 (WB = 8,
// int8 [K][N]) product over K rows [k0, k1): sum of x[k] * (q - z) * s in fp32.
// The split-K recompute path of the XCD-local exchange (q4_common.h): slow,
// taken only when a split ran on another XCD.
__device__ __forceinline__ _Float16 rms_apply(_Float16 x, float rstd, _Float16 w);

// With NORM the row is the raw activation row of a fused RMSNorm: each element
// is normalised as the kernel normalised it (rms_apply with the row's rstd and
// the norm weight wn) before the product.
template <int WB, bool NORM = false>
__device__ __forceinline__ float i4_dot_range(const _Float16 *xrow, const uint8_t *P, const void *scales,
                                           const void *zeros, int sz_dt, int N, int gs, int n, int k0,
                                           int k1, const _Float16 *wn = nullptr, float rstd = 0.f) {
    float acc = 0.f;
    for (int k = k0; k < k1; ++k) {
        float q;
        if constexpr (WB == 4) q = (float)((P[(int64_t)(k >> 1) * N + n] >> (4 * (k & 1))) & 0xF);
        else q = (float)(int8_t)P[(int64_t)k * N + n];
        const int64_t gi = (int64_t)(k / gs) * N + n;
        const _Float16 x = NORM ? rms_apply(xrow[k], rstd, wn[k]) : xrow[k];
        acc += (float)x * ((q - load_dt(zeros, gi, sz_dt)) * load_dt(scales, gi, sz_dt));
    }
    return acc;
}

// Fused activations of native/quant_kernels.metal: SiLU y / (1 + exp(-y))
// (:996-998) and the tanh form of GELU (:1126-1132).
template <int ACT>
__device__ __forceinline__ float activate(float y) {
    if constexpr (ACT == ACT_SILU) {
        return y / (1.0f + expf(-y));
    } else if constexpr (ACT == ACT_GELU) {
        const float k0 = 0.7978845608028654f;   // sqrt(2/pi)
        return 0.5f * y * (1.0f + tanhf(k0 * (y + 0.044715f * y * y * y)));
    } else {
        return y;
    }
}

// RMSNorm of one activation row (native/training_kernels.metal:425-488):
// rstd = 1 / sqrt(sum(x^2) / K + eps) with the sum in fp32, and
// x_norm = fp16((x * rstd) * w).  Every kernel that normalises a row sums in the
// same order, so the fused and the two-kernel paths give identical bits:
// RMS_WAVES waves; thread t (= 64 wave + lane) adds the squares of the
// 8-element chunks t, t + 64 RMS_WAVES, ... (elements in order, fmaf), then
// tail element 8 (K / 8) + t; an xor butterfly over 32, 16, ..., 1 sums each
// wave's lanes (rms_sumsq_part); the wave totals are added in wave order
// (rms_sumsq_total).  vec16: x is 16-byte aligned (one 16-byte load per chunk).
constexpr int RMS_WAVES = 8;
__device__ __forceinline__ float rms_sumsq_part(const _Float16 *x, int K, int t, bool vec16) {
    float ss = 0.f;
    const int nc = K >> 3;
    for (int ch = t; ch < nc; ch += 64 * RMS_WAVES) {
        _Float16 v[8];
        if (vec16) {
            const half8_t h = *(const half8_t *)(x + 8 * ch);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = h[i];
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = x[8 * ch + i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = __builtin_fmaf((float)v[i], (float)v[i], ss);
    }
    if (8 * nc + t < K) {
        const float v = (float)x[8 * nc + t];
        ss = __builtin_fmaf(v, v, ss);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    return ss;
}
__device__ __forceinline__ float rms_sumsq_total(const float *wave_sums) {
    float ss = wave_sums[0];
#pragma unroll
    for (int w = 1; w < RMS_WAVES; ++w) ss += wave_sums[w];
    return ss;
}
__device__ __forceinline__ float rms_rstd(float ss, int K, float eps) {
    return 1.0f / sqrtf(ss / (float)K + eps);
}
// The product is rounded to fp32 and then to fp16, as the reference does.
// Without the canonicalize (a no-op on a product, no instruction) the backend
// folds the second multiply and the conversion into v_fma_mixlo_f16, which
// rounds once, straight to fp16 (1 ulp apart on about 2 elements in 10^4).
__device__ __forceinline__ _Float16 rms_apply(_Float16 x, float rstd, _Float16 w) {
    return (_Float16)__builtin_canonicalizef(((float)x * rstd) * (float)w);
}

}  // namespace mcq4
