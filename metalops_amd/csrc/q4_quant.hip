// block_q4_0 quantize / dequantize kernels for gfx950.
//
// One thread owns one block (kb, n): it reads the 32 weights of column n in
// rows kb*32 .. kb*32+31 (coalesced across the wave along n) and writes the 18
// block bytes with 2-byte stores.  These are one-time conversion kernels; the
// hot path is the matmul.
#include "i4_common.h"

namespace mcq4 {

// Rounds an fp32 value to fp16 (nearest even) with its sign of zero intact.
// The empty asm keeps the compiler from folding the preceding fp32 multiply and
// this conversion into v_fma_mix*_f16 with a +0 addend, which turns -0 into +0.
__device__ __forceinline__ _Float16 to_half_exact(float v) {
    asm volatile("" : "+v"(v));
    return (_Float16)v;
}

// Reference rule, quantization.py:333-369, for a weight of dtype DT (fp32,
// fp16 or bf16).  The reference runs every step as a torch op on the weight's
// own dtype, so each step here is one fp32 IEEE operation (the file is
// compiled with -ffp-contract=off, and '/' is the correctly rounded divide)
// followed by a rounding to DT: amax (exact), amax/7, x/d, +8, round half to
// even (rintf, exact in DT), clamp.  For fp16 and bf16 the fp32 result rounded
// to DT equals the correctly rounded DT operation (fp32 carries more than
// 2p + 2 bits for both, so the double rounding is innocuous).  d is stored as
// fp16 (d.to(float16), quantization.py:352), one more rounding for bf16.
template <int DT>
__global__ void __launch_bounds__(256)
quantize_ref_kernel(const void *__restrict__ W, int64_t ldw, int nb, int N,
                    uint8_t *__restrict__ out) {
#pragma clang fp contract(off)
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const int kb = blockIdx.y;
    if (n >= N || kb >= nb) return;
    const int64_t base = (int64_t)kb * QK * ldw + n;
    float x[QK];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        x[j] = load_dt(W, base + (int64_t)j * ldw, DT);
        amax = fmaxf(amax, fabsf(x[j]));
    }
    float d = round_dt(amax / 7.0f, DT);
    d = (d > 0.0f) ? d : 1.0f;
    uint32_t q[QK];
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        const float t = round_dt(round_dt(x[j] / d, DT) + 8.0f, DT);
        float r = __builtin_rintf(t);
        r = fminf(fmaxf(r, 0.0f), 15.0f);
        q[j] = (uint32_t)r;
    }
    uint16_t *dst = (uint16_t *)(out + ((int64_t)kb * N + n) * BLOCK_BYTES);
    dst[0] = bitcast<uint16_t>(to_half_exact(d));
#pragma unroll
    for (int i = 0; i < 8; ++i)
        dst[1 + i] = (uint16_t)(q[4 * i] | (q[4 * i + 1] << 4) | (q[4 * i + 2] << 8) |
                                (q[4 * i + 3] << 12));
}

// llama.cpp quantize_row_q4_0_ref rule in the same layout: d = max_signed / -8,
// id = 1/d (0 if d == 0), q = min(15, trunc(x*id + 8.5)).
__global__ void __launch_bounds__(256)
quantize_llama_kernel(const float *__restrict__ W, int64_t ldw, int nb, int N,
                      uint8_t *__restrict__ out) {
#pragma clang fp contract(off)
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const int kb = blockIdx.y;
    if (n >= N || kb >= nb) return;
    const float *src = W + (int64_t)kb * QK * ldw + n;
    float x[QK];
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        x[j] = src[(int64_t)j * ldw];
        if (amax < fabsf(x[j])) { amax = fabsf(x[j]); mx = x[j]; }
    }
    const float d = mx / -8.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint32_t q[QK];
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        float t = x[j] * id;   // two roundings: this file is built with -ffp-contract=off
        t = t + 8.5f;
        int v = (int)__builtin_truncf(t);
        v = v < 0 ? 0 : v;  // x*id >= -8 keeps t >= 0.5; guards non-finite input
        q[j] = (uint32_t)(v < 15 ? v : 15);
    }
    uint16_t *dst = (uint16_t *)(out + ((int64_t)kb * N + n) * BLOCK_BYTES);
    dst[0] = bitcast<uint16_t>(to_half_exact(d));
#pragma unroll
    for (int i = 0; i < 8; ++i)
        dst[1 + i] = (uint16_t)(q[4 * i] | (q[4 * i + 1] << 4) | (q[4 * i + 2] << 8) |
                                (q[4 * i + 3] << 12));
}

// quantization.py:396-419: W = (q - 8) * d, exact in fp32; the fp16 variant
// rounds that exact product once (nearest even).
template <typename OutT>
__global__ void __launch_bounds__(256)
dequant_kernel(const uint8_t *__restrict__ blocks, int nb, int N, OutT *__restrict__ out,
               int64_t ldo) {
#pragma clang fp contract(off)
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const int kb = blockIdx.y;
    if (n >= N || kb >= nb) return;
    const uint16_t *b = (const uint16_t *)(blocks + ((int64_t)kb * N + n) * BLOCK_BYTES);
    const float d = (float)bitcast<_Float16>(b[0]);
    OutT *dst = out + (int64_t)kb * QK * ldo + n;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t w = b[1 + i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = (float)((int)((w >> (4 * e)) & 0xF) - 8) * d;
            if constexpr (sizeof(OutT) == 2)
                dst[(int64_t)(4 * i + e) * ldo] = to_half_exact(v);
            else
                dst[(int64_t)(4 * i + e) * ldo] = v;
        }
    }
}

}  // namespace mcq4

// ---- launchers (called from the C ABI layer) -------------------------------
namespace mcq4 {

hipError_t launch_quantize(bool llama_rule, const float *W, int64_t ldw, int nb, int N,
                           uint8_t *out, hipStream_t s) {
    dim3 grid((N + 255) / 256, nb), block(256);
    if (llama_rule)
        hipLaunchKernelGGL(quantize_llama_kernel, grid, block, 0, s, W, ldw, nb, N, out);
    else
        hipLaunchKernelGGL(quantize_ref_kernel<DT_F32>, grid, block, 0, s, (const void *)W, ldw, nb, N, out);
    return hipGetLastError();
}

hipError_t launch_quantize_typed(int w_dtype, const void *W, int64_t ldw, int nb, int N,
                                 uint8_t *out, hipStream_t s) {
    dim3 grid((N + 255) / 256, nb), block(256);
    if (w_dtype == DT_F16)
        hipLaunchKernelGGL(quantize_ref_kernel<DT_F16>, grid, block, 0, s, W, ldw, nb, N, out);
    else if (w_dtype == DT_BF16)
        hipLaunchKernelGGL(quantize_ref_kernel<DT_BF16>, grid, block, 0, s, W, ldw, nb, N, out);
    else
        hipLaunchKernelGGL(quantize_ref_kernel<DT_F32>, grid, block, 0, s, W, ldw, nb, N, out);
    return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t *blocks, int nb, int N, void *out, int64_t ldo,
                          bool f16, hipStream_t s) {
    dim3 grid((N + 255) / 256, nb), block(256);
    if (f16)
        hipLaunchKernelGGL(dequant_kernel<_Float16>, grid, block, 0, s, blocks, nb, N,
                           (_Float16 *)out, ldo);
    else
        hipLaunchKernelGGL(dequant_kernel<float>, grid, block, 0, s, blocks, nb, N,
                           (float *)out, ldo);
    return hipGetLastError();
}

}  // namespace mcq4

// ---- workspace counter area -------------------------------------------------
namespace mcq4 {

// Zero-fills `n16` 16-byte words (a kernel rather than hipMemsetAsync, so the
// call can sit in a captured HIP graph).
__global__ void __launch_bounds__(256) zero16_kernel(uint4_t *p, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n16) p[i] = uint4_t{0u, 0u, 0u, 0u};
}

hipError_t launch_zero_counters(void *ws, hipStream_t s) {
    const int64_t n16 = (int64_t)COUNTER_BYTES / 16;
    hipLaunchKernelGGL(zero16_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, s, (uint4_t *)ws, n16);
    return hipGetLastError();
}

}  // namespace mcq4
