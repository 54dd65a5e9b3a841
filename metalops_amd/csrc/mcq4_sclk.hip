// Measurement helpers for the benchmark (no counterpart in the reference):
// the shader clock under an MFMA load, and a plain streaming read that gives
// the HBM read rate one launch of a given size can reach.
//
// Clock:
// 512 workgroups of 4 waves (two waves per SIMD) each run `iters` rounds of four
// independent v_mfma_f32_32x32x16_f16 chains on pseudo-random operands and
// record, per wave, the shader clock ticks (s_memtime) and the 100 MHz
// real-time ticks (s_memrealtime) the loop took.
// sclk = 100 MHz * d(memtime) / d(realtime).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mcq4.h"
#include "q4_common.h"

namespace mcq4 {

constexpr int SCLK_WGS = 512;

__global__ void __launch_bounds__(256, 2) sclk_probe_kernel(uint64_t *ticks, int iters) {
    const int lane = threadIdx.x & 63;
    // Fresh pseudo-random operands every round (xorshift32 per lane, each half
    // masked to a finite value in [0, 2)): the clock under the power limit
    // depends on how many operand bits toggle, and random data is what a GEMM
    // on real weights and activations sees.
    uint32_t x = 0x9E3779B9u * (uint32_t)(threadIdx.x + 1) + 0x632BE5ABu * (uint32_t)blockIdx.x;
    constexpr uint32_t FIN = 0x3FFF3FFFu;
    float16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        const uint32_t y = x * 0x2545F491u;
        const half8_t a = bitcast<half8_t>(uint4_t{x & FIN, __builtin_amdgcn_alignbit(x, x, 8) & FIN,
                                                   __builtin_amdgcn_alignbit(x, x, 16) & FIN,
                                                   __builtin_amdgcn_alignbit(x, x, 24) & FIN});
        const half8_t b = bitcast<half8_t>(uint4_t{y & FIN, __builtin_amdgcn_alignbit(y, y, 8) & FIN,
                                                   __builtin_amdgcn_alignbit(y, y, 16) & FIN,
                                                   __builtin_amdgcn_alignbit(y, y, 24) & FIN});
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    const float keep = c0[0] + c1[1] + c2[2] + c3[3];   // keeps the chains live
    if (lane == 0) {
        ticks[2 * w] = t1 - t0 + (keep == -1.0f ? 1u : 0u);
        ticks[2 * w + 1] = r1 - r0;
    }
}

// Plain read: workgroup b of 256 threads reads the 16 KiB at 16384 b (four
// 16-byte loads per thread, all issued before any is used), XORs them and
// stores only if the XOR hits a magic value (so the loads stay live).
__global__ void __launch_bounds__(256) read_probe_kernel(const uint4_t *p, size_t n16, uint32_t *sink) {
    const size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x;
    uint4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const size_t i = base + 256 * u;
        v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : uint4_t{0u, 0u, 0u, 0u};
    }
    uint32_t s = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) s ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    if (s == 0x9E3779B9u) sink[0] = s;
}

}  // namespace mcq4

extern "C" int mcq4_read_probe(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (!src || !sink || bytes < 16 || ((uintptr_t)src & 15)) return MCQ4_ERR_INVALID_ARG;
    const size_t n16 = bytes / 16;
    const size_t grid = (n16 + 1023) / 1024;
    if (grid > 0x7fffffffu) return MCQ4_ERR_SHAPE;
    hipLaunchKernelGGL(mcq4::read_probe_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const mcq4::uint4_t *)src, n16, sink);
    return hipGetLastError() == hipSuccess ? MCQ4_OK : MCQ4_ERR_HIP;
}

extern "C" int mcq4_measure_sclk(uint64_t *ticks, int iters, void *stream) {
    if (!ticks || iters <= 0) return MCQ4_ERR_INVALID_ARG;
    hipLaunchKernelGGL(mcq4::sclk_probe_kernel, dim3(mcq4::SCLK_WGS), dim3(256), 0, (hipStream_t)stream,
                       ticks, iters);
    return hipGetLastError() == hipSuccess ? MCQ4_OK : MCQ4_ERR_HIP;
}
