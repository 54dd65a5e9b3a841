// Measurement probes for bench.py (libmcq4_bench.so); see mcq4_bench.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mcq4_bench.h"
#include "../q4_common.h"

namespace {

using mcq4::half8_t;
using mcq4::float16_t;
using mcq4::uint4_t;
using mcq4::bitcast;

constexpr int kOk = 0, kInvalid = 1, kHip = 5;
int hip_status() { return hipGetLastError() == hipSuccess ? kOk : kHip; }

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

// Workgroup (t, s) = (blockIdx.x % ntile, blockIdx.x / ntile) reads its tile's
// row range in 16-byte chunks, row-major, four loads in flight per thread.
template <int NW>
__global__ void __launch_bounds__(NW * 64)
read_tiles_kernel(const uint8_t *W, int nb, int64_t grow, int cpr, int ksplit, int ntile, uint32_t *sink) {
    const int t = blockIdx.x % ntile, s = blockIdx.x / ntile;
    const int r0 = (int)((int64_t)nb * s / ksplit), r1 = (int)((int64_t)nb * (s + 1) / ksplit);
    const int nq = (r1 - r0) * cpr;
    const uint8_t *base = W + (int64_t)r0 * grow + (int64_t)t * cpr * 16;
    uint32_t acc = 0;
    for (int q0 = threadIdx.x; q0 < nq; q0 += NW * 64 * 4) {
        uint4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * NW * 64;
            const int r = q / cpr, c = q - r * cpr;
            v[u] = q < nq ? __builtin_nontemporal_load((const uint4_t *)(base + r * grow + c * 16))
                          : uint4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

__global__ void empty_kernel() {}

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

__global__ void atomic_chain_kernel(int64_t *p, int iters, uint64_t *ticks) {
    if (threadIdx.x != 0) return;     // one lane: one atomic per step of the chain
    int64_t v = blockIdx.x;
    int64_t *a = p + (int64_t)blockIdx.x * 64;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i)   // each address depends on the previous result
        v = __hip_atomic_fetch_add(a + (v & 1), (int64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    ticks[blockIdx.x] = t1 - t0;
    if (v == -1) p[0] = 0;            // keeps the chain live
}

__device__ __forceinline__ uint32_t hw_xcc() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 7;
}

template <int SM, int LM>
__global__ void exchange_kernel(uint64_t *slots, uint64_t *out, int d, int polls) {
    const int wg = blockIdx.x;
    const int pair = wg % d + (wg / (2 * d)) * d;
    const bool producer = (wg / d) % 2 == 0;
    uint64_t *p = slots + pair * 16;
    uint64_t tw = 0, tr = 0, ok = 1;
    if (threadIdx.x == 0) {
        if (producer) {
            for (int i = 0; i < 200; ++i) __builtin_amdgcn_s_sleep(10);   // the consumer polls first
            const uint64_t v = 0x100000001ull * (uint64_t)(pair + 1);
            tw = __builtin_amdgcn_s_memrealtime();
            if (SM == 0) *p = v;
            else if (SM == 1) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else __builtin_nontemporal_store(v, p);
        } else {
            uint64_t w = 0;
            for (int it = 0; it < polls && !w; ++it) {
                if (LM == 0) {
                    const __amdgpu_buffer_rsrc_t rs =
                        __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, 8, 0x00020000);
                    w = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(rs, 0, 0, 1));
                } else {
                    w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            tr = __builtin_amdgcn_s_memrealtime();
            ok = w != 0;
        }
        out[wg * 4 + 0] = hw_xcc();
        out[wg * 4 + 1] = tw;
        out[wg * 4 + 2] = tr;
        out[wg * 4 + 3] = ok;
    }
}

}  // namespace

extern "C" int mcqb_read_probe(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (!src || !sink || bytes < 16 || ((uintptr_t)src & 15)) return kInvalid;
    const size_t n16 = bytes / 16, grid = (n16 + 1023) / 1024;
    if (grid > 0x7fffffffu) return kInvalid;
    hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint4_t *)src, n16, sink);
    return hip_status();
}

// Row pieces of piece_bytes of `rows` rows of row_bytes each, ksplit row ranges per
// piece column: the shared body of mcqb_read_tiles and mcqb_read_rows.
static int read_pieces(const void *W, int64_t rows, int64_t row_bytes, int64_t piece_bytes, int ksplit, int waves,
                       uint32_t *sink, void *stream) {
    if (!W || !sink || ((uintptr_t)W & 15) || rows < 1 || rows > 0x7fffffff || row_bytes < 16 || row_bytes % 16 ||
        piece_bytes < 16 || piece_bytes % 16 || row_bytes % piece_bytes || ksplit < 1 || ksplit > rows ||
        (row_bytes / piece_bytes) * ksplit > 0x7fffffff || rows * row_bytes / 16 > 0x7fffffff)
        return kInvalid;
    const int ntile = (int)(row_bytes / piece_bytes), grid = ntile * ksplit, cpr = (int)(piece_bytes / 16);
    const hipStream_t s = (hipStream_t)stream;
    const int nb = (int)rows;
    const int64_t grow = row_bytes;
    switch (waves) {
        case 4: hipLaunchKernelGGL(read_tiles_kernel<4>, dim3(grid), dim3(256), 0, s, (const uint8_t *)W, nb, grow, cpr, ksplit, ntile, sink); break;
        case 8: hipLaunchKernelGGL(read_tiles_kernel<8>, dim3(grid), dim3(512), 0, s, (const uint8_t *)W, nb, grow, cpr, ksplit, ntile, sink); break;
        case 16: hipLaunchKernelGGL(read_tiles_kernel<16>, dim3(grid), dim3(1024), 0, s, (const uint8_t *)W, nb, grow, cpr, ksplit, ntile, sink); break;
        default: return kInvalid;
    }
    return hip_status();
}

extern "C" int mcqb_read_tiles(const void *W, int64_t K, int64_t N, int tile_cols, int ksplit, int waves,
                               uint32_t *sink, void *stream) {
    if (K < 32 || K % 32 || N < 1 || tile_cols < 1 || (tile_cols * 18) % 16 || N % tile_cols || ksplit > K / 32)
        return kInvalid;
    return read_pieces(W, K / 32, N * 18, (int64_t)tile_cols * 18, ksplit, waves, sink, stream);
}

extern "C" int mcqb_read_rows(const void *W, int64_t rows, int64_t row_bytes, int64_t piece_bytes, int ksplit,
                              int waves, uint32_t *sink, void *stream) {
    return read_pieces(W, rows, row_bytes, piece_bytes, ksplit, waves, sink, stream);
}

extern "C" int mcqb_empty(int grid, int block, void *stream) {
    if (grid < 1 || block < 1 || block > 1024) return kInvalid;
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(block), 0, (hipStream_t)stream);
    return hip_status();
}

extern "C" int mcqb_measure_sclk(uint64_t *ticks, int iters, void *stream) {
    if (!ticks || iters <= 0) return kInvalid;
    hipLaunchKernelGGL(sclk_probe_kernel, dim3(SCLK_WGS), dim3(256), 0, (hipStream_t)stream, ticks, iters);
    return hip_status();
}

extern "C" int mcqb_atomic_chain(int64_t *p, int iters, int grid, uint64_t *ticks, void *stream) {
    if (!p || !ticks || iters <= 0 || grid < 1 || grid > 4096) return kInvalid;
    hipLaunchKernelGGL(atomic_chain_kernel, dim3(grid), dim3(64), 0, (hipStream_t)stream, p, iters, ticks);
    return hip_status();
}

extern "C" int mcqb_exchange(uint64_t *slots, uint64_t *out, int pair_stride, int store_mode, int load_mode,
                             int polls, void *stream) {
    if (!slots || !out || pair_stride < 1 || pair_stride > 128 || 256 % (2 * pair_stride) || store_mode < 0 ||
        store_mode > 2 || load_mode < 0 || load_mode > 1 || polls < 1)
        return kInvalid;
    const hipStream_t s = (hipStream_t)stream;
    const dim3 g(256), b(64);
#define MCQB_X(sm, lm) \
    if (store_mode == sm && load_mode == lm) hipLaunchKernelGGL((exchange_kernel<sm, lm>), g, b, 0, s, slots, out, pair_stride, polls);
    MCQB_X(0, 0) MCQB_X(0, 1) MCQB_X(1, 0) MCQB_X(1, 1) MCQB_X(2, 0) MCQB_X(2, 1)
#undef MCQB_X
    return hip_status();
}
