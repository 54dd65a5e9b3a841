// Per-group INT4 quantize / dequantize kernels (exact rounding; compiled with
// -ffp-contract=off so no multiply-add is fused).
//
// quantize (quantization.py:49-92): one thread per (column, range of groups).
// For an even group size a range is one group: the group's rows start at an
// even row, so no packed byte is shared between threads.  For an odd group
// size one thread walks every group of its column.  Per group: pass 1 finds
// min/max, then scale = R(R(max - min) / 15) clamped to >= R(1e-8),
// zero = R(-min / scale), and pass 2 quantizes q = rne(R(R(w / scale) + zero))
// clamped to [0, 15] (NaN -> 0), where R rounds to the weight dtype (the
// reference runs each step as a torch op in that dtype).  Rows come in pairs:
// an even row's q waits in a register for the odd row, and the byte is stored
// once.  Loads and stores are coalesced across the threads (columns).
//
// The GPU-side quantizer quantize_to_int4 (native/quant_kernels.metal:634-686,
// binding core_mps.mm:4655-4700) is the same computation in fp32 with Metal's
// round() (half away from zero); `away` selects it.
//
// dequantize (quantization.py:139-151): one thread per packed byte:
// w = R_out(((float)q - zero) * scale) for its two rows.
#include <math.h>

#include "i4_common.h"

namespace mcq4 {

struct I4QuantArgs {
    const void *W;
    int w_dt;
    int64_t ldw, K, N, gs, G;
    int64_t gpt;               // groups per thread (1, or G for odd group sizes)
    int away;                  // 1: round half away from zero (Metal round()), 0: half to even
    uint8_t *packed;
    void *scales, *zeros;
};

__global__ void __launch_bounds__(256) i4_quantize_kernel(I4QuantArgs a) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= a.N) return;
    const int dt = a.w_dt;
    const float clamp_min = round_dt(1e-8f, dt);
    const int64_t nranges = (a.G + a.gpt - 1) / a.gpt;
    for (int64_t r = blockIdx.y; r < nranges; r += gridDim.y) {
        uint32_t pending = 0;
        const int64_t g_end = r * a.gpt + a.gpt < a.G ? r * a.gpt + a.gpt : a.G;
        for (int64_t g = r * a.gpt; g < g_end; ++g) {
            const int64_t k0 = g * a.gs;
            const int64_t k1 = k0 + a.gs < a.K ? k0 + a.gs : a.K;
            float mn = INFINITY, mx = -INFINITY;
            for (int64_t k = k0; k < k1; ++k) {
                const float w = load_dt(a.W, k * a.ldw + n, dt);
                mn = fminf(mn, w);
                mx = fmaxf(mx, w);
            }
            float scale = round_dt(round_dt(mx - mn, dt) / 15.0f, dt);
            scale = fmaxf(scale, clamp_min);
            const float zero = round_dt(-mn / scale, dt);
            store_dt(a.scales, g * a.N + n, scale, dt);
            store_dt(a.zeros, g * a.N + n, zero, dt);
            for (int64_t k = k0; k < k1; ++k) {
                const float w = load_dt(a.W, k * a.ldw + n, dt);
                const float t = round_dt(round_dt(w / scale, dt) + zero, dt);
                // rintf: half to even; roundf: half away from zero; fmaxf/fminf
                // map NaN to the bound 0.
                const float r = a.away ? roundf(t) : rintf(t);
                const uint32_t q = (uint32_t)fminf(fmaxf(r, 0.0f), 15.0f);
                if ((k & 1) == 0) {
                    pending = q;
                } else {
                    a.packed[(k >> 1) * a.N + n] = (uint8_t)(pending | (q << 4));
                }
            }
        }
    }
}

struct I4DequantArgs {
    const uint8_t *packed;
    const void *scales, *zeros;
    int sz_dt, out_dt;
    int64_t Kh, N, gs, ldo;
    void *out;
};

__global__ void __launch_bounds__(256) i4_dequant_kernel(I4DequantArgs a) {
    const int64_t total = a.Kh * a.N;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
        const int64_t kp = i / a.N, n = i - kp * a.N;
        const uint32_t b = a.packed[i];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t k = 2 * kp + h;
            const int64_t g = k / a.gs;
            const float s = load_dt(a.scales, g * a.N + n, a.sz_dt);
            const float z = load_dt(a.zeros, g * a.N + n, a.sz_dt);
            const float q = (float)((b >> (4 * h)) & 0xFu);
            const float w = (q - z) * s;
            store_dt(a.out, k * a.ldo + n, w, a.out_dt);
        }
    }
}

hipError_t launch_i4_quantize(const void *W, int w_dt, int64_t ldw, int64_t K, int64_t N,
                              int64_t gs, uint8_t *packed, void *scales, void *zeros,
                              hipStream_t s, int away) {
    I4QuantArgs a;
    a.away = away;
    a.W = W; a.w_dt = w_dt; a.ldw = ldw; a.K = K; a.N = N; a.gs = gs;
    a.G = (K + gs - 1) / gs;
    a.gpt = gs % 2 == 0 ? 1 : a.G;
    a.packed = packed; a.scales = scales; a.zeros = zeros;
    const int64_t nranges = (a.G + a.gpt - 1) / a.gpt;
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)(nranges < 65535 ? nranges : 65535));
    hipLaunchKernelGGL(i4_quantize_kernel, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_i4_dequant(const uint8_t *packed, const void *scales, const void *zeros,
                             int sz_dt, int64_t K, int64_t N, int64_t gs, void *out,
                             int64_t ldo, int out_dt, hipStream_t s) {
    I4DequantArgs a;
    a.packed = packed; a.scales = scales; a.zeros = zeros;
    a.sz_dt = sz_dt; a.out_dt = out_dt;
    a.Kh = K / 2; a.N = N; a.gs = gs; a.ldo = ldo; a.out = out;
    const int64_t total = a.Kh * N;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(i4_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mcq4
