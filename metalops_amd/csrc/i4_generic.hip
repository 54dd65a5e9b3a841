// General per-group INT4 / INT8 matmul: any activation dtype (fp32 / fp16 /
// bf16), any group size, any N, even K (INT4).  This is the path for shapes and
// dtypes the MFMA kernels do not take (not the hot path).
//
// Semantics follow quantization.py:207-239 (INT4) and :268-286 (INT8): the
// weight is dequantized as ((float)q - zero) * scale in fp32 and rounded to X's
// dtype (the reference builds W in X.dtype), then Y = X @ W with fp32
// accumulation, the fused activation applied to the fp32 sum, and one rounding
// to X's dtype.
//
// Workgroup = 32 columns x 8 K slices (256 threads); each thread accumulates 8
// rows of its column over its slice's byte rows (kp = slice, slice + 8, ...:
// the 8 slices of a wave pair read neighbouring rows), then the 8 slices are
// summed through LDS in slice order (deterministic).
#include "i4_common.h"

namespace mcq4 {

constexpr int GN_COLS = 32, GN_SLICES = 8, GN_MR = 8;

struct I4GenericArgs {
    const void *X;
    int x_dt;
    int64_t ldx;
    const uint8_t *packed;
    const void *scales, *zeros;
    int sz_dt;
    void *Y;
    int64_t ldy;
    int64_t M, K, N, gs;
};

// WB = weight bits: 4 (packed[K/2][N], two rows per byte) or 8 (int8 [K][N]).
template <int ACT, int WB>
__global__ void __launch_bounds__(256) i4_generic_kernel(I4GenericArgs a) {
    __shared__ float red[GN_SLICES][GN_MR][GN_COLS];
    const int cx = threadIdx.x % GN_COLS, ks = threadIdx.x / GN_COLS;
    const int64_t n = (int64_t)blockIdx.x * GN_COLS + cx;
    const int64_t m0 = (int64_t)blockIdx.y * GN_MR;
    const int mr = (int)(a.M - m0 < GN_MR ? a.M - m0 : GN_MR);
    float acc[GN_MR];
#pragma unroll
    for (int i = 0; i < GN_MR; ++i) acc[i] = 0.f;
    if (n < a.N) {
        int64_t gcur = -1;
        float s = 0.f, z = 0.f;
        constexpr int RPB = WB == 4 ? 2 : 1;           // K rows per stored byte row
        for (int64_t kp = ks; kp < a.K / RPB; kp += GN_SLICES) {
            const uint32_t b = a.packed[kp * a.N + n];
#pragma unroll
            for (int h = 0; h < RPB; ++h) {
                const int64_t k = RPB * kp + h;
                const int64_t g = k / a.gs;
                if (g != gcur) {
                    gcur = g;
                    s = load_dt(a.scales, g * a.N + n, a.sz_dt);
                    z = load_dt(a.zeros, g * a.N + n, a.sz_dt);
                }
                const float q = WB == 4 ? (float)((b >> (4 * h)) & 0xFu) : (float)(int8_t)b;
                const float w = round_dt((q - z) * s, a.x_dt);
#pragma unroll
                for (int i = 0; i < GN_MR; ++i)
                    if (i < mr) acc[i] += load_dt(a.X, (m0 + i) * a.ldx + k, a.x_dt) * w;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < GN_MR; ++i) red[ks][i][cx] = acc[i];
    __syncthreads();
    for (int v = threadIdx.x; v < GN_MR * GN_COLS; v += 256) {
        const int i = v / GN_COLS, c = v % GN_COLS;
        const int64_t nn = (int64_t)blockIdx.x * GN_COLS + c;
        if (i >= mr || nn >= a.N) continue;
        float sum = 0.f;
#pragma unroll
        for (int sl = 0; sl < GN_SLICES; ++sl) sum += red[sl][i][c];
        store_dt(a.Y, (m0 + i) * a.ldy + nn, activate<ACT>(sum), a.x_dt);
    }
}

template <int WB>
static void launch_generic_wb(const I4GenericArgs &a, dim3 grid, int act, hipStream_t s) {
    if (act == ACT_SILU) hipLaunchKernelGGL((i4_generic_kernel<ACT_SILU, WB>), grid, dim3(256), 0, s, a);
    else if (act == ACT_GELU) hipLaunchKernelGGL((i4_generic_kernel<ACT_GELU, WB>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((i4_generic_kernel<ACT_NONE, WB>), grid, dim3(256), 0, s, a);
}

hipError_t launch_i4_generic(const void *X, int x_dt, int64_t ldx, const uint8_t *packed,
                             const void *scales, const void *zeros, int sz_dt, void *Y,
                             int64_t ldy, int64_t M, int64_t K, int64_t N, int64_t gs, int act,
                             hipStream_t s, int wb) {
    I4GenericArgs a;
    a.X = X; a.x_dt = x_dt; a.ldx = ldx; a.packed = packed; a.scales = scales; a.zeros = zeros;
    a.sz_dt = sz_dt; a.Y = Y; a.ldy = ldy; a.M = M; a.K = K; a.N = N; a.gs = gs;
    const dim3 grid((unsigned)((N + GN_COLS - 1) / GN_COLS), (unsigned)((M + GN_MR - 1) / GN_MR));
    if (wb == 8) launch_generic_wb<8>(a, grid, act, s);
    else launch_generic_wb<4>(a, grid, act, s);
    return hipGetLastError();
}

}  // namespace mcq4
