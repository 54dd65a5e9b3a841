// q4_0 matmul with bf16 or fp32 activations: the reference's semantics for
// activations that are not fp16 (quantization.py:452-454, the path every
// non-fp16 X takes there): W = dequantize_ggml_q4_0(blocks, X.dtype), i.e. the
// exact fp32 product (q - 8)*d rounded once to X's dtype, then Y = X @ W with
// fp32 accumulation and one rounding of the sum to X's dtype.  bf16 x bf16
// products are exact in fp32, so only the summation order differs from torch.
//
// Not the hot path (the fp16 kernels are).  Workgroup = 32 columns x 8 K
// slices (256 threads); each thread owns one column and 8 rows and walks the
// K blocks slice, slice + 8, ...; the slices are summed through LDS in slice
// order (deterministic).  A column's block is read as nine 2-byte words (blocks
// are 18 bytes, so only 2-byte alignment holds), 32 lanes of a wave covering
// 576 contiguous bytes.
#include "i4_common.h"

namespace mcq4 {

constexpr int XA_COLS = 32, XA_SLICES = 8, XA_MR = 8;

struct XactArgs {
    const void *X;
    int x_dt;
    int64_t ldx;
    const uint8_t *W;
    void *Y;
    int64_t ldy;
    int64_t M, nb, N;
};

template <int DT>
__global__ void __launch_bounds__(256) q4_xact_kernel(XactArgs a) {
    __shared__ float red[XA_SLICES][XA_MR][XA_COLS];
    const int cx = threadIdx.x % XA_COLS, ks = threadIdx.x / XA_COLS;
    const int64_t n = (int64_t)blockIdx.x * XA_COLS + cx;
    const int64_t m0 = (int64_t)blockIdx.y * XA_MR;
    const int mr = (int)(a.M - m0 < XA_MR ? a.M - m0 : XA_MR);
    float acc[XA_MR];
#pragma unroll
    for (int i = 0; i < XA_MR; ++i) acc[i] = 0.f;
    if (n < a.N) {
        for (int64_t kb = ks; kb < a.nb; kb += XA_SLICES) {
            const uint16_t *b = (const uint16_t *)(a.W + (kb * a.N + n) * BLOCK_BYTES);
            const float d = (float)bitcast<_Float16>(b[0]);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t w4 = b[1 + i];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t k = kb * QK + 4 * i + e;
                    // exact in fp32 (|q-8| <= 8, d has 11 significant bits), then X's dtype
                    const float w = round_dt((float)((int)((w4 >> (4 * e)) & 0xF) - 8) * d, DT);
#pragma unroll
                    for (int r = 0; r < XA_MR; ++r)
                        if (r < mr) acc[r] += load_dt(a.X, (m0 + r) * a.ldx + k, DT) * w;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < XA_MR; ++r) red[ks][r][cx] = acc[r];
    __syncthreads();
    for (int v = threadIdx.x; v < XA_MR * XA_COLS; v += 256) {
        const int r = v / XA_COLS, c = v % XA_COLS;
        const int64_t nn = (int64_t)blockIdx.x * XA_COLS + c;
        if (r >= mr || nn >= a.N) continue;
        float sum = 0.f;
#pragma unroll
        for (int sl = 0; sl < XA_SLICES; ++sl) sum += red[sl][r][c];
        store_dt(a.Y, (m0 + r) * a.ldy + nn, sum, DT);
    }
}

hipError_t launch_q4_xact(const void *X, int x_dt, int64_t ldx, const uint8_t *W, void *Y,
                          int64_t ldy, int64_t M, int64_t K, int64_t N, hipStream_t s) {
    XactArgs a;
    a.X = X; a.x_dt = x_dt; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    const dim3 grid((unsigned)((N + XA_COLS - 1) / XA_COLS), (unsigned)((M + XA_MR - 1) / XA_MR));
    if (x_dt == DT_BF16) hipLaunchKernelGGL(q4_xact_kernel<DT_BF16>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(q4_xact_kernel<DT_F32>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mcq4
