// RMSNorm prologue of fused_rmsnorm_linear_int4 (native/core_mps.mm:3017-3103,
// RMSNorm kernel native/training_kernels.metal:425-488): per row of X (fp16,
// K elements) rstd = 1 / sqrt(sum(x^2) / K + eps) with the sum in fp32, and
// X_norm = fp16((x * rstd) * w) with w the fp16 norm weight.  One workgroup per
// row; the matmul that follows reads X_norm from the caller's workspace on the
// same stream.
#include "i4_common.h"

namespace mcq4 {

__global__ void __launch_bounds__(256)
i4_rmsnorm_kernel(const _Float16 *X, int64_t ldx, const _Float16 *w, float eps, int K,
                  _Float16 *out, int64_t ldo) {
    __shared__ float part[4];
    const int64_t row = blockIdx.x;
    const _Float16 *x = X + row * ldx;
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += 256) {
        const float v = (float)x[i];
        ss = __builtin_fmaf(v, v, ss);
    }
    // wave reduction (64 lanes), then the 4 waves in order
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = ((part[0] + part[1]) + part[2]) + part[3];
    const float rstd = 1.0f / sqrtf(total / (float)K + eps);
    _Float16 *o = out + row * ldo;
    for (int i = threadIdx.x; i < K; i += 256) o[i] = (_Float16)(((float)x[i] * rstd) * (float)w[i]);
}

hipError_t launch_i4_rmsnorm(const _Float16 *X, int64_t ldx, const _Float16 *w, float eps, int M,
                             int K, _Float16 *out, int64_t ldo, hipStream_t s) {
    hipLaunchKernelGGL(i4_rmsnorm_kernel, dim3(M), dim3(256), 0, s, X, ldx, w, eps, K, out, ldo);
    return hipGetLastError();
}

}  // namespace mcq4
