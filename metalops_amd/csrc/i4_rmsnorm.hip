// RMSNorm prologue of fused_rmsnorm_linear_int4 (native/core_mps.mm:3017-3103,
// RMSNorm kernel native/training_kernels.metal:425-488) where the matmul that
// follows cannot normalise its own activations (M > 1, or shapes the
// single-row async-copy GEMV does not take): X_norm = fp16((x * rstd) * w) per
// row into the caller's workspace, the matmul reading it next on the same
// stream.  One RMS_WAVES-wave workgroup per row, summing the squares in the
// order i4_common.h fixes (the fused GEMV's order), so both paths normalise to
// the same bits.
#include "i4_common.h"

namespace mcq4 {

__global__ void __launch_bounds__(64 * RMS_WAVES)
i4_rmsnorm_kernel(const _Float16 *X, int64_t ldx, const _Float16 *w, float eps, int K,
                  _Float16 *out, int64_t ldo) {
    __shared__ float part[RMS_WAVES];
    const int64_t row = blockIdx.x;
    const _Float16 *x = X + row * ldx;
    const float ss = rms_sumsq_part(x, K, threadIdx.x, ((uintptr_t)x % 16) == 0);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float rstd = rms_rstd(rms_sumsq_total(part), K, eps);
    _Float16 *o = out + row * ldo;
    for (int i = threadIdx.x; i < K; i += 64 * RMS_WAVES) o[i] = rms_apply(x[i], rstd, w[i]);
}

hipError_t launch_i4_rmsnorm(const _Float16 *X, int64_t ldx, const _Float16 *w, float eps, int M,
                             int K, _Float16 *out, int64_t ldo, hipStream_t s) {
    hipLaunchKernelGGL(i4_rmsnorm_kernel, dim3(M), dim3(64 * RMS_WAVES), 0, s, X, ldx, w, eps, K, out, ldo);
    return hipGetLastError();
}

}  // namespace mcq4
