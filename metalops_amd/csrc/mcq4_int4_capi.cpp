// C ABI of the gfx950 per-group INT4 path: argument validation, status codes
// and dispatch.  No allocation, no exceptions; everything is enqueued on the
// caller's stream.
//
// Reference boundary replaced: metalcore's quantize_int4 / dequantize_int4 /
// matmul_int4 (quantization.py:26-239) and the pybind11 bindings
// matmul_int4_metal / matmul_int4_silu_metal / matmul_int4_gelu_metal
// (native/core_mps.mm:5612-5914, registered at :6935-6937): TORCH_CHECK
// failures become status codes, the Metal encode on the current MPS stream
// becomes a launch on the given HIP stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../include/mcq4.h"
#include "mcq4_options.h"

namespace mcq4 {
hipError_t launch_i4_quantize(const void *W, int w_dt, int64_t ldw, int64_t K, int64_t N,
                              int64_t gs, uint8_t *packed, void *scales, void *zeros,
                              hipStream_t s, int away);
hipError_t launch_i4_dequant(const uint8_t *packed, const void *scales, const void *zeros,
                             int sz_dt, int64_t K, int64_t N, int64_t gs, void *out,
                             int64_t ldo, int out_dt, hipStream_t s);
hipError_t launch_i4_generic(const void *X, int x_dt, int64_t ldx, const uint8_t *packed,
                             const void *scales, const void *zeros, int sz_dt, void *Y,
                             int64_t ldy, int64_t M, int64_t K, int64_t N, int64_t gs, int act,
                             hipStream_t s, int wb);
bool i4_gemv_supported(int64_t M, int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                       const void *P, const void *scales, const void *zeros, int wb);
size_t i4_gemv_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t gs, int wb);
bool i4_gemv1_supported(int64_t M, int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                        const void *P, const void *scales, const void *zeros, int wb);
hipError_t launch_i4_gemv(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                          const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K,
                          int N, int gs, int act, void *ws, hipStream_t s, int wb);
bool i4_gemm_supported(int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                       const void *P, const void *scales, const void *zeros, const void *Y,
                       int64_t ldy);
size_t i4_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N);
hipError_t launch_i4_gemm(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                          const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K,
                          int N, int gs, int act, void *ws, hipStream_t s, int wb);
hipError_t launch_i4_rmsnorm(const _Float16 *X, int64_t ldx, const _Float16 *w, float eps, int M,
                             int K, _Float16 *out, int64_t ldo, hipStream_t s);
bool i4_gemv1_rms_supported(int64_t K, int64_t N, int64_t gs, const void *X, const void *wn,
                            const void *P, const void *scales, const void *zeros);
hipError_t launch_i4_gemv1_rms(const _Float16 *X, const _Float16 *wn, float eps, const uint8_t *P,
                               const void *scales, const void *zeros, int sz_dt, _Float16 *Y, int K,
                               int N, int gs, void *ws, hipStream_t s);
// Records the message returned by mcq4_last_error (mcq4_capi.cpp); returns code.
int set_error(int code, const char *msg);
}  // namespace mcq4

namespace {

// The q4_0 C ABI keeps the per-thread message; this file reports through it.
int fail(int code, const char *fmt, ...);

constexpr int64_t kMaxDim = (int64_t)1 << 30;

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
bool valid_dt(int dt) { return dt == MCQ4_DTYPE_F32 || dt == MCQ4_DTYPE_F16 || dt == MCQ4_DTYPE_BF16; }
size_t dt_size(int dt) { return dt == MCQ4_DTYPE_F32 ? 4 : 2; }

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return MCQ4_OK;
    return fail(MCQ4_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int check_kng(int64_t K, int64_t N, int64_t gs) {
    if (K <= 0 || N <= 0) return fail(MCQ4_ERR_SHAPE, "K (%lld) and N (%lld) must be positive",
                                      (long long)K, (long long)N);
    if (K % 2) return fail(MCQ4_ERR_SHAPE, "K (%lld) must be even (two rows per byte)", (long long)K);
    if (gs <= 0) return fail(MCQ4_ERR_SHAPE, "group_size (%lld) must be positive", (long long)gs);
    if (K > kMaxDim || N > kMaxDim || (K / 2) * N > ((int64_t)1 << 40))
        return fail(MCQ4_ERR_SHAPE, "shape K=%lld N=%lld exceeds the supported size",
                    (long long)K, (long long)N);
    return MCQ4_OK;
}

// Matmul kernel choice: the MFMA kernels for fp16 activations in the shapes
// they take (GEMV for M <= 16, and for M <= 32 where the async-copy INT4 GEMV
// takes the shape; GEMM above), the general kernel otherwise.
// MCQ4_I4_PATH=generic forces the general kernel (tests, comparisons).
enum class I4Path { Generic, Gemv, Gemm };
I4Path i4_path(const void *X, int x_dt, int64_t ldx, const uint8_t *P, const void *s,
               const void *z, const void *Y, int64_t ldy, int64_t M, int64_t K, int64_t N,
               int64_t gs, int wb) {
    if (mcq4::opt_is("MCQ4_I4_PATH", 'g')) return I4Path::Generic;
    if (x_dt != MCQ4_DTYPE_F16) return I4Path::Generic;
    if (M <= 16) return mcq4::i4_gemv_supported(M, K, N, gs, X, ldx, P, s, z, wb) ? I4Path::Gemv
                                                                                  : I4Path::Generic;
    if (M <= 32 && wb == 4 && mcq4::i4_gemv1_supported(M, K, N, gs, X, ldx, P, s, z, wb)) return I4Path::Gemv;
    return mcq4::i4_gemm_supported(K, N, gs, X, ldx, P, s, z, Y, ldy) ? I4Path::Gemm
                                                                     : I4Path::Generic;
}

// Upper bound over the kernels a shape can take (the general kernel needs none).
size_t ws_bytes(int64_t M, int64_t K, int64_t N, int64_t gs, int x_dt, int wb = 4) {
    const int ks = wb == 4 ? 32 : 16;
    if (M <= 0 || K <= 0 || N <= 0 || gs <= 0 || K % ks || gs % ks || x_dt != MCQ4_DTYPE_F16)
        return 0;
    if (M <= 16) return mcq4::i4_gemv_workspace_bytes(M, K, N, gs, wb);
    if (K % 32 || gs % 32) return 0;
    // 17..32 rows take the GEMV or the GEMM depending on alignment: cover both.
    if (M <= 32 && wb == 4)
        return std::max(mcq4::i4_gemv_workspace_bytes(M, K, N, gs, wb), mcq4::i4_gemm_workspace_bytes(M, K, N));
    return mcq4::i4_gemm_workspace_bytes(M, K, N);
}

int matmul_common(int act, const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                  const void *scales, const void *zeros, int sz_dtype, void *Y, int64_t ldy,
                  int64_t M, int64_t K, int64_t N, int64_t gs, void *workspace,
                  size_t workspace_bytes, void *stream, int wb = 4) {
    if (!X || !packed || !scales || !zeros || !Y) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (!valid_dt(x_dtype) || !valid_dt(sz_dtype))
        return fail(MCQ4_ERR_INVALID_ARG, "x_dtype / sz_dtype must be MCQ4_DTYPE_F32, F16 or BF16");
    if (M <= 0 || M > kMaxDim) return fail(MCQ4_ERR_SHAPE, "M (%lld) out of range", (long long)M);
    if (wb == 4) {
        if (int st = check_kng(K, N, gs)) return st;
    } else if (K <= 0 || N <= 0 || gs <= 0 || K > kMaxDim || N > kMaxDim || K * N > ((int64_t)1 << 40)) {
        return fail(MCQ4_ERR_SHAPE, "K=%lld N=%lld group_size=%lld out of range", (long long)K,
                    (long long)N, (long long)gs);
    }
    if ((M + 7) / 8 > 65535) return fail(MCQ4_ERR_SHAPE, "M (%lld) too large", (long long)M);
    if (ldx < K) return fail(MCQ4_ERR_SHAPE, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
    if (ldy < N) return fail(MCQ4_ERR_SHAPE, "ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
    if (!aligned(X, dt_size(x_dtype)) || !aligned(Y, dt_size(x_dtype)))
        return fail(MCQ4_ERR_ALIGNMENT, "X and Y must be aligned to their element size");
    if (!aligned(scales, dt_size(sz_dtype)) || !aligned(zeros, dt_size(sz_dtype)))
        return fail(MCQ4_ERR_ALIGNMENT, "scales and zeros must be aligned to their element size");
    I4Path path = i4_path(X, x_dtype, ldx, packed, scales, zeros, Y, ldy, M, K, N, gs, wb);
    if (path == I4Path::Gemm && (K % 32 || gs % 32)) path = I4Path::Generic;
    const size_t need = path == I4Path::Generic ? 0 : ws_bytes(M, K, N, gs, x_dtype, wb);
    if (need && (!workspace || workspace_bytes < need))
        return fail(MCQ4_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                    workspace ? workspace_bytes : (size_t)0);
    if (need && !aligned(workspace, 16))
        return fail(MCQ4_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (path) {
        case I4Path::Gemv:
            e = mcq4::launch_i4_gemv((const _Float16 *)X, ldx, packed, scales, zeros, sz_dtype,
                                     (_Float16 *)Y, ldy, (int)M, (int)K, (int)N, (int)gs, act,
                                     workspace, st, wb);
            break;
        case I4Path::Gemm:
            e = mcq4::launch_i4_gemm((const _Float16 *)X, ldx, packed, scales, zeros, sz_dtype,
                                     (_Float16 *)Y, ldy, (int)M, (int)K, (int)N, (int)gs, act,
                                     workspace, st, wb);
            break;
        default:
            e = mcq4::launch_i4_generic(X, x_dtype, ldx, packed, scales, zeros, sz_dtype, Y, ldy,
                                        M, K, N, gs, act, st, wb);
            break;
    }
    return hip_status(e, "int4 matmul launch");
}

}  // namespace

extern "C" {

int mcq4_quantize_int4(const void *W, int w_dtype, int64_t ldw, int64_t K, int64_t N,
                       int64_t group_size, uint8_t *packed, void *scales, void *zeros,
                       void *stream) {
    fail(MCQ4_OK, "");
    if (!W || !packed || !scales || !zeros) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (!valid_dt(w_dtype))
        return fail(MCQ4_ERR_INVALID_ARG, "w_dtype must be MCQ4_DTYPE_F32, F16 or BF16");
    if (int st = check_kng(K, N, group_size)) return st;
    if (ldw < N) return fail(MCQ4_ERR_SHAPE, "ldw (%lld) < N (%lld)", (long long)ldw, (long long)N);
    const size_t es = dt_size(w_dtype);
    if (!aligned(W, es) || !aligned(scales, es) || !aligned(zeros, es))
        return fail(MCQ4_ERR_ALIGNMENT, "W, scales and zeros must be aligned to their element size");
    return hip_status(mcq4::launch_i4_quantize(W, w_dtype, ldw, K, N, group_size, packed, scales,
                                               zeros, (hipStream_t)stream, 0),
                      "int4 quantize launch");
}

int mcq4_quantize_to_int4(const float *W, int64_t ldw, int64_t K, int64_t N, int64_t group_size,
                          uint8_t *packed, float *scales, float *zeros, void *stream) {
    fail(MCQ4_OK, "");
    if (!W || !packed || !scales || !zeros) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (int st = check_kng(K, N, group_size)) return st;
    if (group_size % 2)
        return fail(MCQ4_ERR_SHAPE, "group_size (%lld) must be even", (long long)group_size);
    if (ldw < N) return fail(MCQ4_ERR_SHAPE, "ldw (%lld) < N (%lld)", (long long)ldw, (long long)N);
    if (!aligned(W, 4) || !aligned(scales, 4) || !aligned(zeros, 4))
        return fail(MCQ4_ERR_ALIGNMENT, "W, scales and zeros must be 4-byte aligned");
    return hip_status(mcq4::launch_i4_quantize(W, MCQ4_DTYPE_F32, ldw, K, N, group_size, packed,
                                               scales, zeros, (hipStream_t)stream, 1),
                      "quantize_to_int4 launch");
}

size_t mcq4_matmul_int8_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                        int x_dtype) {
    return ws_bytes(M, K, N, group_size, x_dtype, 8);
}

int mcq4_matmul_int8(const void *X, int x_dtype, int64_t ldx, const int8_t *W, const void *scales,
                     const void *zeros, int sz_dtype, void *Y, int64_t ldy, int64_t M, int64_t K,
                     int64_t N, int64_t group_size, void *workspace, size_t workspace_bytes,
                     void *stream) {
    fail(MCQ4_OK, "");
    return matmul_common(0, X, x_dtype, ldx, (const uint8_t *)W, scales, zeros, sz_dtype, Y, ldy,
                         M, K, N, group_size, workspace, workspace_bytes, stream, 8);
}

int mcq4_dequantize_int4(const uint8_t *packed, const void *scales, const void *zeros,
                         int sz_dtype, int64_t K, int64_t N, int64_t group_size, void *out,
                         int64_t ldo, int out_dtype, void *stream) {
    fail(MCQ4_OK, "");
    if (!packed || !scales || !zeros || !out) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (!valid_dt(sz_dtype) || !valid_dt(out_dtype))
        return fail(MCQ4_ERR_INVALID_ARG, "sz_dtype / out_dtype must be MCQ4_DTYPE_F32, F16 or BF16");
    if (int st = check_kng(K, N, group_size)) return st;
    if (ldo < N) return fail(MCQ4_ERR_SHAPE, "ldo (%lld) < N (%lld)", (long long)ldo, (long long)N);
    if (!aligned(scales, dt_size(sz_dtype)) || !aligned(zeros, dt_size(sz_dtype)) ||
        !aligned(out, dt_size(out_dtype)))
        return fail(MCQ4_ERR_ALIGNMENT, "scales, zeros and out must be aligned to their element size");
    return hip_status(mcq4::launch_i4_dequant(packed, scales, zeros, sz_dtype, K, N, group_size,
                                              out, ldo, out_dtype, (hipStream_t)stream),
                      "int4 dequantize launch");
}

size_t mcq4_matmul_int4_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                        int x_dtype) {
    return ws_bytes(M, K, N, group_size, x_dtype);
}

int mcq4_matmul_int4(const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                     const void *scales, const void *zeros, int sz_dtype, void *Y, int64_t ldy,
                     int64_t M, int64_t K, int64_t N, int64_t group_size, void *workspace,
                     size_t workspace_bytes, void *stream) {
    fail(MCQ4_OK, "");
    return matmul_common(0, X, x_dtype, ldx, packed, scales, zeros, sz_dtype, Y, ldy, M, K, N,
                         group_size, workspace, workspace_bytes, stream);
}

int mcq4_matmul_int4_silu(const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                          const void *scales, const void *zeros, int sz_dtype, void *Y,
                          int64_t ldy, int64_t M, int64_t K, int64_t N, int64_t group_size,
                          void *workspace, size_t workspace_bytes, void *stream) {
    fail(MCQ4_OK, "");
    return matmul_common(1, X, x_dtype, ldx, packed, scales, zeros, sz_dtype, Y, ldy, M, K, N,
                         group_size, workspace, workspace_bytes, stream);
}

int mcq4_matmul_int4_gelu(const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                          const void *scales, const void *zeros, int sz_dtype, void *Y,
                          int64_t ldy, int64_t M, int64_t K, int64_t N, int64_t group_size,
                          void *workspace, size_t workspace_bytes, void *stream) {
    fail(MCQ4_OK, "");
    return matmul_common(2, X, x_dtype, ldx, packed, scales, zeros, sz_dtype, Y, ldy, M, K, N,
                         group_size, workspace, workspace_bytes, stream);
}

// Workspace layout: the matmul's own workspace (its zero-filled 256 KiB counter
// area first, then split-K partials), then X_norm (M x K fp16) from
// max(matmul workspace, 256 KiB) on, so the counter area is never written with
// activations and one zero-filled buffer keeps serving every entry point.
constexpr size_t kCounterArea = (size_t)65536 * 4;
static size_t norm_offset(int64_t M, int64_t K, int64_t N, int64_t gs) {
    const size_t w = std::max(ws_bytes(M, K, N, gs, MCQ4_DTYPE_F16), kCounterArea);
    return (w + 255) / 256 * 256;
}

size_t mcq4_fused_rmsnorm_linear_int4_workspace_bytes(int64_t M, int64_t K, int64_t N,
                                                      int64_t group_size) {
    if (M <= 0 || K <= 0 || N <= 0 || group_size <= 0) return 0;
    return norm_offset(M, K, N, group_size) + (size_t)M * K * 2;
}

int mcq4_fused_rmsnorm_linear_int4(const void *X, int64_t ldx, const void *w_norm, float eps,
                                   const uint8_t *packed, const void *scales, const void *zeros,
                                   int sz_dtype, void *Y, int64_t ldy, int64_t M, int64_t K,
                                   int64_t N, int64_t group_size, void *workspace,
                                   size_t workspace_bytes, void *stream) {
    fail(MCQ4_OK, "");
    if (!X || !w_norm || !packed || !scales || !zeros || !Y)
        return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (M <= 0 || M > kMaxDim) return fail(MCQ4_ERR_SHAPE, "M (%lld) out of range", (long long)M);
    if (int st = check_kng(K, N, group_size)) return st;
    if (M > 65535 * 8) return fail(MCQ4_ERR_SHAPE, "M (%lld) too large", (long long)M);
    if (ldx < K) return fail(MCQ4_ERR_SHAPE, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
    if (!aligned(X, 2) || !aligned(w_norm, 2))
        return fail(MCQ4_ERR_ALIGNMENT, "X and w_norm must be 2-byte aligned (fp16)");
    const size_t need = mcq4_fused_rmsnorm_linear_int4_workspace_bytes(M, K, N, group_size);
    if (!workspace || workspace_bytes < need)
        return fail(MCQ4_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                    workspace ? workspace_bytes : (size_t)0);
    if (!aligned(workspace, 256)) return fail(MCQ4_ERR_ALIGNMENT, "workspace must be 256-byte aligned");
    // One row on the async-copy GEMV: the kernel normalises its own activations.
    if (M == 1 && mcq4::i4_gemv1_rms_supported(K, N, group_size, X, w_norm, packed, scales, zeros)) {
        if (!valid_dt(sz_dtype))
            return fail(MCQ4_ERR_INVALID_ARG, "sz_dtype must be MCQ4_DTYPE_F32, F16 or BF16");
        if (ldy < N) return fail(MCQ4_ERR_SHAPE, "ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
        if (!aligned(Y, 2)) return fail(MCQ4_ERR_ALIGNMENT, "X and Y must be aligned to their element size");
        if (!aligned(scales, dt_size(sz_dtype)) || !aligned(zeros, dt_size(sz_dtype)))
            return fail(MCQ4_ERR_ALIGNMENT, "scales and zeros must be aligned to their element size");
        return hip_status(mcq4::launch_i4_gemv1_rms((const _Float16 *)X, (const _Float16 *)w_norm, eps,
                                                     packed, scales, zeros, sz_dtype, (_Float16 *)Y,
                                                     (int)K, (int)N, (int)group_size, workspace,
                                                     (hipStream_t)stream),
                          "fused rmsnorm + int4 launch");
    }
    _Float16 *xn = (_Float16 *)((char *)workspace + norm_offset(M, K, N, group_size));
    if (int st = hip_status(mcq4::launch_i4_rmsnorm((const _Float16 *)X, ldx,
                                                    (const _Float16 *)w_norm, eps, (int)M, (int)K,
                                                    xn, K, (hipStream_t)stream),
                            "rmsnorm launch"))
        return st;
    // The matmul validates the rest (scales/zeros, Y, its own workspace share).
    return matmul_common(0, xn, MCQ4_DTYPE_F16, K, packed, scales, zeros, sz_dtype, Y, ldy, M, K,
                         N, group_size, workspace, norm_offset(M, K, N, group_size), stream);
}

}  // extern "C"

namespace {
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return mcq4::set_error(code, buf);
}
}  // namespace
