// C ABI of the gfx950 q4_0 path: argument validation, status codes and
// dispatch to the kernel launchers.  No allocation, no exceptions; everything
// is enqueued on the caller's stream.
//
// Reference boundary replaced: metalcore's pybind11 binding
// matmul_ggml_q4_0_metal (native/core_mps.mm:5917-5975): shape/dtype checks
// (core_mps.mm:5923-5938) become status codes, the Metal encode on the current
// MPS stream (core_mps.mm:5947-5969) becomes a launch on the given HIP stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/mcq4.h"
#include "q4_prefill.h"

namespace mcq4 {
hipError_t launch_quantize(bool llama_rule, const float *W, int64_t ldw, int nb, int N,
                           uint8_t *out, hipStream_t s);
hipError_t launch_dequant(const uint8_t *blocks, int nb, int N, void *out, int64_t ldo,
                          bool f16, hipStream_t s);
size_t skinny_workspace_bytes(int64_t M, int64_t K, int64_t N);
hipError_t launch_skinny(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                         int64_t ldy, int M, int K, int N, void *ws, hipStream_t s);
size_t gemm_workspace_bytes(int64_t M, int64_t K, int64_t N);
hipError_t launch_gemm(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                       int64_t ldy, int M, int K, int N, void *ws, hipStream_t s);
bool gemm2_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t K, int64_t N);
hipError_t launch_gemm2(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, hipStream_t s);
hipError_t launch_quantize_typed(int w_dtype, const void *W, int64_t ldw, int nb, int N,
                                 uint8_t *out, hipStream_t s);
hipError_t launch_zero_counters(void *ws, hipStream_t s);
size_t gemm7_workspace_bytes(int64_t M, int64_t K, int64_t N);
bool gemm7_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N);
hipError_t launch_gemm7(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s);
hipError_t q4_gemvm_split_fallbacks(uint64_t *count, bool reset);
hipError_t q4_gemm6_split_fallbacks(uint64_t *count, bool reset);
hipError_t i4_gemv_split_fallbacks(uint64_t *count, bool reset);
hipError_t i4_gemv1_split_fallbacks(uint64_t *count, bool reset);
hipError_t i4_gemm6_split_fallbacks(uint64_t *count, bool reset);
hipError_t q4_gemv_span_split_fallbacks(uint64_t *count, bool reset);
hipError_t q4_gemm8_split_fallbacks(uint64_t *count, bool reset);
hipError_t launch_q4_xact(const void *X, int x_dt, int64_t ldx, const uint8_t *W, void *Y,
                          int64_t ldy, int64_t M, int64_t K, int64_t N, hipStream_t s);
bool gemv_dma_supported(const _Float16 *X, const uint8_t *W, int64_t K, int64_t N);
hipError_t launch_gemv_dma_group(const _Float16 *X, const uint8_t *const *W, _Float16 *const *Y, int count,
                                 int K, int N, int *n_done, hipStream_t s);
}  // namespace mcq4

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return MCQ4_OK;
    return fail(MCQ4_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int64_t kMaxBlocksK = 65535;        // grid.y limit of the conversion kernels
constexpr int64_t kMaxDim = (int64_t)1 << 30;  // keeps 32-bit lane offsets safe

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// Prefill kernel choice (M > 64).  When N % 128 == 0 and the pointers are
// 16-byte aligned: the few-tile GEMM (q4_gemm8) when its plan is one round of
// workgroups, the 256 x 256-tile GEMM (q4_gemm7) on grids that nearly fill the
// CUs, else the 128 x 256-tile LDS-staged GEMM with two waves per SIMD
// (q4_gemm6).  Otherwise the async-copy GEMM (q4_gemm2) when its alignment
// needs hold and the output has at least 128 tiles of 128x256; otherwise the
// register-staged split-K kernel.  MCQ4_GEMM_PATH=sync|async|6|7|8 forces one
// kernel (tests).
enum class Prefill { Sync, Async2, Staged6, Wide7, Few8 };
Prefill prefill_kernel(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K,
                       int64_t N) {
    const bool ok2 = mcq4::gemm2_supported(X, ldx, W, K, N);
    const bool ok6 = mcq4::gemm6_supported(X, ldx, W, M, K, N);
    if (const char *env = mcq4::opt("MCQ4_GEMM_PATH")) {
        if (env[0] == 's') return Prefill::Sync;
        if (env[0] == 'a' && ok2) return Prefill::Async2;
        if (env[0] == '6' && ok6) return Prefill::Staged6;
        if (env[0] == '7' && mcq4::gemm7_supported(X, ldx, W, M, K, N)) return Prefill::Wide7;
        if (env[0] == '8' && mcq4::gemm8_supported(X, ldx, W, M, K, N)) return Prefill::Few8;
    }
    // Measured (us per launch, `python bench.py --part prefill-routing`, one box;
    // default / q4_gemm6 / q4_gemm7 / q4_gemm8 forced):
    //   M=512 11008x4096 55.8 / 59.5 / 64.1 / 56.5, 4096x4096 29.3 / 31.7 / 35.6 / 29.3
    //   M=768 4096x4096 35.1 / 43.9 / 43.6 / 35.0; M=1024 4096x4096 40.8 / 50.2 / 53.2 / 41.0
    //   M=256 4096x14336 39.7 / 46.7 / 49.1 / 39.7
    //   M=1024 4096x11008 96.1 / 109.0 / 96.4 / 116.1; M=768 4096x14336 94.7 / 107.9 / 94.8 / 114.8
    //   M=1280 4096x8192 92.2 / 106.2 / 92.4 / 111.6
    //   M=640 4096x11008 69.9 / 69.1 / 85.8 / 75.7; M=1536 4096x4096 63.3 / 63.2 / 65.3 / 72.6
    //   M=256 11008x4096 38.0 / 38.6 / 43.6 / 41.1; M=2048 4096x4096 75.0 / 75.1 / 81.0 / 81.5
    // The few-tile GEMM (128 x 128 tiles, eight waves, K split four ways
    // inside the workgroup and at most twice across) wins when its plan is one
    // round of 192..256 workgroups, and loses with more rounds or a half-empty
    // grid.  The 256 x 256-tile GEMM (one wave per SIMD, half the dequant per
    // MFMA) wins from 160 tiles, or from 96 on long K where two K splits and
    // their reduction cost little; the 128 x 256-tile q4_gemm6 below that.
    if (ok6 && mcq4::gemm8_supported(X, ldx, W, M, K, N)) {
        const int g8 = mcq4::gemm8_workgroups(M, K, N);
        if (g8 >= 192 && g8 <= 256) return Prefill::Few8;
    }
    if (ok6 && mcq4::gemm7_supported(X, ldx, W, M, K, N)) {
        const int64_t t7 = ((M + 255) / 256) * ((N + 255) / 256);
        if (t7 >= 160 || (t7 >= 96 && K >= 8192)) return Prefill::Wide7;
    }
    if (ok6) return Prefill::Staged6;
    if (ok2 && ((M + 127) / 128) * ((N + 255) / 256) >= 128) return Prefill::Async2;
    return Prefill::Sync;
}

int check_kn(int64_t K, int64_t N) {
    if (K <= 0 || N <= 0) return fail(MCQ4_ERR_SHAPE, "K (%lld) and N (%lld) must be positive",
                                      (long long)K, (long long)N);
    if (K % 32 != 0) return fail(MCQ4_ERR_SHAPE, "K (%lld) must be divisible by 32", (long long)K);
    if (K / 32 > kMaxBlocksK || N > kMaxDim || (K / 32) * N * 18 > ((int64_t)1 << 40))
        return fail(MCQ4_ERR_SHAPE, "shape K=%lld N=%lld exceeds the supported size",
                    (long long)K, (long long)N);
    return MCQ4_OK;
}

// Scratch of the allocation-free matmul entry point: one split-K workspace per
// GPU in the library's own device memory (zero at load; every completed call
// leaves its counter area zero again).  Host code uses only the per-device
// address from hipGetSymbolAddress, never the array's name.  16 MiB of partials
// hold every decode shape's split-K plan (1.25 MiB at M = 16..32, K = 14336) and
// prefill plans up to M = 64 at K = 14336; larger split-K plans are rejected.
// The array is part of the library image, so every GPU the library is loaded on
// holds it (16.25 MiB) whether or not the entry point is called.
constexpr size_t kNoAllocScratchBytes = mcq4::COUNTER_BYTES + ((size_t)16 << 20);
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];
std::atomic<bool> g_scratch_dirty[kMaxDevices];   // a failed call may have left counters set
std::mutex g_scratch_mu;

// The current device's scratch address, resolved once per device.
int scratch_ptr(void **out, int *dev_out) {
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(MCQ4_ERR_INVALID_ARG, "device %d out of range", dev);
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_acquire);
        if (!p) {
            if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))
                return hip_status(e, "hipGetSymbolAddress(scratch)");
            if (!p) return fail(MCQ4_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    *dev_out = dev;
    return MCQ4_OK;
}

}  // namespace

namespace mcq4 {
int set_error(int code, const char *msg) {
    snprintf(g_err, sizeof(g_err), "%s", msg);
    return code;
}
}  // namespace mcq4

extern "C" {

int mcq4_version(void) { return 1 * 10000 + 1 * 100 + 0; }

const char *mcq4_status_string(int status) {
    switch (status) {
        case MCQ4_OK: return "ok";
        case MCQ4_ERR_INVALID_ARG: return "invalid argument";
        case MCQ4_ERR_SHAPE: return "unsupported shape";
        case MCQ4_ERR_ALIGNMENT: return "misaligned pointer or leading dimension";
        case MCQ4_ERR_WORKSPACE: return "workspace missing or too small";
        case MCQ4_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char *mcq4_last_error(void) { return g_err; }

static int quantize_common(bool llama, const float *W, int64_t ldw, int64_t K, int64_t N,
                           uint8_t *blocks, void *stream) {
    g_err[0] = 0;
    if (!W || !blocks) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (int st = check_kn(K, N)) return st;
    if (ldw < N) return fail(MCQ4_ERR_SHAPE, "ldw (%lld) < N (%lld)", (long long)ldw, (long long)N);
    if (!aligned(W, 4)) return fail(MCQ4_ERR_ALIGNMENT, "W must be 4-byte aligned");
    if (!aligned(blocks, 2)) return fail(MCQ4_ERR_ALIGNMENT, "blocks must be 2-byte aligned");
    return hip_status(mcq4::launch_quantize(llama, W, ldw, (int)(K / 32), (int)N, blocks,
                                            (hipStream_t)stream),
                      "quantize launch");
}

int mcq4_quantize_q4_0(const float *W, int64_t ldw, int64_t K, int64_t N, uint8_t *blocks,
                       void *stream) {
    return quantize_common(false, W, ldw, K, N, blocks, stream);
}

int mcq4_quantize_q4_0_typed(const void *W, int w_dtype, int64_t ldw, int64_t K, int64_t N,
                             uint8_t *blocks, void *stream) {
    g_err[0] = 0;
    if (!W || !blocks) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (w_dtype != MCQ4_DTYPE_F32 && w_dtype != MCQ4_DTYPE_F16 && w_dtype != MCQ4_DTYPE_BF16)
        return fail(MCQ4_ERR_INVALID_ARG, "w_dtype must be MCQ4_DTYPE_F32, F16 or BF16");
    if (int st = check_kn(K, N)) return st;
    if (ldw < N) return fail(MCQ4_ERR_SHAPE, "ldw (%lld) < N (%lld)", (long long)ldw, (long long)N);
    if (!aligned(W, w_dtype == MCQ4_DTYPE_F32 ? 4 : 2))
        return fail(MCQ4_ERR_ALIGNMENT, "W is misaligned for its dtype");
    if (!aligned(blocks, 2)) return fail(MCQ4_ERR_ALIGNMENT, "blocks must be 2-byte aligned");
    return hip_status(mcq4::launch_quantize_typed(w_dtype, W, ldw, (int)(K / 32), (int)N, blocks,
                                                  (hipStream_t)stream),
                      "quantize launch");
}

int mcq4_quantize_q4_0_llama(const float *W, int64_t ldw, int64_t K, int64_t N,
                             uint8_t *blocks, void *stream) {
    return quantize_common(true, W, ldw, K, N, blocks, stream);
}

int mcq4_dequantize_q4_0(const uint8_t *blocks, int64_t K, int64_t N, void *out, int64_t ldo,
                         int out_dtype, void *stream) {
    g_err[0] = 0;
    if (!blocks || !out) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (out_dtype != MCQ4_DTYPE_F32 && out_dtype != MCQ4_DTYPE_F16)
        return fail(MCQ4_ERR_INVALID_ARG, "out_dtype must be MCQ4_DTYPE_F32 or MCQ4_DTYPE_F16");
    if (int st = check_kn(K, N)) return st;
    if (ldo < N) return fail(MCQ4_ERR_SHAPE, "ldo (%lld) < N (%lld)", (long long)ldo, (long long)N);
    if (!aligned(blocks, 2)) return fail(MCQ4_ERR_ALIGNMENT, "blocks must be 2-byte aligned");
    if (!aligned(out, out_dtype == MCQ4_DTYPE_F32 ? 4 : 2))
        return fail(MCQ4_ERR_ALIGNMENT, "out is misaligned for its dtype");
    return hip_status(mcq4::launch_dequant(blocks, (int)(K / 32), (int)N, out, ldo,
                                           out_dtype == MCQ4_DTYPE_F16, (hipStream_t)stream),
                      "dequantize launch");
}

size_t mcq4_matmul_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M <= 0 || K <= 0 || N <= 0 || K % 32) return 0;
    if (M <= 32) return mcq4::skinny_workspace_bytes(M, K, N);
    // The largest of the split-K kernels' needs: an upper bound for any prefill kernel.
    const size_t pre = std::max({mcq4::gemm_workspace_bytes(M, K, N), mcq4::gemm6_workspace_bytes(M, K, N),
                                 mcq4::gemm7_workspace_bytes(M, K, N), mcq4::gemm8_workspace_bytes(M, K, N)});
    // 33..64 rows run either family, depending on the pointers' alignment.
    return M <= 64 ? std::max(pre, mcq4::skinny_workspace_bytes(M, K, N)) : pre;
}

int mcq4_matmul_q4_0_f16(const void *X, int64_t ldx, const uint8_t *W, void *Y, int64_t ldy,
                         int64_t M, int64_t K, int64_t N, void *workspace,
                         size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    if (!X || !W || !Y) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (M <= 0) return fail(MCQ4_ERR_SHAPE, "M (%lld) must be positive", (long long)M);
    if (int st = check_kn(K, N)) return st;
    if (M > kMaxDim) return fail(MCQ4_ERR_SHAPE, "M (%lld) too large", (long long)M);
    if (ldx < K) return fail(MCQ4_ERR_SHAPE, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
    if (ldy < N) return fail(MCQ4_ERR_SHAPE, "ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
    if (!aligned(X, 16) || ldx % 8)
        return fail(MCQ4_ERR_ALIGNMENT, "X must be 16-byte aligned with ldx %% 8 == 0");
    if (!aligned(W, 2)) return fail(MCQ4_ERR_ALIGNMENT, "W must be 2-byte aligned");
    if (!aligned(Y, 2)) return fail(MCQ4_ERR_ALIGNMENT, "Y must be 2-byte aligned");
    const size_t need = mcq4_matmul_workspace_bytes(M, K, N);
    if (need && (!workspace || workspace_bytes < need))
        return fail(MCQ4_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                    workspace ? workspace_bytes : (size_t)0);
    if (need && !aligned(workspace, 16))
        return fail(MCQ4_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
    hipError_t e;
    // 33..64 rows: q4_gemm6 (flat ~31 us for any M <= 128 on 4096x14336) beats the
    // register-load decode kernel (40-77 us) wherever its alignment rules hold.
    const bool skinny = M <= 32 || (M <= 64 && !mcq4::gemm6_supported((const _Float16 *)X, ldx, W, M, K, N));
    if (skinny)
        e = mcq4::launch_skinny((const _Float16 *)X, ldx, W, (_Float16 *)Y, ldy, (int)M, (int)K,
                                (int)N, workspace, (hipStream_t)stream);
    else {
        const _Float16 *x = (const _Float16 *)X;
        _Float16 *y = (_Float16 *)Y;
        hipStream_t st = (hipStream_t)stream;
        switch (prefill_kernel(x, ldx, W, M, K, N)) {
            case Prefill::Staged6: e = mcq4::launch_gemm6(x, ldx, W, y, ldy, (int)M, (int)K, (int)N, workspace, st); break;
            case Prefill::Wide7: e = mcq4::launch_gemm7(x, ldx, W, y, ldy, (int)M, (int)K, (int)N, workspace, st); break;
            case Prefill::Few8: e = mcq4::launch_gemm8(x, ldx, W, y, ldy, (int)M, (int)K, (int)N, workspace, st); break;
            case Prefill::Async2: e = mcq4::launch_gemm2(x, ldx, W, y, ldy, (int)M, (int)K, (int)N, st); break;
            default: e = mcq4::launch_gemm(x, ldx, W, y, ldy, (int)M, (int)K, (int)N, workspace, st); break;
        }
    }
    return hip_status(e, "matmul launch");
}

int mcq4_matmul_q4_0_f16_grouped(const void *X, int64_t ldx, int count, const uint8_t *const *W,
                                 void *const *Y, int64_t ldy, int64_t M, int64_t K, int64_t N,
                                 void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    if (!W || !Y || count < 1) return fail(MCQ4_ERR_INVALID_ARG, "need count >= 1 weights and outputs");
    for (int g = 0; g < count; ++g)
        if (!W[g] || !Y[g]) return fail(MCQ4_ERR_INVALID_ARG, "null weight or output pointer %d", g);
    // The same argument checks as the per-weight calls, whichever path runs.
    if (ldy < N) return fail(MCQ4_ERR_SHAPE, "ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
    // One launch for M == 1 when every weight takes the M == 1 kernel whole
    // (16-byte aligned, N a multiple of 16) and there are at most 4 of them.
    bool one = M == 1 && count <= 4 && N % 16 == 0 && X && aligned(X, 16) && ldx % 8 == 0 && ldx >= K &&
               K > 0 && K % 32 == 0 && N > 0 && !check_kn(K, N);
    for (int g = 0; one && g < count; ++g)
        one = aligned(Y[g], 2) && mcq4::gemv_dma_supported((const _Float16 *)X, W[g], K, N * count);
    g_err[0] = 0;
    if (!one) {
        for (int g = 0; g < count; ++g)
            if (int st = mcq4_matmul_q4_0_f16(X, ldx, W[g], Y[g], ldy, M, K, N, workspace, workspace_bytes,
                                              stream))
                return st;
        return MCQ4_OK;
    }
    int n_done = 0;
    const hipError_t e = mcq4::launch_gemv_dma_group((const _Float16 *)X, W, (_Float16 *const *)Y, count, (int)K,
                                                     (int)N, &n_done, (hipStream_t)stream);
    return hip_status(e, "grouped matmul launch");
}

int mcq4_matmul_q4_0(const void *X, int x_dtype, int64_t ldx, const uint8_t *W, void *Y,
                     int64_t ldy, int64_t M, int64_t K, int64_t N, void *workspace,
                     size_t workspace_bytes, void *stream) {
    if (x_dtype == MCQ4_DTYPE_F16)
        return mcq4_matmul_q4_0_f16(X, ldx, W, Y, ldy, M, K, N, workspace, workspace_bytes, stream);
    g_err[0] = 0;
    if (x_dtype != MCQ4_DTYPE_F32 && x_dtype != MCQ4_DTYPE_BF16)
        return fail(MCQ4_ERR_INVALID_ARG, "x_dtype must be MCQ4_DTYPE_F32, F16 or BF16");
    if (!X || !W || !Y) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    if (M <= 0) return fail(MCQ4_ERR_SHAPE, "M (%lld) must be positive", (long long)M);
    if (int st = check_kn(K, N)) return st;
    if (M > ((int64_t)65535 * 8)) return fail(MCQ4_ERR_SHAPE, "M (%lld) too large", (long long)M);
    if (ldx < K) return fail(MCQ4_ERR_SHAPE, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
    if (ldy < N) return fail(MCQ4_ERR_SHAPE, "ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
    const uintptr_t al = x_dtype == MCQ4_DTYPE_F32 ? 4 : 2;
    if (!aligned(X, al) || !aligned(Y, al))
        return fail(MCQ4_ERR_ALIGNMENT, "X and Y must be aligned to their dtype");
    if (!aligned(W, 2)) return fail(MCQ4_ERR_ALIGNMENT, "W must be 2-byte aligned");
    (void)workspace; (void)workspace_bytes;
    return hip_status(mcq4::launch_q4_xact(X, x_dtype, ldx, W, Y, ldy, M, K, N, (hipStream_t)stream),
                      "matmul launch");
}

int mcq4_reset_workspace(void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    if (!workspace) return fail(MCQ4_ERR_INVALID_ARG, "null workspace");
    if (workspace_bytes < mcq4::COUNTER_BYTES)
        return fail(MCQ4_ERR_WORKSPACE, "workspace of %zu bytes is smaller than its %zu-byte counter area",
                    workspace_bytes, (size_t)mcq4::COUNTER_BYTES);
    if (!aligned(workspace, 16)) return fail(MCQ4_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
    return hip_status(mcq4::launch_zero_counters(workspace, (hipStream_t)stream), "workspace reset launch");
}

int mcq4_split_fallback_count(uint64_t *count, int reset) {
    g_err[0] = 0;
    if (!count) return fail(MCQ4_ERR_INVALID_ARG, "null pointer");
    *count = 0;
    hipError_t (*const readers[])(uint64_t *, bool) = {
        mcq4::q4_gemvm_split_fallbacks, mcq4::q4_gemm6_split_fallbacks, mcq4::i4_gemv_split_fallbacks,
        mcq4::i4_gemv1_split_fallbacks, mcq4::i4_gemm6_split_fallbacks, mcq4::q4_gemv_span_split_fallbacks,
        mcq4::q4_gemm8_split_fallbacks};
    for (auto rd : readers)
        if (int st = hip_status(rd(count, reset != 0), "split fallback counter")) return st;
    return MCQ4_OK;
}

size_t mcq4_matmul_noalloc_max_workspace_bytes(void) { return kNoAllocScratchBytes; }

int mcq4_matmul_q4_0_f16_noalloc(const void *X, int64_t ldx, const uint8_t *W, void *Y, int64_t ldy,
                                 int64_t M, int64_t K, int64_t N, void *stream) {
    g_err[0] = 0;
    if (M > 0 && K > 0 && N > 0 && K % 32 == 0) {
        const size_t need = mcq4_matmul_workspace_bytes(M, K, N);
        if (need > kNoAllocScratchBytes)
            return fail(MCQ4_ERR_WORKSPACE,
                        "shape M=%lld K=%lld N=%lld needs a %zu-byte workspace; the allocation-free entry "
                        "point holds at most %zu (use mcq4_matmul_q4_0_f16 with a caller workspace)",
                        (long long)M, (long long)K, (long long)N, need, kNoAllocScratchBytes);
    }
    void *ws = nullptr;
    int dev = 0;
    if (int st = scratch_ptr(&ws, &dev)) return st;
    if (g_scratch_dirty[dev].load(std::memory_order_acquire)) {
        if (int st = hip_status(mcq4::launch_zero_counters(ws, (hipStream_t)stream), "scratch reset launch"))
            return st;
        g_scratch_dirty[dev].store(false, std::memory_order_release);
    }
    const int st = mcq4_matmul_q4_0_f16(X, ldx, W, Y, ldy, M, K, N, ws, kNoAllocScratchBytes, stream);
    // Any failure may follow a launch that drew split-K tickets: the next call
    // zeroes the counter area first.
    if (st != MCQ4_OK) g_scratch_dirty[dev].store(true, std::memory_order_release);
    return st;
}

}  // extern "C"
