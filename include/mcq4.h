/*
 * mcq4 -- C ABI of the MI355X (gfx950) GGML block_q4_0 INT4 matmul path.
 *
 * Drop-in for metalcore's q4_0 path (reference: myfykris/metalops,
 * packages/metalcore/src/metalcore/).  Every entry point:
 *   - takes plain device pointers, sizes and an opaque HIP stream (hipStream_t
 *     passed as void*; NULL = the default stream);
 *   - allocates nothing: the caller owns every buffer, including the optional
 *     split-K workspace;
 *   - enqueues asynchronously on the given stream and returns a status code (no
 *     exceptions cross the ABI); mcq4_last_error() gives a message for the last
 *     failure on the calling thread;
 *   - is re-entrant: the only global state is a once-per-device raise of the
 *     kernels' dynamic-LDS limit (hipFuncSetAttribute), guarded by an atomic.
 *
 * Weight format (quantization.py:296-304): blocks[K/32][N][18] uint8; bytes 0..1
 * of a block are the fp16 scale d (little endian), byte 2+i holds element 2i in
 * the low nibble and element 2i+1 in the high nibble; W[kb*32+j][n] = (q_j - 8)*d.
 */
#ifndef MCQ4_H
#define MCQ4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mcq4_status {
    MCQ4_OK = 0,
    MCQ4_ERR_INVALID_ARG = 1,  /* null pointer, negative size, bad dtype code */
    MCQ4_ERR_SHAPE = 2,        /* K not a multiple of 32, leading dim too small, size limits */
    MCQ4_ERR_ALIGNMENT = 3,    /* pointer / leading-dimension alignment requirement violated */
    MCQ4_ERR_WORKSPACE = 4,    /* workspace missing or smaller than mcq4_matmul_workspace_bytes */
    MCQ4_ERR_HIP = 5           /* a HIP runtime call (launch) failed */
} mcq4_status;

enum { MCQ4_DTYPE_F32 = 0, MCQ4_DTYPE_F16 = 1, MCQ4_DTYPE_BF16 = 2 };

/* Library version: major*10000 + minor*100 + patch. */
int mcq4_version(void);
const char *mcq4_status_string(int status);
/* Message for the most recent failing call on this thread ("" if none). */
const char *mcq4_last_error(void);

/*
 * quantize_ggml_q4_0 (quantization.py:307-371), reference rule:
 *   d = amax/7 (0 -> 1), q = round_half_even(x/d + 8) clamped to [0, 15].
 * W: fp32 row-major [K][ldw] (ldw >= N), blocks: [K/32][N][18], 2-byte aligned.
 */
int mcq4_quantize_q4_0(const float *W, int64_t ldw, int64_t K, int64_t N,
                       uint8_t *blocks, void *stream);

/*
 * quantize_ggml_q4_0 (quantization.py:307-371) for a weight of any float dtype
 * (w_dtype MCQ4_DTYPE_F32 / F16 / BF16).  The reference runs every step as a
 * torch op in the weight's own dtype (quantization.py:335-347): amax, amax/7,
 * the zero test, x/d, +8 and the rounding are each rounded to w_dtype here as
 * there; d is then stored as fp16 (:352).  W: [K][ldw] in w_dtype, aligned to
 * its element size.  For MCQ4_DTYPE_F32 this is mcq4_quantize_q4_0.
 */
int mcq4_quantize_q4_0_typed(const void *W, int w_dtype, int64_t ldw, int64_t K, int64_t N,
                             uint8_t *blocks, void *stream);

/*
 * llama.cpp quantize_row_q4_0_ref scale/rounding rule, emitted in the same
 * [K/32][N][18] layout and nibble order.  No counterpart in the reference: it
 * generates the benchmark configurations (signed scales, q = 0 reachable).
 */
int mcq4_quantize_q4_0_llama(const float *W, int64_t ldw, int64_t K, int64_t N,
                             uint8_t *blocks, void *stream);

/*
 * dequantize_ggml_q4_0 (quantization.py:374-419): out[K][ldo] = (q - 8)*d,
 * exact in fp32 (out_dtype MCQ4_DTYPE_F32) or rounded once to nearest-even fp16
 * (MCQ4_DTYPE_F16).
 */
int mcq4_dequantize_q4_0(const uint8_t *blocks, int64_t K, int64_t N, void *out,
                         int64_t ldo, int out_dtype, void *stream);

/*
 * Workspace bytes mcq4_matmul_q4_0_f16 needs for this shape (0 = none).  The
 * workspace starts with a fixed 256 KiB area of per-tile arrival counters,
 * followed by fp32 split-K partials and, for the kernels whose splits signal
 * each other with per-split flag words, those words (any starting value: each
 * call reads them as it starts and moves each by a fixed step).  The counter
 * area must be zero-filled
 * before first use; every completed call leaves it zero again, so one zeroed
 * buffer can be reused for any later call whose requirement it covers.  Calls
 * that share a workspace must not overlap (use one workspace per stream).
 */
size_t mcq4_matmul_workspace_bytes(int64_t M, int64_t K, int64_t N);

/*
 * matmul_ggml_q4_0 (quantization.py:422-454; Metal host binding
 * native/core_mps.mm:5917-5975): Y[M][ldy] = X[M][ldx] @ dequant(W), fp16 in,
 * fp32 accumulation, fp16 out.  M <= 64 runs the decode GEMV kernels, larger M
 * the prefill MFMA GEMM kernels.
 * Requirements: K % 32 == 0; X 16-byte aligned with ldx % 8 == 0; W 2-byte
 * aligned; Y 2-byte aligned; ldx >= K, ldy >= N.
 */
int mcq4_matmul_q4_0_f16(const void *X, int64_t ldx, const uint8_t *W, void *Y,
                         int64_t ldy, int64_t M, int64_t K, int64_t N,
                         void *workspace, size_t workspace_bytes, void *stream);

/*
 * Allocation-free variant of mcq4_matmul_q4_0_f16.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments minus the workspace: the split-K workspace is the library's own
 * device array (one per GPU, held until the process ends) of
 * mcq4_matmul_noalloc_max_workspace_bytes() bytes (256 KiB of counters +
 * 16 MiB: every decode plan, prefill split-K plans up to M = 64 at
 * K = 14336); a shape whose mcq4_matmul_workspace_bytes exceeds it returns
 * MCQ4_ERR_WORKSPACE.  Calls allocate nothing (no hipMalloc / hipFree, no
 * allocating library routine).  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, two threads) race and give wrong
 * results; serialise them.  Results are bit-identical to mcq4_matmul_q4_0_f16.
 */
int mcq4_matmul_q4_0_f16_noalloc(const void *X, int64_t ldx, const uint8_t *W, void *Y,
                                 int64_t ldy, int64_t M, int64_t K, int64_t N, void *stream);
size_t mcq4_matmul_noalloc_max_workspace_bytes(void);

/*
 * Several q4_0 products that share the activations: Y[g] = X @ dequant(W[g]) for
 * g < count, every W[g] of shape [K/32][N][18] and every Y[g] [M][ldy] fp16.
 * No counterpart in the reference (its API takes one weight per call); it is
 * for decode loops that project one activation row through several weights --
 * gate and up of an MLP -- and would otherwise pay a launch per weight.  W and
 * Y are host arrays of device pointers.  At M == 1 with count <= 4, N % 16 == 0
 * and 16-byte aligned weights this is one launch of the M == 1 kernel over all
 * count * N columns; otherwise it calls mcq4_matmul_q4_0_f16 per weight (same
 * workspace rules).
 */
int mcq4_matmul_q4_0_f16_grouped(const void *X, int64_t ldx, int count, const uint8_t *const *W,
                                 void *const *Y, int64_t ldy, int64_t M, int64_t K, int64_t N,
                                 void *workspace, size_t workspace_bytes, void *stream);

/*
 * matmul_ggml_q4_0 for activations of any float dtype (quantization.py:422-454).
 * x_dtype MCQ4_DTYPE_F16 is mcq4_matmul_q4_0_f16 (the fp16 MFMA kernels, the
 * semantics of the reference's GPU binding, core_mps.mm:5917-5975).
 * MCQ4_DTYPE_BF16 / F32 follow the reference's path for those dtypes
 * (quantization.py:452-454): W dequantized to x_dtype (one rounding of the
 * exact product), Y = X @ W with fp32 accumulation, Y in x_dtype.  X and Y
 * aligned to x_dtype; no workspace is needed for them (may be NULL).
 */
int mcq4_matmul_q4_0(const void *X, int x_dtype, int64_t ldx, const uint8_t *W, void *Y,
                     int64_t ldy, int64_t M, int64_t K, int64_t N, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * Re-zeroes the counter area (the first 256 KiB) of a split-K workspace with a
 * fill kernel on `stream`.  Every completed call leaves the area zero; a call
 * that was interrupted (a failed launch, a killed stream) may not, and a
 * workspace is then reset before its next use.  No counterpart in the
 * reference (its Metal binding keeps no workspace).
 */
int mcq4_reset_workspace(void *workspace, size_t workspace_bytes, void *stream);

/*
 * Number of split-K tiles, on the current device, whose XCD-local exchange
 * found a split that ran on another XCD than the summing workgroup and
 * recomputed that split's partial instead of reading it (the results stay
 * correct; on MI355X in its default partition mode the count stays 0).
 * Synchronous (reads device counters); reset != 0 clears them.  Diagnostic
 * only; no counterpart in the reference.
 */
int mcq4_split_fallback_count(uint64_t *count, int reset);

/*
 * Re-reads the library's MCQ4_* test and experiment switches from the
 * environment (they are read once, at the first launch, and never per call).
 * No counterpart in the reference.
 */
int mcq4_reload_options(void);

/* ---------------------------------------------------------------------------
 * Per-group INT4 (metalcore quantization.py:26-239, Int4Linear :457-613).
 *
 * Format: packed[K/2][N] uint8, row k in byte row k/2 (even k low nibble, odd
 * k high nibble); scales[G][N] and zeros[G][N] with G = ceil(K/group_size), in
 * one float dtype (sz_dtype: MCQ4_DTYPE_F32 / F16 / BF16);
 * W[k][n] = (q - zeros[k/group_size][n]) * scales[k/group_size][n].
 * Rows are dense: packed row stride N bytes, scales/zeros row stride N.
 * ------------------------------------------------------------------------- */

/*
 * quantize_int4 (quantization.py:26-92): per group and column
 *   scale = (max - min)/15 clamped to >= 1e-8, zero = -min/scale,
 *   q = round_half_even(w/scale + zero) clamped to [0, 15],
 * every step rounded to w_dtype as the reference's torch ops on a weight of
 * that dtype are.  W: [K][ldw] in w_dtype (ldw >= N); scales/zeros are written
 * in w_dtype.  K must be even; group_size >= 1.
 */
int mcq4_quantize_int4(const void *W, int w_dtype, int64_t ldw, int64_t K, int64_t N,
                       int64_t group_size, uint8_t *packed, void *scales, void *zeros,
                       void *stream);

/*
 * dequantize_int4 (quantization.py:95-153): out[K][ldo] =
 * ((float)q - zero) * scale in fp32 (zero and scale upcast exactly, two fp32
 * roundings), then one rounding to out_dtype (F32 / F16 / BF16).
 */
int mcq4_dequantize_int4(const uint8_t *packed, const void *scales, const void *zeros,
                         int sz_dtype, int64_t K, int64_t N, int64_t group_size, void *out,
                         int64_t ldo, int out_dtype, void *stream);

/* Workspace bytes the int4 matmul entry points need for this shape (0 = none);
 * same conventions as mcq4_matmul_workspace_bytes (zero-filled counter area
 * first, reusable, one workspace per stream). */
size_t mcq4_matmul_int4_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                        int x_dtype);

/*
 * matmul_int4 (quantization.py:156-239; Metal binding matmul_int4_metal,
 * native/core_mps.mm:5612-5776): Y[M][ldy] = X[M][ldx] @ dequant(W) with
 * fp32 accumulation; X and Y in x_dtype (F16, BF16 or F32).  fp16 activations
 * with group_size % 32 == 0, K % 32 == 0 and N % 8 == 0 run the MFMA kernels
 * (decode GEMV for M <= 16, and for M <= 32 with N % 128 == 0 and 16-byte
 * aligned operands; prefill GEMM above); every other case runs a
 * general fp32 kernel.  X needs x_dtype alignment (16 bytes and ldx % 8 == 0
 * for the MFMA kernels; the general kernel is used otherwise), Y x_dtype
 * alignment; ldx >= K, ldy >= N.
 */
int mcq4_matmul_int4(const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                     const void *scales, const void *zeros, int sz_dtype, void *Y, int64_t ldy,
                     int64_t M, int64_t K, int64_t N, int64_t group_size, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * matmul_int4_silu / matmul_int4_gelu (native/core_mps.mm:5780-5914, fused
 * kernels native/quant_kernels.metal:884-1145): the same product with the
 * activation applied to the fp32 result before the store, as the fused kernels
 * do: silu(y) = y / (1 + exp(-y)) (:996-998);
 * gelu(y) = y/2 * (1 + tanh(sqrt(2/pi) * (y + 0.044715 y^3))) (:1126-1132).
 */
int mcq4_matmul_int4_silu(const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                          const void *scales, const void *zeros, int sz_dtype, void *Y,
                          int64_t ldy, int64_t M, int64_t K, int64_t N, int64_t group_size,
                          void *workspace, size_t workspace_bytes, void *stream);
int mcq4_matmul_int4_gelu(const void *X, int x_dtype, int64_t ldx, const uint8_t *packed,
                          const void *scales, const void *zeros, int sz_dtype, void *Y,
                          int64_t ldy, int64_t M, int64_t K, int64_t N, int64_t group_size,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * GPU-side quantize_to_int4 (binding native/core_mps.mm:4655-4700, kernel
 * native/quant_kernels.metal:634-686): the quantize_int4 computation in fp32
 * with round-half-away-from-zero (Metal round()).  W fp32 [K][ldw];
 * packed [K/2][N]; scales, zeros fp32 [ceil(K/group_size)][N]; group_size even.
 */
int mcq4_quantize_to_int4(const float *W, int64_t ldw, int64_t K, int64_t N, int64_t group_size,
                          uint8_t *packed, float *scales, float *zeros, void *stream);

/* ---------------------------------------------------------------------------
 * Per-group INT8 (quantization.py:242-286; Metal binding matmul_int8_metal,
 * native/core_mps.mm:4516-4565): W int8 [K][N] (row stride N),
 * W[k][n] = (q - zeros[k/group_size][n]) * scales[k/group_size][n].
 * ------------------------------------------------------------------------- */
size_t mcq4_matmul_int8_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                        int x_dtype);

/* Y[M][ldy] = X[M][ldx] @ dequant(W), fp32 accumulation, X and Y in x_dtype.
 * fp16 activations with group_size % 16 == 0, K % 16 == 0 and N % 8 == 0 run
 * the MFMA GEMV (M <= 16); K and group_size % 32 == 0 with N % 128 == 0 the
 * MFMA GEMM; everything else the general fp32 kernel. */
int mcq4_matmul_int8(const void *X, int x_dtype, int64_t ldx, const int8_t *W, const void *scales,
                     const void *zeros, int sz_dtype, void *Y, int64_t ldy, int64_t M, int64_t K,
                     int64_t N, int64_t group_size, void *workspace, size_t workspace_bytes,
                     void *stream);

/* Workspace bytes of mcq4_fused_rmsnorm_linear_int4: the matmul's own
 * workspace (zero-filled counter area first, same conventions), then the
 * normalized fp16 activations after it. */
size_t mcq4_fused_rmsnorm_linear_int4_workspace_bytes(int64_t M, int64_t K, int64_t N,
                                                      int64_t group_size);

/*
 * fused_rmsnorm_linear_int4 (native/core_mps.mm:3017-3103): Y = matmul_int4(
 * rmsnorm(X, w_norm, eps), packed, scales, zeros) with X [M][ldx] fp16, w_norm
 * [K] fp16, Y [M][ldy] fp16.  RMSNorm as native/training_kernels.metal:425-488:
 * rstd = 1/sqrt(sum(x^2)/K + eps) in fp32, X_norm = fp16(x * rstd * w_norm).
 * M == 1 with X and w_norm 16-byte aligned, on the shapes the async-copy INT4
 * GEMV takes: one launch that normalises inside the GEMV.  Otherwise X_norm is
 * written to the workspace behind the matmul's share (workspace 256-byte
 * aligned), then the INT4 matmul runs on the same stream.  Both forms give the
 * same bits.
 */
int mcq4_fused_rmsnorm_linear_int4(const void *X, int64_t ldx, const void *w_norm, float eps,
                                   const uint8_t *packed, const void *scales, const void *zeros,
                                   int sz_dtype, void *Y, int64_t ldy, int64_t M, int64_t K,
                                   int64_t N, int64_t group_size, void *workspace,
                                   size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MCQ4_H */
