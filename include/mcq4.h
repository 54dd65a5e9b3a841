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

enum { MCQ4_DTYPE_F32 = 0, MCQ4_DTYPE_F16 = 1 };

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
 * followed by fp32 split-K partials.  The counter area must be zero-filled
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

#ifdef __cplusplus
}
#endif

#endif /* MCQ4_H */
