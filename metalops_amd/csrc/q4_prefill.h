// Shared plan and arguments of the LDS-staged q4_0 prefill GEMM (q4_gemm6):
// output tiles of 128 x 256, optional split-K over grid.z with fp32 partial
// tiles in the caller's workspace.
#pragma once

#include "q4_common.h"

namespace mcq4 {

constexpr int G6_BM = 128;   // output tile rows
constexpr int G6_BN = 256;   // output tile columns

struct Gemm6Args {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int tiles_m, tiles_n;
    int S;               // K splits (grid.z)
    float *partials;     // [tiles][S][128*256] when S > 1
    // S == 2 with an XCD-local exchange: grid.x padded to a multiple of 8, the
    // second split of a tile to finish adds the first's partial and stores Y
    // (64-bit tickets [8][4096] by blockIdx.x mod 8 at the workspace start).
    uint64_t *tickets = nullptr;
    uint32_t foreign = 0;    // splits treated as run on another XCD (test switch)
};

// Needs N % 128 == 0, 16-byte aligned W and activation rows, K >= 32, M * ldx <
// 2^30 and W below 2^31 bytes (buffer loads).
bool gemm6_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N);
size_t gemm6_workspace_bytes(int64_t M, int64_t K, int64_t N);
hipError_t launch_gemm6(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s);

// Few-tile prefill GEMM (q4_gemm8): 128 x 128 tiles, eight waves with K split
// four ways inside the workgroup, at most two K splits across workgroups
// summed through the XCD's L2 (partials [tiles][2][128*128] after the ticket
// area).  Needs what q4_gemm6 needs.
constexpr int G8_BM = 128;
constexpr int G8_BN = 128;
bool gemm8_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N);
size_t gemm8_workspace_bytes(int64_t M, int64_t K, int64_t N);
int gemm8_workgroups(int64_t M, int64_t K, int64_t N);   // tiles x K splits of its plan
hipError_t launch_gemm8(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s);

}  // namespace mcq4
