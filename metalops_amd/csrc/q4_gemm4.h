// Shared plan and arguments of the 256-column prefill GEMMs (q4_gemm4 and
// q4_gemm5): output tiles of BM x 256, optional split-K over grid.z with fp32
// partial tiles in the caller's workspace, summed by q4_gemm4_reduce_kernel.
#pragma once

#include "q4_common.h"

namespace mcq4 {

constexpr int G4_BN = 256;

struct Gemm4Args {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int tiles_m, tiles_n;
    int S;               // K splits (grid.z)
    float *partials;     // [tiles][S][BM*256] when S > 1
    // S == 2 with an XCD-local exchange: grid.x padded to a multiple of 8, the
    // second split of a tile to finish adds the first's partial and stores Y
    // (64-bit tickets [8][4096] by blockIdx.x mod 8 at the workspace start).
    uint64_t *tickets = nullptr;
};

// Row-tile height and number of K splits of a prefill shape.
struct G4Cfg {
    int bm, S;
};
G4Cfg gemm4_config(int64_t M, int64_t K, int64_t N);
// Plan of the LDS-staged kernels (q4_gemm5, q4_gemm6): 256-row tiles, split-K.
G4Cfg gemm5_config(int64_t M, int64_t K, int64_t N);

// Sums the S partial tiles per output tile in split order and stores fp16.
hipError_t launch_gemm4_reduce(const Gemm4Args &a, int bm, hipStream_t s);

}  // namespace mcq4
