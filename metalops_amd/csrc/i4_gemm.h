// Shared arguments of the per-group INT4 / INT8 prefill GEMMs (i4_gemm,
// i4_gemm6): output tiles of BM x 256, optional split-K over grid.z with fp32
// partial tiles [tile][split][BM x 256] in the caller's workspace, summed by
// i4_gemm_reduce_kernel (which applies the fused activation).
#pragma once

#include "i4_common.h"

namespace mcq4 {

constexpr int I4G_BN = 256;

// Scale group of K step k (k < 2^16, spg < 2^16) without a division or a
// branch in the copy schedule: the high word of k times ceil(2^32 / spg), exact
// since k * (ceil(2^32 / spg) * spg - 2^32) < k * spg < 2^32 keeps the error
// below 1 / spg; for spg == 1 (ceil(2^32) does not fit) the multiplier is 0 and
// k itself passes through the mask.
__device__ __forceinline__ int i4_group_of(int k, uint32_t spg_magic, uint32_t spg_ident) {
    return (int)(__umulhi((uint32_t)k, spg_magic) + ((uint32_t)k & spg_ident));
}
inline uint32_t i4_spg_magic(int spg) {
    return spg > 1 ? (uint32_t)((((uint64_t)1 << 32) + (uint64_t)spg - 1) / (uint64_t)spg) : 0u;
}
inline uint32_t i4_spg_ident(int spg) { return spg == 1 ? 0xFFFFFFFFu : 0u; }

struct I4GemmArgs {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *P;
    const void *scales, *zeros;
    void *Y;
    int64_t ldy;
    int M, nsteps, N, spg;
    uint32_t spg_magic, spg_ident;   // i4_group_of's constants for spg
    int tiles_m, tiles_n;
    int S;               // K splits (grid.z)
    float *partials;     // [tiles][S][BM*256] when S > 1
    // i4_gemm6 with S == 2 and an XCD-local exchange: grid.x padded to a multiple
    // of 8, the second split of a tile to finish adds the first's partial and
    // stores act(sum) (64-bit tickets [8][4096] by blockIdx.x mod 8 at the
    // workspace start); null: i4_gemm_reduce_kernel.
    uint64_t *tickets = nullptr;
    uint32_t foreign = 0;    // splits treated as run on another XCD (test switch)
};

// Sums the S partial tiles per output tile in split order and stores act(sum) as fp16.
hipError_t launch_i4_gemm_reduce(const I4GemmArgs &a, int bm, int act, hipStream_t s);

}  // namespace mcq4
