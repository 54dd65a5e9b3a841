// Small-batch (2 <= M <= 32) q4_0 GEMV/GEMM on gfx950: the M = 1 kernel's
// structure (q4_gemv.hip) with a 16-row MFMA A operand.  launch_gemvm first hands
// M <= 16 to the span kernels of q4_gemv_span.hip where they fit (4096 < N <=
// 16384 at K <= 4096; N <= 4096 with long K, split along K) and runs this strip
// kernel for the rest.
//
//   * Column tile = 16 columns; item = one tile's batch of 8 K blocks (2304 bytes
//     of strip rows), copied with three global_load_lds_dwordx4 into a 2-slot
//     per-wave LDS ring; item k+1 is issued before the wave waits for item k.
//   * Workgroup = WAVES waves owning TPW tiles (XCD-renumbered); wave w owns
//     batches w, w+WAVES, ... of every tile, walked batch-major.
//   * Row groups: with GR distinct activation rows per 16-row MFMA (GR = 4 for
//     M <= 4, 8 for M <= 8, else 16), A row r holds activation row
//     min(r / (16/GR), M-1), so the four accumulator rows 4g..4g+3 of lane
//     (c, g) hold GR/4 distinct output rows, (4g+i) GR/16: one
//     fp32 update per K-block row at M <= 4 (as at M = 1), two at M <= 8, four
//     above (measured at M = 4: 4096x14336 8.6 against 9.6 us, 14336x4096 10.5
//     against 11.7 us).
//   * Activations: lane (r = l%16, g = l/16) holds row min(r / (16/GR), M-1)
//     (rows >= M only feed output rows that are never stored), elements 8g..8g+7 of each of
//     the batch's 8 K blocks, loaded from global memory into registers right
//     before the batch's first weight copy is issued (so the in-order vmcnt never
//     makes a weight wait stall behind them), then rearranged to
//     x' = [x0, x4, x1, x5, x2, x6, x3, x7].
//   * Per K block row: B = [1024+q0, 1024+q4, 64+q1, 64+q5, ...] from four
//     v_and_or_b32 (a high nibble left in place under the exponent of 64 is
//     64 + q), and mfma(x', B, -S) with -S = mfma(x', -C) of that row
//     (C = [1032, 1032, 72, 72, ...]) gives sum x*(q-8) for the lane's four
//     output rows 4g..4g+3 of column r; acc += d * that in fp32, four rows at a
//     time after their LDS reads and MFMAs.
//   * Epilogue: per-wave partials through LDS, summed over waves in order
//     (deterministic), stored as fp16 for rows < M.
#include <algorithm>
#include <atomic>

#include "q4_common.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(q4_gemvm_split_fallbacks)

constexpr int GM_B = 8;                      // K blocks per item
constexpr int GM_ROW = 288;                  // strip bytes per K block (16 columns)
constexpr int GM_WCH = GM_B * 18;            // 144 strip chunks per item
constexpr int GM_SLOT = GM_WCH * 16 + 64;    // + read overhang
constexpr int GM_TPW_MAX = 4;
constexpr int GM_NT = 2;                     // cache policy of the weight copies: non-temporal
#ifndef GM_GU_SET
constexpr int GM_GU = 4;                     // K-block rows unpacked per group
#else
constexpr int GM_GU = GM_GU_SET;
#endif

struct GemvMArgs {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N, ntiles, nbt;
    int S, bps;          // K splits (grid.y) and batches per split
    float *part;         // [S][M][16 * ntiles] fp32 partials when S > 1 (after the counter area)
    // S > 1 with the XCD-local exchange: grid.x padded to a multiple of 8, split 0
    // of each workgroup sums the partials once the other splits' flags ([grid.x][S]
    // words behind the partials) show them stored; null: the reduction kernel.
    uint32_t *flags;
    uint32_t spin;       // polls of a flag before its split is recomputed
    uint32_t foreign;    // splits treated as run on another XCD (test switch)
    // Columns of the last tile: 16, or 8 when N % 16 == 8 (its copies of chunks
    // 9..17 of a row re-read chunks 0..8; outputs past N are not stored).
    int tail_cols;
};

// RB row blocks of 16 activation rows (M <= 16 RB): each K-block row's B
// operand is built once and feeds the MFMAs of every row block.
// HOIST: every wave has at most one batch (launcher), so its activations are
// loaded once, and x' and -S are built once per wave: one MFMA per K-block row
// instead of two (the registers the next batch's activations would take hold -S).
template <int WAVES, int TPW, int RB, int GR, bool HOIST = false>
__global__ void __launch_bounds__(WAVES * 64)
q4_gemvm_kernel(GemvMArgs a) {
    static_assert(GR == 16 || (RB == 1 && (GR == 4 || GR == 8)), "row groups");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    // MFMA lane rows g = 0..3 take K quarters kq = 0, 2, 1, 3 of each block (the
    // activations to match): a 32-lane half then reads quarters {0, 2} or {1, 3}
    // of the 16 columns' nibbles, whose words fall on the 32 LDS banks with fewer
    // conflicts than {0, 1} / {2, 3} (M = 1: 9 against 11 cycles per four
    // half-wave reads, M >= 2: 8 against 12).
    const int kq = ((g & 1) << 1) | (g >> 1);
    const uint32_t grow = (uint32_t)a.N * BLOCK_BYTES;

    // LDS: [WAVES x 2 slots][partials: TPW x WAVES x 16 rows x 16 columns]
    uint8_t *ring = smem + wave * (2 * GM_SLOT);
    float *red = (float *)(smem + WAVES * 2 * GM_SLOT);

    const int G = (int)gridDim.x, G8 = G & ~7;
    int wg = (int)blockIdx.x;
    if (wg < G8) wg = (wg & 7) * (G8 >> 3) + (wg >> 3);
    // Tiles of this workgroup (wg + j G) by compares: no integer division ahead
    // of the first copy.
    int ntl = 0;
#pragma unroll
    for (int j = 0; j < TPW; ++j) ntl += wg + j * G < a.ntiles ? 1 : 0;
    if (ntl <= 0) return;                         // grid padding (XCD-local exchange)
    // This split's batches [b0, b0 + nbs); wave w owns b0 + w, b0 + w + WAVES, ...
    const int sp = (int)blockIdx.y;
    // XCD-local exchange: the workgroup's split flags as the launch starts (lane q
    // of wave 0: split q).
    uint32_t fb = 0;
    if (a.S > 1 && a.flags && wave == 0 && lane < a.S)
        fb = __hip_atomic_load(a.flags + wg * a.S + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int b0 = sp * a.bps;
    const int nbs = max(0, min(a.bps, a.nbt - b0));
    const int nbm = nbs > wave ? (nbs - wave + WAVES - 1) / WAVES : 0;
    const int nmine = nbm * ntl;

    int crow[3];
    uint32_t coff[3];
    uint32_t past8 = 0;                           // bit i: copy i's chunk lies past a row's 9th
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int q = lane + 64 * i;
        crow[i] = q < GM_WCH ? q / 18 : 0;
        coff[i] = q < GM_WCH ? (uint32_t)(q / 18) * grow + 16u * (uint32_t)(q % 18) : 0u;
        past8 |= (q < GM_WCH && q % 18 >= 9 ? 1u : 0u) << i;
    }
    const uint8_t *xrow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
        xrow[rb] = (const uint8_t *)a.X + (int64_t)min(16 * rb + c / (16 / GR), a.M - 1) * a.ldx * 2 + 16 * kq;
    uint4_t xr[RB][GM_B];
    auto load_x = [&](int m) {
        const int row0 = (b0 + wave + WAVES * m) * GM_B;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int u = 0; u < GM_B; ++u)
                xr[rb][u] = *(const uint4_t *)(xrow[rb] + (int64_t)min(row0 + u, a.nb - 1) * (QK * 2));
    };
    auto copy_item = [&](int m, int j, int slot) {
        const int row0 = (b0 + wave + WAVES * m) * GM_B;
        const int rows = min(GM_B, a.nb - row0);
        const uint8_t *wb = a.W + (int64_t)(wg + j * G) * GM_ROW + (int64_t)row0 * grow;
        // An 8-column last tile: chunks 9..17 of a row re-read chunks 0..8 (the
        // row's valid bytes; those columns are not stored).
        const bool half = a.tail_cols < 16 && wg + j * G == a.ntiles - 1;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            uint32_t off = crow[i] < rows ? coff[i] : coff[i] - (uint32_t)crow[i] * grow;
            if (half && ((past8 >> i) & 1)) off -= 144u;
            if (i < 2 || lane < GM_WCH - 128)
                __builtin_amdgcn_global_load_lds(
                    (void *)(wb + off),
                    (__attribute__((address_space(3))) void *)(ring + slot * GM_SLOT + 1024 * i),
                    16, 0, GM_NT);
        }
    };
    // Issue cursor: a batch's activation loads go right before its first copy.
    int im = 0, ij = 0, islot = 0;
    auto issue_next = [&]() {
        if (!HOIST && ij == 0) load_x(im);
        copy_item(im, ij, islot);
        islot ^= 1;
        if (++ij == ntl) { ij = 0; ++im; }
    };
    if constexpr (HOIST) {
        if (nmine > 0) load_x(0);
    }
    if (nmine > 0) issue_next();

    const int qoff = c * BLOCK_BYTES + 2 + 4 * kq;
    const uint32_t qal = (uint32_t)(qoff & ~3), qsh = (uint32_t)(qoff & 3) * 8;
    const uint32_t doff = (uint32_t)(c * BLOCK_BYTES);
    // fp16 exponent words: 1024 + q for a low nibble, 64 + q for a high nibble
    // left in place (bits 4..7 of the half: 64 * (1 + 16q/1024)).
    const uint32_t e1024 = opaque_vgpr(0x64006400u), e64 = opaque_vgpr(0x54005400u);
    const uint32_t mlo = opaque_sgpr(0x000F000Fu), mhi = opaque_sgpr(0x00F000F0u);
    const uint32_t nlo = 0xE408E408u, nhi = 0xD480D480u;     // -1032, -72 pairs
    const half8_t negc = bitcast<half8_t>(uint4_t{nlo, nhi, nlo, nhi});
    const float4_t z = {0.f, 0.f, 0.f, 0.f};

    float4_t acc[RB][TPW];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < TPW; ++j) acc[rb][j] = z;

    int k = 0, slot = 0;
    for (int m = 0; m < nbm; ++m) {
        const int rows = min(GM_B, a.nb - (b0 + wave + WAVES * m) * GM_B);
        half8_t xq[RB][GM_B];
        float4_t nsh[HOIST ? RB : 1][HOIST ? GM_B : 1];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int u = 0; u < GM_B; ++u) {
            const uint4_t x = xr[rb][u];
            const uint4_t v = {__builtin_amdgcn_perm(x[2], x[0], 0x05040100u),     // x0, x4
                               __builtin_amdgcn_perm(x[2], x[0], 0x07060302u),     // x1, x5
                               __builtin_amdgcn_perm(x[3], x[1], 0x05040100u),     // x2, x6
                               __builtin_amdgcn_perm(x[3], x[1], 0x07060302u)};    // x3, x7
            xq[rb][u] = bitcast<half8_t>(v);
            if constexpr (HOIST) nsh[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb][u], negc, z, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            if (j < ntl) {
                // Younger than item k after this issue: the next item's 3 copies,
                // plus its batch's 8 activation loads when it starts a batch.
                const bool more = k + 1 < nmine;
                const bool xnext = more && ij == 0;
                if (more) issue_next();
                if (!more) wait_vmcnt<0>();
                else if (xnext) wait_vmcnt<RB * GM_B + 3>();
                else wait_vmcnt<3>();
                const uint32_t base = lds_addr(ring + slot * GM_SLOT);
                const uint32_t qa = base + qal, da = base + doff;
                // GU K-block rows at a time: their LDS reads first, then the
                // unpacks and MFMAs, then the scaled sums, so a wave is not
                // serialised on LDS and MFMA latency row by row.
                constexpr int GU = GM_GU;
                auto rows4 = [&](int u0, int nrows) {
                    uint32_t q0[GU], q1[GU];
                    float d[GU];
#pragma unroll
                    for (int v = 0; v < GU; ++v) {
                        const lds_u32 *qp = (const lds_u32 *)(lds_ptr(qa) + (u0 + v) * GM_ROW);
                        q0[v] = qp[0];
                        q1[v] = qp[1];
                        d[v] = (float)bitcast<_Float16>(*(const lds_u16 *)(lds_ptr(da) + (u0 + v) * GM_ROW));
                    }
                    float4_t blk[RB][GU];
#pragma unroll
                    for (int v = 0; v < GU; ++v) {
                        const int u = u0 + v;
                        const uint32_t w = __builtin_amdgcn_alignbit(q1[v], q0[v], qsh);
                        const uint32_t w8 = __builtin_amdgcn_alignbit(q1[v], q0[v], qsh + 8);
                        const uint4_t bq = {and_or(w, mlo, e1024), and_or(w, mhi, e64),
                                            and_or(w8, mlo, e1024), and_or(w8, mhi, e64)};
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb) {
                            // -S of this row, recomputed per item unless hoisted: keeps 32
                            // VGPRs free so a 16-wave workgroup fits in 128 VGPRs.
                            float4_t ns;
                            if constexpr (HOIST) ns = nsh[rb][u];
                            else ns = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb][u], negc, z, 0, 0, 0);
                            blk[rb][v] =
                                __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb][u], bitcast<half8_t>(bq), ns, 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int v = 0; v < GU; ++v) {
                        if (v >= nrows) break;
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb) {
                            if constexpr (GR == 4) {
                                acc[rb][j][0] += d[v] * blk[rb][v][0];
                            } else if constexpr (GR == 8) {
                                acc[rb][j][0] += d[v] * blk[rb][v][0];
                                acc[rb][j][2] += d[v] * blk[rb][v][2];
                            } else {
                                acc[rb][j] += d[v] * blk[rb][v];
                            }
                        }
                    }
                };
                if (rows == GM_B) {
#pragma unroll
                    for (int u0 = 0; u0 < GM_B; u0 += GU) rows4(u0, GU);
                } else {
                    // Rows past K hold a copy of row 0 (valid data, never summed).
#pragma unroll
                    for (int u0 = 0; u0 < GM_B; u0 += GU)
                        if (u0 < rows) rows4(u0, min(rows - u0, GU));
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                slot ^= 1;
                ++k;
            }
        }
    }

    // Partials: lane (c, g) holds rows 4g..4g+3 of column c (of row block rb).
    // One row block at a time through the LDS partial area.
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (rb > 0) __syncthreads();              // the previous block's sums are read
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (j < ntl) {
                // Accumulator i of lane (c, g) is output row (4g + i) GR / 16.
#pragma unroll
                for (int i = 0; i < 4; i += 16 / GR)
                    red[((j * WAVES + wave) * 16 + (4 * g + i) * GR / 16) * 16 + c] = nbm > 0 ? acc[rb][j][i] : 0.f;
            }
        __syncthreads();
        for (int v = tid; v < ntl * 256; v += WAVES * 64) {
            const int j = v >> 8, rr = 16 * rb + ((v >> 4) & 15), col = v & 15;
            if (rr >= a.M) continue;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) s += red[((j * WAVES + w) * 16 + (rr & 15)) * 16 + col];
            const int n = (wg + j * G) * 16 + col;
            if (a.S == 1) {
                if (n < a.N) a.Y[(int64_t)rr * a.ldy + n] = (_Float16)s;
            }
            else a.part[((int64_t)sp * a.M + rr) * (16 * a.ntiles) + n] = s;
        }
    }
    if (a.S == 1 || !a.flags) return;
    // Every split of this workgroup runs on this XCD (same blockIdx.x, grid.x a
    // multiple of 8).  Split 0 sums the partials, in split order as the reduction
    // kernel does, from the XCD's L2 (its own too with RB > 1: the LDS area holds
    // only the last row block's wave sums), once each other split's flag shows
    // its partial stored.  A flag is one word per (workgroup, split), written only
    // by that split, which adds 8 to the value it held when the launch started and
    // puts its XCD id in the low 3 bits; split 0 read the same starting values and
    // polls (at most a.spin times).  A split whose flag comes from another XCD, or
    // not in time, is recomputed from the inputs.
    wait_vmcnt<0>();
    __syncthreads();
    const uint32_t xcc = xcc_id();
    uint32_t *last_flag = (uint32_t *)smem;       // the ring is idle from here
    if (sp != 0) {
        if (wave == 0 && lane == sp)
            __hip_atomic_store(a.flags + wg * a.S + sp, (fb & ~7u) + 8u + xcc, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        return;
    }
    if (wave == 0) {
        const bool mine = lane >= 1 && lane < a.S;
        const uint32_t want = (fb & ~7u) + 8u;
        uint32_t v = 0;
        bool seen = !mine;
        for (uint32_t it = 0; it < a.spin; ++it) {
            if (!seen) {
                v = __hip_atomic_load(a.flags + wg * a.S + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                seen = (v & ~7u) == want;
            }
            if (__all(seen)) break;
            __builtin_amdgcn_s_sleep(1);
        }
        const uint64_t good = __ballot(mine && seen && (v & 7u) == xcc);
        if (lane == 0) {
            const uint32_t local = ((uint32_t)good | 1u) & ~a.foreign;
            *last_flag = local;
            if (local != (1u << a.S) - 1) note_split_fallback();
        }
    }
    __syncthreads();
    const uint32_t lf = *last_flag;
    const uint32_t local = lf;                     // splits whose partial is in this L2
    const int64_t pstride = (int64_t)a.M * 16 * a.ntiles;         // floats per split
    for (int v = tid; v < TPW * 256 * RB; v += WAVES * 64) {   // v = (rb, j, row, col)
        const int j = (v >> 8) % TPW, rr = 16 * (v / (256 * TPW)) + ((v >> 4) & 15), col = v & 15;
        const int n = (wg + j * G) * 16 + col;
        if (j >= ntl || rr >= a.M || n >= a.N) continue;          // (columns past N: none stored)
        float own = 0.f;
        if (RB == 1) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) own += red[((j * WAVES + w) * 16 + rr) * 16 + col];
        }
        const float *base = a.part + (int64_t)rr * (16 * a.ntiles) + n;
        float pv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            pv[q] = q < a.S && (RB > 1 || q != sp) && ((local >> q) & 1)
                        ? load_l2_f32(a.part, (int)(((int64_t)q * pstride + (base - a.part)) * 4)) : own;
        if (local != (1u << a.S) - 1) {            // splits from another XCD: recompute
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (q < a.S && !((local >> q) & 1))
                    pv[q] = q4_dot_range(a.X + (int64_t)rr * a.ldx, a.W, a.N, n, min(q * a.bps * GM_B, a.nb),
                                         min((q + 1) * a.bps * GM_B, a.nb));
        }
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q)
            if (q < a.S) t += pv[q];
        a.Y[(int64_t)rr * a.ldy + n] = (_Float16)t;
    }
}

// Sums the S fp32 partials of every output in split order (deterministic) and
// stores fp16; the kernel boundary orders it after the GEMV.
__global__ void __launch_bounds__(256) q4_gemvm_reduce_kernel(GemvMArgs a) {
    const int nc = 16 * a.ntiles;
    const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (v >= (int64_t)a.M * nc) return;
    const int rr = (int)(v / nc), n = (int)(v % nc);
    float s = 0.f;
    for (int sp = 0; sp < a.S; ++sp) s += a.part[((int64_t)sp * a.M + rr) * nc + n];
    if (n < a.N) a.Y[(int64_t)rr * a.ldy + n] = (_Float16)s;
}

static size_t gemvm_lds_bytes(int waves, int tpw) {
    return (size_t)waves * 2 * GM_SLOT + (size_t)tpw * waves * 256 * sizeof(float);
}

template <int WAVES, int TPW, int RB, int GR, bool HOIST>
static hipError_t launch_gemvm_t(const GemvMArgs &a, int grid, hipStream_t s) {
    const size_t lds = gemvm_lds_bytes(WAVES, TPW);
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemvm_kernel<WAVES, TPW, RB, GR, HOIST>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int gx = a.flags ? (grid + 7) / 8 * 8 : grid;
    hipLaunchKernelGGL((q4_gemvm_kernel<WAVES, TPW, RB, GR, HOIST>), dim3(gx, a.S), dim3(WAVES * 64), lds, s, a);
    if (a.S > 1 && !a.flags) {
        const int64_t n = (int64_t)a.M * 16 * a.ntiles;
        hipLaunchKernelGGL(q4_gemvm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

template <int WAVES, int RB, int GR, bool HOIST>
static hipError_t launch_gemvm_h(const GemvMArgs &a, int grid, int tpw, hipStream_t s) {
    switch (tpw) {
        case 1: return launch_gemvm_t<WAVES, 1, RB, GR, HOIST>(a, grid, s);
        case 2: return launch_gemvm_t<WAVES, 2, RB, GR, HOIST>(a, grid, s);
        case 3: return launch_gemvm_t<WAVES, 3, RB, GR, HOIST>(a, grid, s);
        default: return launch_gemvm_t<WAVES, 4, RB, GR, HOIST>(a, grid, s);
    }
}

template <int WAVES, int RB, int GR = 16>
static hipError_t launch_gemvm_w(const GemvMArgs &a, int grid, int tpw, bool hoist, hipStream_t s) {
    if constexpr (RB == 1) {
        if (hoist) return launch_gemvm_h<WAVES, RB, GR, true>(a, grid, tpw, s);
    }
    return launch_gemvm_h<WAVES, RB, GR, false>(a, grid, tpw, s);
}

// 2 <= M <= 32 (two row blocks above 16), 16-byte aligned weights and
// activation rows, N % 8 == 0, at least one 16-column tile and at most 4 tiles
// per workgroup on a 512-workgroup grid (N <= 32768).
bool gemvm_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K,
                     int64_t N) {
    if (opt_is("MCQ4_GEMV_PATH", 'o')) return false;
    return M >= 2 && M <= 32 && N % 8 == 0 && N >= 16 && N / 16 <= 512 * GM_TPW_MAX &&
           ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 && K >= QK &&
           N * 18 * 8 < ((int64_t)1 << 31);
}

// K split: with one tile per 16-wave workgroup every workgroup reads the whole
// activation block (M x K halves) from L2, and at M >= 8 those loads -- one
// line per row per instruction -- outnumber the weight copies.  Two tiles per
// workgroup over half of K each keeps 256 workgroups and halves the activation
// traffic; the fp32 partials are summed in split order by split 0 of each
// workgroup (XCD-local exchange) or, with MCQ4_XCD_LOCAL=0, by a second kernel
// (M=16 K=14336 N=4096: 15.6 us with the second kernel, was 18.7; M=8: 13.4,
// was 14.3).  Up to 16 rows the split goes on until every wave has one batch
// at most, the form with the activations and -S built once per wave (M=4
// K=14336 N=4096: 11.6 us with four splits against 12.2 with none; M=8: 12.4
// against 12.5 with two).  MCQ4_GEMVM_SPLIT=1|2|4|8 overrides.
struct GmPlan {
    int waves, tpw, grid, S, bps;
};
static GmPlan gemvm_plan(int64_t M, int64_t K, int64_t N) {
    const int ntiles = (int)((N + 15) / 16), nbt = (int)((K / QK + GM_B - 1) / GM_B);
    int waves = 16;
    // Two row blocks: 8-wave workgroups, one per CU (their registers fill the SIMDs).
    if (M > 16) waves = 8;
    const int cap = waves == 8 && M <= 16 ? 512 : 256;
    int S = 1;
    if (M <= 16) {
        if (ntiles <= cap)
            while (S < 8 && (nbt + S - 1) / S > waves) S *= 2;
    } else if (ntiles <= cap && nbt >= 2 * waves) {
        S = 2;
    }
    if (const char *env = opt("MCQ4_GEMVM_SPLIT")) {
        const int v = atoi(env);
        S = v == 2 || v == 4 || v == 8 ? v : 1;
    }
    S = std::max(1, std::min(S, nbt));
    // Without a split: every CU gets a workgroup (tiles wg, wg + grid, ...: three
    // or four each at N = 14336) rather than ceil(ntiles / 4) full ones.
    const int grid0 = S > 1 ? 0 : std::min(ntiles, cap);
    const int tpw = S > 1 ? std::min(GM_TPW_MAX, S) : std::min(GM_TPW_MAX, (ntiles + grid0 - 1) / grid0);
    const int grid = S > 1 ? (ntiles + tpw - 1) / tpw : std::max(grid0, (ntiles + tpw - 1) / tpw);
    const int bps = (nbt + S - 1) / S;
    return {waves, tpw, grid, (nbt + bps - 1) / bps, bps};
}

size_t gemv_span_split_workspace_bytes(int64_t M, int64_t K, int64_t N);

size_t gemvm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M < 2 || M > 32 || N < 16 || K < QK) return 0;
    const GmPlan p = gemvm_plan(M, K, N);
    // Partials follow the workspace's counter area, which other kernels rely on staying zero.
    const size_t own = p.S > 1 ? COUNTER_BYTES + (size_t)p.S * M * ((N + 15) / 16) * 16 * sizeof(float) +
                                     (size_t)(p.grid + 7) / 8 * 8 * p.S * sizeof(uint32_t)
                               : 0;
    return std::max(own, gemv_span_split_workspace_bytes(M, K, N));
}

bool gemv_span_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N);
hipError_t launch_gemv_span(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y, int64_t ldy, int M,
                            int K, int N, hipStream_t s);
bool gemv_span_split_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N);
hipError_t launch_gemv_span_split(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y, int64_t ldy,
                                  int M, int K, int N, void *ws, hipStream_t s);

hipError_t launch_gemvm(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, int *n_done, hipStream_t s) {
    // M <= 16 with 4096 < N <= 16384 at K <= 4096: contiguous spans of 16-column
    // groups per workgroup (q4_gemv_span.hip), no K split and no workspace.
    if (gemv_span_supported(X, ldx, W, M, K, N)) {
        *n_done = N;
        return launch_gemv_span(X, ldx, W, Y, ldy, M, K, N, s);
    }
    // 2 <= M <= 16 at N <= 4096: 64-column spans over K splits, summed through the
    // XCD's L2 (q4_gemv_span.hip).
    if (ws && gemv_span_split_supported(X, ldx, W, M, K, N)) {
        *n_done = N;
        return launch_gemv_span_split(X, ldx, W, Y, ldy, M, K, N, ws, s);
    }
    GemvMArgs a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.ntiles = (N + 15) / 16;
    a.tail_cols = N % 16 ? N % 16 : 16;
    a.nbt = (a.nb + GM_B - 1) / GM_B;
    *n_done = N;
    const GmPlan p = gemvm_plan(M, K, N);
    a.S = p.S; a.bps = p.bps;
    a.part = nullptr;
    a.flags = nullptr;
    a.spin = split_spin();
    a.foreign = split_foreign_mask();
    if (p.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.part = (float *)((char *)ws + COUNTER_BYTES);
        // Split 0 waits for the other splits' flags, so the exchange needs every
        // workgroup resident at once (one per CU); a larger grid (only a forced
        // MCQ4_GEMVM_SPLIT makes one) sums in the reduction kernel instead.
        if (!opt_is("MCQ4_XCD_LOCAL", '0') && p.S <= 8 && (p.grid + 7) / 8 * 8 * p.S <= 256)
            a.flags = (uint32_t *)(a.part + (int64_t)p.S * M * a.ntiles * 16);
    }
    // One batch per wave at most: the activations and -S once per wave
    // (MCQ4_GEMVM_HOIST=0 turns it off).
    const bool hoist = p.bps <= p.waves && !opt_is("MCQ4_GEMVM_HOIST", '0');
    if (M > 16) return launch_gemvm_w<8, 2>(a, p.grid, p.tpw, hoist, s);
    // M <= 16: 16-wave workgroups (gemvm_plan).
    if (M <= 4) return launch_gemvm_w<16, 1, 4>(a, p.grid, p.tpw, hoist, s);
    if (M <= 8) return launch_gemvm_w<16, 1, 8>(a, p.grid, p.tpw, hoist, s);
    return launch_gemvm_w<16, 1>(a, p.grid, p.tpw, hoist, s);
}

}  // namespace mcq4
