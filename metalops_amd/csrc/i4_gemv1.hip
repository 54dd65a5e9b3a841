// Decode per-group INT4 (M = 1..32) and INT8 (M = 1..16) GEMV on gfx950 with
// the weight stream in asynchronous global->LDS copies.
//
// Y[M][N] = X[M][K] @ W, W[k][n] = (q - z) * s per (group, column), packed[K/2][N]
// (byte row k/2: even k in the low nibble), fp16 activations, fp32 sums.  The
// roofline is HBM bandwidth: 0.5 byte per weight plus the group's scale/zero.
// The description below is the M == 1 form; the MR form (M >= 2) differs only
// where the kernel's MR comment says.
//
// Work decomposition
//   * Tile = 128 columns (whole 128-byte pieces of each byte row); step = 32 K
//     (16 byte rows, 2 KiB of the tile).  Workgroup (tile, split sp) = 8 waves;
//     wave w owns steps [(8 sp + w) spw, +spw).  The plan aims at one workgroup
//     per CU.
//   * Per wave, oldest first: one copy per group of the group's scale and zero
//     rows (128 columns each, one 1 KiB slot), one copy of the range's activations (up to 16
//     steps), then the steps: two global_load_lds_dwordx4 each (byte rows 0..7
//     and 8..15; lane l -> row l/8, 16-byte piece l%8) into a ring of I1_R
//     slots.  Step k+R-1 is issued into the slot step k-1 freed before the
//     wave waits for step k; steps past the range re-copy the last one, so the
//     vmcnt waits are exact.
//   * Lane (c = l%16, g = l/16): columns 8c..8c+7 of the tile, byte rows
//     4g..4g+3 of the step, i.e. K elements 8g..8g+7.  The K order inside the
//     MFMA is [e0, e2, e1, e3, e4, e6, e5, e7] (e = 8g + i): for column 8c+j, one
//     v_perm_b32 puts byte j of rows 4g and 4g+1 into bytes 0 and 2, and two
//     v_and_or_b32 give the fp16 pairs {1024 + q(e0), 1024 + q(e2)} (low
//     nibbles) and {1024 + 16 q(e1), 1024 + 16 q(e3)} (high nibbles in place).
//     The activations x' = [x0, x2, x1/16, x3/16, x4, x6, x5/16, x7/16] are
//     built once per step for all eight MFMAs.
//   * Per group: P_j = sum x' B_j (MFMA chain), C = sum x' (-1024) and
//     S = sum x' [1,1,16,16,1,1,16,16] = sum x; then acc_j += s_j (P_j + C - z_j S)
//     = s_j sum x (q - z) in fp32.  All 16 MFMA rows are the same activation
//     row, so element 0 of each result is used.
//   * Epilogue: the 8 waves' sums in wave order through LDS; with K split over
//     workgroups, the splits are summed in split order.  Default (XL): the
//     grid's x extent is a multiple of 8, so every split of a tile has the same
//     linear id mod 8 and runs on one XCD; the partials go through that XCD's L2
//     (plain stores, L1-bypassing loads); split 0 sums them once each other
//     split's flag shows its partial stored, and recomputes a split whose flag
//     comes from another XCD or not in time.  Otherwise agent-scope stores and
//     loads and a ticket, as in the general INT4 GEMV.  Store act(sum) as fp16.
//
// Int8 weights (WB = 8, W int8 [K][N], M <= 16): a step is 32 byte rows (4 KiB,
// four copies), lane (c, g) reads byte rows 8g..8g+7, the K order is natural,
// x' = x, and the B pair of rows 2p, 2p+1 is one v_perm_b32 and one xor with
// 0x64806480: fp16 1152 + q exactly (q + 128 in the low byte).  C uses -1152
// and S ones.
#include <algorithm>
#include <atomic>
#include <stdlib.h>

#include "i4_common.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(i4_gemv1_split_fallbacks)

constexpr int I1_W = 8;          // waves per workgroup
constexpr int I1_TC = 128;       // tile columns
constexpr int I1_STEP = 2048;    // 4-bit weight bytes per step and tile (16 byte rows x 128)
constexpr int I1_R = 2;          // ring slots (steps) per wave
constexpr int I1_XB = 1024;      // activation bytes per wave (16 steps)
constexpr int I1_SMAX = 16;      // K splits at most
constexpr int I1_NT = 2;         // cache policy of the weight copies: non-temporal (read once)

struct I4Gemv1Args {
    const _Float16 *X;
    const uint8_t *P;
    const void *scales, *zeros;
    _Float16 *Y;
    int K, N, nsteps, spg, spw, S;
    int spg_log2;         // log2(spg) when spg is a power of two, else -1
    int ngr_max;          // scale/zero slots per wave
    int wave_bytes;       // LDS bytes per wave
    int M;                // activation rows (1 .. 16)
    int64_t ldx, ldy;     // row strides of X and Y (elements)
    float *part;          // [tiles][S][M][128] when S > 1
    uint32_t *flags;      // XL: [tiles][S] split flags, behind the partials
    uint32_t spin;        // XL: polls of a flag before its split is recomputed
    uint32_t *counters;   // [tiles]
    uint32_t foreign;     // splits treated as run on another XCD (test switch)
    const _Float16 *wn;   // NORM: RMSNorm weight [K] (X is the raw row)
    float eps;            // NORM: RMSNorm epsilon
};

constexpr int I1_SZSLOT = 1024; // scale/zero bytes per group (one 16-byte-per-lane copy)
constexpr int I1_XSTEP = 1024;  // MR: a step's activations, 16 rows x 32 halves, after its weights

// RB = 0: M == 1.  RB = 1, 2 (the MR forms, M = 2..16 and 17..32): each ring
// slot also holds the step's activation blocks of 16 rows (one more
// 16-byte-per-lane copy per block and step: lane -> row min(16 rb + l/4, M-1),
// 8 halves 8(l%4)..), lane (c, g) feeds activation row 16 rb + c into block rb's
// MFMAs (the B operand is built once for all blocks), and the four output rows
// 4g..4g+3 of each column are all live.  RB = 2 runs one workgroup per CU (its
// registers fill the SIMDs).
//
// NORM (M == 1, 4-bit weights): the row is RMS-normalised in the kernel
// (fused_rmsnorm_linear_int4).  Each wave copies the norm weights of its range
// beside its activations and issues its first R steps; then the workgroup sums
// the squares of the whole row, an eighth per wave (register loads, after the
// copies so the weight stream starts as early as without the norm), combines
// the wave totals through LDS at one barrier (which also waits for every copy
// issued so far), and each wave normalises its activations in place before
// its first step.
template <int SZ, int ACT, bool XL, int RB, int WB, bool NORM = false>
__global__ void __launch_bounds__(I1_W * 64, RB == 2 ? 1 : 2)
i4_gemv1_kernel(I4Gemv1Args a) {
    static_assert(WB == 4 || (WB == 8 && RB < 2), "int8 form covers M <= 16");
    static_assert(!NORM || (RB == 0 && WB == 4 && ACT == ACT_NONE), "the fused norm is the M == 1 INT4 form");
    static_assert(!NORM || I1_W == RMS_WAVES, "the norm's sum order is per RMS_WAVES-wave workgroup");
    constexpr bool MR = RB > 0;
    constexpr int NB = MR ? RB : 1;              // row blocks
    constexpr int NR = MR ? 4 : 1;               // output rows per lane and block
    constexpr int WROWS = WB == 4 ? 16 : 32;     // weight byte rows per step
    constexpr int STEPW = WROWS * I1_TC;         // weight bytes per step
    constexpr int NCOPY = WROWS / 8 + (MR ? RB : 0);     // copies per step
    constexpr int STEPB = STEPW + (MR ? RB * I1_XSTEP : 0);   // ring slot bytes
    constexpr int ESZ = SZ == DT_F32 ? 4 : 2;
    constexpr int SLOT = I1_SZSLOT;
    constexpr int PPR = I1_TC * ESZ / 16;        // 16-byte pieces per scale (or zero) row
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int G = (int)gridDim.x, G8 = G & ~7;
    int t = (int)blockIdx.x;
    if (t < G8) t = (t & 7) * (G8 >> 3) + (t >> 3);      // consecutive tiles on one XCD
    if (XL && t >= a.N / I1_TC) return;                  // grid padding to a multiple of 8
    const int sp = (int)blockIdx.y;
    const int N = a.N;
    const int col0 = t * I1_TC;
    const int s_begin = (sp * I1_W + wave) * a.spw;
    // XL: the tile's split flags as this launch starts (lane q of wave 0: split q).
    uint32_t fb = 0;
    if (XL && a.S > 1 && wave == 0 && lane < a.S)
        fb = __hip_atomic_load(a.flags + t * a.S + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int ns = max(0, min(a.spw, a.nsteps - s_begin));

    // [ring R x STEPB][x 1 KiB, M == 1 only][norm weights 1 KiB, NORM only][s/z slots]
    uint8_t *const wl = smem + wave * a.wave_bytes;
    uint8_t *const ring = wl;
    uint8_t *const xs = wl + I1_R * STEPB;
    uint8_t *const wns = xs + I1_XB;
    uint8_t *const szs = xs + (MR ? 0 : I1_XB) + (NORM ? I1_XB : 0);

    float acc[NB][8][NR];
#pragma unroll
    for (int rb = 0; rb < NB; ++rb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < NR; ++i) acc[rb][j][i] = 0.f;

    // NORM: this workgroup's share of the row's sum of squares, the wave totals
    // through LDS behind the waves' areas, one barrier (every wave takes it once,
    // with or without steps), then rstd in every thread.
    auto norm_rstd = [&]() -> float {
        float *part = (float *)(smem + I1_W * a.wave_bytes);
        const float ss = rms_sumsq_part(a.X, a.K, tid, true);
        if (lane == 0) part[wave] = ss;
        __syncthreads();
        return rms_rstd(rms_sumsq_total(part), a.K, a.eps);
    };
    // rstd of the row, kept for the split-K recompute path (which rebuilds the
    // normalised activations of a split that ran on another XCD).
    float rstd_row = 0.f;
    if (NORM && ns == 0) rstd_row = norm_rstd();
    if (ns > 0) {
        // ---- scale/zero rows of the wave's groups, then its activations ----
        // Group of a step: a shift for the usual power-of-two group sizes (no
        // integer division ahead of the first copy), else a division.
        auto group_of = [&](int step) { return a.spg_log2 >= 0 ? step >> a.spg_log2 : step / a.spg; };
        const int g_first = group_of(s_begin);
        const int ngr = group_of(s_begin + ns - 1) - g_first + 1;      // <= ngr_max by launch
        {
            // One 16-byte-per-lane copy per group: the scale row's PPR pieces, then
            // the zero row's (slot bytes 0 .. 2*128*ESZ); for 16-bit dtypes lanes
            // 32..63 re-read lanes 0..31's pieces into the slot's unused half.
            const int li = lane % (2 * PPR);
            const bool is_z = li >= PPR;
            const uint8_t *src = (const uint8_t *)(is_z ? a.zeros : a.scales) +
                                 ((int64_t)g_first * N + col0) * ESZ + 16 * (li % PPR);
            for (int gl = 0; gl < ngr; ++gl)
                __builtin_amdgcn_global_load_lds(
                    (void *)(src + (int64_t)gl * N * ESZ),
                    (__attribute__((address_space(3))) void *)(szs + gl * SLOT), 16, 0, 0);
        }
        if constexpr (!MR) {
            // 16 halves-pieces of 8 activations; pieces past K re-read the last one.
            const int e = min(s_begin * 32 + 8 * lane, a.K - 8);
            __builtin_amdgcn_global_load_lds((void *)(a.X + e),
                                             (__attribute__((address_space(3))) void *)xs, 16, 0, 0);
            if constexpr (NORM)
                __builtin_amdgcn_global_load_lds((void *)(a.wn + e),
                                                 (__attribute__((address_space(3))) void *)wns, 16, 0, 0);
        }

        // ---- weight steps ----
        const uint8_t *wsrc = a.P + ((int64_t)s_begin * WROWS + (lane >> 3)) * N + col0 + 16 * (lane & 7);
        const _Float16 *xsrc[NB];
#pragma unroll
        for (int rb = 0; rb < NB; ++rb)
            xsrc[rb] = a.X + (int64_t)min(16 * rb + (lane >> 2), a.M - 1) * a.ldx + (int64_t)s_begin * 32 +
                       8 * (lane & 3);
        auto issue = [&](int k) {                     // step k of the range into slot k % R
            const int kk = min(k, ns - 1);
            const uint8_t *src = wsrc + (int64_t)kk * WROWS * N;
            uint8_t *dst = ring + (k % I1_R) * STEPB;
#pragma unroll
            for (int q = 0; q < WROWS / 8; ++q)           // byte rows 8q..8q+7
                __builtin_amdgcn_global_load_lds((void *)(src + (int64_t)8 * q * N),
                                                 (__attribute__((address_space(3))) void *)(dst + 1024 * q), 16, 0,
                                                 I1_NT);
            if constexpr (MR) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    __builtin_amdgcn_global_load_lds((void *)(xsrc[rb] + kk * 32),
                                                     (__attribute__((address_space(3))) void *)(dst + STEPW + I1_XSTEP * rb),
                                                     16, 0, 0);
            }
        };
#pragma unroll
        for (int k = 0; k < I1_R - (NORM ? 0 : 1); ++k) issue(k);
        if constexpr (NORM) {
            // The first R steps stay in flight while the row is summed; the
            // activations and norm weights have to have landed before they are
            // normalised (nothing left to wait for in practice: the loads in
            // norm_rstd are younger than every copy above).
            const float rstd = norm_rstd();
            rstd_row = rstd;
            wait_vmcnt<0>();
            typedef __attribute__((address_space(3))) half8_t lds_h8;
            lds_h8 *xp = (lds_h8 *)lds_ptr(lds_addr(xs + 16 * lane));
            const half8_t xv = *xp;
            const half8_t wv = *(const lds_h8 *)lds_ptr(lds_addr(wns + 16 * lane));
            half8_t nv;
#pragma unroll
            for (int i = 0; i < 8; ++i) nv[i] = rms_apply(xv[i], rstd, wv[i]);
            *xp = nv;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }

        const uint32_t c64 = opaque_vgpr(0x64006400u);
        const uint32_t mlo = opaque_sgpr(0x000F000Fu), mhi = opaque_sgpr(0x00F000F0u);
        constexpr uint32_t NEGC = WB == 4 ? 0xE400E400u : 0xE480E480u;     // -1024 / -1152
        constexpr uint32_t EW1 = WB == 4 ? 0x4C004C00u : 0x3C003C00u;      // 16 / 1
        const half8_t negc = bitcast<half8_t>(uint4_t{NEGC, NEGC, NEGC, NEGC});
        const half8_t ew = bitcast<half8_t>(uint4_t{0x3C003C00u, EW1, 0x3C003C00u, EW1});
        const half2_t s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
        const float4_t zf = {0.f, 0.f, 0.f, 0.f};
        float4_t P[NB][8], Cc[NB], Sx[NB];
#pragma unroll
        for (int rb = 0; rb < NB; ++rb) {
            Cc[rb] = zf;
            Sx[rb] = zf;
#pragma unroll
            for (int j = 0; j < 8; ++j) P[rb][j] = zf;
        }

        auto flush = [&](int gl) {
            const lds_u8 *sl = lds_ptr(lds_addr(szs + gl * SLOT));
            float sv[8], zv[8];
            if constexpr (SZ == DT_F32) {
                typedef __attribute__((address_space(3))) float4_t lds_f4;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float4_t s4 = *(const lds_f4 *)(sl + 32 * c + 16 * h);
                    const float4_t z4 = *(const lds_f4 *)(sl + 4 * I1_TC + 32 * c + 16 * h);
#pragma unroll
                    for (int i = 0; i < 4; ++i) { sv[4 * h + i] = s4[i]; zv[4 * h + i] = z4[i]; }
                }
            } else {
                const uint4_t s4 = *(const __attribute__((address_space(3))) uint4_t *)(sl + 16 * c);
                const uint4_t z4 = *(const __attribute__((address_space(3))) uint4_t *)(sl + 2 * I1_TC + 16 * c);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (SZ == DT_F16) {
                        const half2_t sh = bitcast<half2_t>(s4[i]), zh = bitcast<half2_t>(z4[i]);
                        sv[2 * i] = (float)sh[0]; sv[2 * i + 1] = (float)sh[1];
                        zv[2 * i] = (float)zh[0]; zv[2 * i + 1] = (float)zh[1];
                    } else {
                        sv[2 * i] = __uint_as_float(s4[i] << 16); sv[2 * i + 1] = __uint_as_float(s4[i] & 0xFFFF0000u);
                        zv[2 * i] = __uint_as_float(z4[i] << 16); zv[2 * i + 1] = __uint_as_float(z4[i] & 0xFFFF0000u);
                    }
                }
            }
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
#pragma unroll
                    for (int i = 0; i < NR; ++i) {
                        const float tq = __builtin_fmaf(-zv[j], Sx[rb][i], P[rb][j][i] + Cc[rb][i]);
                        acc[rb][j][i] = __builtin_fmaf(sv[j], tq, acc[rb][j][i]);
                    }
                    P[rb][j] = zf;
                }
                Cc[rb] = zf;
                Sx[rb] = zf;
            }
        };

        for (int k = 0; k < ns; ++k) {
            if (!NORM || k > 0) issue(k + I1_R - 1);
            wait_vmcnt<(I1_R - 1) * NCOPY>();      // step k (and everything older) landed
            // x' for this step: elements 8g..8g+7 of the step (of row 16 rb + c with MR).
            half8_t xq[NB];
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
                const uint4_t xv = *(const __attribute__((address_space(3))) uint4_t *)(lds_ptr(lds_addr(
                    MR ? ring + (k % I1_R) * STEPB + STEPW + I1_XSTEP * rb + 64 * c + 16 * g
                       : xs + k * 64 + 16 * g)));
                if constexpr (WB == 8) {
                    xq[rb] = bitcast<half8_t>(xv);
                    Cc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb], negc, Cc[rb], 0, 0, 0);
                    Sx[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb], ew, Sx[rb], 0, 0, 0);
                    continue;
                }
                const uint32_t x02 = __builtin_amdgcn_perm(xv[1], xv[0], 0x05040100u);     // x0, x2
                const uint32_t x13 = __builtin_amdgcn_perm(xv[1], xv[0], 0x07060302u);     // x1, x3
                const uint32_t x46 = __builtin_amdgcn_perm(xv[3], xv[2], 0x05040100u);     // x4, x6
                const uint32_t x57 = __builtin_amdgcn_perm(xv[3], xv[2], 0x07060302u);     // x5, x7
                xq[rb] = bitcast<half8_t>(uint4_t{x02, bitcast<uint32_t>(bitcast<half2_t>(x13) * s16),
                                                  x46, bitcast<uint32_t>(bitcast<half2_t>(x57) * s16)});
                Cc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb], negc, Cc[rb], 0, 0, 0);
                Sx[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb], ew, Sx[rb], 0, 0, 0);
            }
            // Byte rows (WROWS/4) g .. +WROWS/4-1, columns 8c..8c+7.
            constexpr int LR = WROWS / 4;
            const lds_u8 *rs = lds_ptr(lds_addr(ring + (k % I1_R) * STEPB + (LR * g) * I1_TC + 8 * c));
            u32x2 r[LR];
#pragma unroll
            for (int i = 0; i < LR; ++i) r[i] = *(const __attribute__((address_space(3))) u32x2 *)(rs + i * I1_TC);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int h = j >> 2, b = j & 3;
                // bytes 0 and 2 <- byte b of the first and second row of the pair
                // (v_perm_b32 selector values 0-3 pick bytes of the second operand, 4-7 of the first)
                const uint32_t sel = (uint32_t)b | (uint32_t)(4 + b) << 16 | 0x0C000C00u;
                uint4_t bq;
                if constexpr (WB == 4) {
                    const uint32_t p01 = __builtin_amdgcn_perm(r[1][h], r[0][h], sel);
                    const uint32_t p23 = __builtin_amdgcn_perm(r[3][h], r[2][h], sel);
                    bq = uint4_t{and_or(p01, mlo, c64), and_or(p01, mhi, c64),
                                 and_or(p23, mlo, c64), and_or(p23, mhi, c64)};
                } else {
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        bq[p] = __builtin_amdgcn_perm(r[2 * p + 1][h], r[2 * p][h], sel) ^ 0x64806480u;
                }
#pragma unroll
                for (int rb = 0; rb < NB; ++rb)
                    P[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[rb], bitcast<half8_t>(bq), P[rb][j], 0, 0, 0);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");     // slot reads done before its refill
            const int sg = s_begin + k;
            if ((sg + 1) % a.spg == 0 || k == ns - 1) flush(sg / a.spg - g_first);
        }
        wait_vmcnt<0>();
    }

    // ---- ordered sum over the waves, one row block at a time ----
    // Output v = row * 128 + column of the tile, rows < M (row 0 only for M == 1).
    constexpr int ROWS = MR ? 16 : 1;
    const int nout = (MR ? a.M : 1) * I1_TC;
    float *red = (float *)smem;                   // [8 waves][ROWS][128]
    auto y_at = [&](int v) -> _Float16 & { return a.Y[(int64_t)(v / I1_TC) * a.ldy + col0 + v % I1_TC]; };
    float *part = a.part + ((int64_t)t * a.S + sp) * nout;
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) {
        __syncthreads();                          // ring reads (or the previous block's sums) done
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int row = MR ? 4 * g + i : 0;
            if (MR ? 16 * rb + row < a.M : g == 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) red[(wave * ROWS + row) * I1_TC + 8 * c + j] = acc[rb][j][i];
            }
        }
        __syncthreads();
        const int nv = (MR ? min(16, a.M - 16 * rb) : 1) * I1_TC;
        for (int v = tid; v < nv; v += I1_W * 64) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < I1_W; ++w) sum += red[w * ROWS * I1_TC + v];
            const int vo = 16 * rb * I1_TC + v;
            if (a.S == 1) y_at(vo) = (_Float16)activate<ACT>(sum);
            else if (XL) part[vo] = sum;          // stays in the XCD's L2
            else __hip_atomic_store(part + vo, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (a.S == 1) return;
    // Split K.  XL: split 0 of the tile sums the partials (plain stores into
    // this XCD's L2, read back through it) in split order.  Every other split,
    // once its partial is stored, raises its flag: one word per (tile, split)
    // behind the partials, written only by that split, which adds 8 to the value
    // it read when the launch started and puts its XCD id in the low 3 bits.
    // Split 0 read the same starting values, so it waits (a bounded number of
    // polls, L1-bypassing loads) for each flag to reach start + 8; a flag that
    // does not arrive in time, or arrives from another XCD, has its split
    // recomputed from the inputs.  Nothing else writes the flags during a
    // launch, so a flag can only hold its starting value or this launch's
    // (whatever other kernels sharing the workspace left there before), and a
    // slow split whose flag was given up on only moves its own count.
    // Otherwise the partials go out write-through (agent-scope atomic stores),
    // one lane takes a ticket, and the last to draw reads them back with
    // L2-bypassing loads.
    wait_vmcnt<0>();
    __syncthreads();
    uint32_t *last_flag = (uint32_t *)smem;
    const float *base = a.part + (int64_t)t * a.S * nout;
    if constexpr (XL) {
        const uint32_t xcc = xcc_id();
        if (sp != 0) {
            if (wave == 0 && lane == sp)
                __hip_atomic_store(a.flags + t * a.S + sp, (fb & ~7u) + 8u + xcc, __ATOMIC_RELAXED,
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
                    v = __hip_atomic_load(a.flags + t * a.S + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        const uint32_t local = *last_flag;         // splits whose partial is in this L2
        constexpr int KS = 32;                     // K per step (both weight widths)
        for (int v = tid; v < nout; v += I1_W * 64) {
            float sum = 0.f;
            for (int q0 = 0; q0 < a.S; q0 += 8) {
                float pv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pv[i] = load_l2_f32(base, (min(q0 + i, a.S - 1) * nout + v) * 4);
                if (local != (1u << a.S) - 1) {    // splits from another XCD: recompute
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (q0 + i < a.S && !((local >> (q0 + i)) & 1))
                            pv[i] = i4_dot_range<WB, NORM>(a.X + (int64_t)(v / I1_TC) * a.ldx, a.P, a.scales,
                                                           a.zeros, SZ, N, a.spg * KS, col0 + v % I1_TC,
                                                           min((q0 + i) * I1_W * a.spw, a.nsteps) * KS,
                                                           min((q0 + i + 1) * I1_W * a.spw, a.nsteps) * KS,
                                                           a.wn, rstd_row);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (q0 + i < a.S) sum += pv[i];
            }
            y_at(v) = (_Float16)activate<ACT>(sum);
        }
        return;
    }
    if (tid == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(&a.counters[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last_flag = prev == (uint32_t)(a.S - 1) ? 1u : 0u;
        if (prev == (uint32_t)(a.S - 1)) __hip_atomic_store(&a.counters[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last_flag) return;
    for (int v = tid; v < nout; v += I1_W * 64) {
        float sum = 0.f;
        for (int q0 = 0; q0 < a.S; q0 += 8) {
            float pv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                pv[i] = __hip_atomic_load(base + (int64_t)min(q0 + i, a.S - 1) * nout + v, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (q0 + i < a.S) sum += pv[i];
        }
        y_at(v) = (_Float16)activate<ACT>(sum);
    }
}

struct I1Cfg {
    int spw, S, ngr_max;
};

// Plan: one 8-wave workgroup per CU.  K splits S = the most that keep the
// grid within 256 workgroups (at least 1, at most 16, and enough that a wave's
// range fits its 16-step activation slot), then steps per wave from S.
// Measured on the Llama-2-7B projections, graph replays: QKV 96 tiles x 2 splits
// 9.6 us (the previous plan's 96 x 6 = 576 workgroups, two rounds of the 512
// that fit two per CU: 10.6 us; 96 x 3: 12.1 us), gate/up 86 x 2 8.4 us (was
// 9.8), down 32 x 8 8.6 us (was 32 x 15: 9.7), O 32 x 8 5.8 us (unchanged).
// Deeper rings were slower on every shape: the decode layer 40.1 us with 2
// slots, 40.8 with 3, 43.0 with 4, 46.9 with 6 (same box).  MCQ4_I4_SPW1 overrides
// the steps per wave.
static I1Cfg i4_gemv1_config(int64_t K, int64_t N, int64_t gs) {
    const int64_t nsteps = K / 32, spg = gs / 32, ntiles = N / I1_TC;
    int64_t S = std::max<int64_t>(1, std::min<int64_t>(I1_SMAX, 256 / std::max<int64_t>(ntiles, 1)));
    S = std::max(S, (nsteps + I1_W * 16 - 1) / (I1_W * 16));
    int64_t spw = (nsteps + I1_W * S - 1) / (I1_W * S);
    if (const char *env = opt("MCQ4_I4_SPW1")) spw = atoi(env);
    spw = std::max<int64_t>(spw, (nsteps + I1_W * I1_SMAX - 1) / (I1_W * I1_SMAX));
    spw = std::min<int64_t>(std::max<int64_t>(spw, 2), 16);
    S = (nsteps + I1_W * spw - 1) / (I1_W * spw);
    const int64_t ngr = spw % spg == 0 ? spw / spg : (spw + spg - 1) / spg + 1;
    return {(int)spw, (int)S, (int)ngr};
}

static size_t i1_wave_bytes(int64_t M, const I1Cfg &c, int wb, bool norm = false) {
    const int rb = M > 16 ? 2 : 1;                // activation blocks per ring slot
    const size_t stepw = (size_t)I1_STEP * (wb / 4);
    return M > 1 ? (size_t)I1_R * (stepw + rb * I1_XSTEP) + c.ngr_max * I1_SZSLOT
                 : (size_t)I1_R * stepw + I1_XB * (norm ? 2 : 1) + c.ngr_max * I1_SZSLOT;
}

// LDS of a workgroup: the waves' rings and slots, and at least the epilogue's
// wave sums ([I1_W waves][16 rows][128] floats when M > 1), which reuse them.
static size_t i1_lds_bytes(int64_t M, size_t wave_bytes) {
    return std::max((size_t)I1_W * wave_bytes, (size_t)I1_W * (M > 1 ? 16 : 1) * I1_TC * sizeof(float));
}

// 1 <= M <= 32 with 4-bit weights (wb = 4), M <= 16 with int8 (wb = 8), whole 128-column tiles, group size a multiple
// of 32, 16-byte aligned operands (and activation rows), and a split count
// within bounds.  MCQ4_I4_GEMV1=0 disables it; =1 limits it to M == 1; =4 to 4-bit
// weights (int8 then runs the register-ring GEMV).  With the 2-slot ring this
// kernel ties the register ring on int8 at M <= 4 within 2% and beats it on
// 4096x11008 (M = 1: 11.7 against 15.2 us), so int8 comes here at every size.
bool i4_gemv1_supported(int64_t M, int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                        const void *P, const void *scales, const void *zeros, int wb) {
    int64_t mmax = wb == 4 ? 32 : 16;
    if (const char *env = opt("MCQ4_I4_GEMV1")) {
        if (env[0] == '0') return false;
        if (env[0] == '1') mmax = 1;
        if (env[0] == '4' && wb != 4) return false;     // 4-bit only
    }
    if (M < 1 || M > mmax || K < 32 || K % 32 || gs % 32 || N % I1_TC || N / I1_TC > COUNTER_SLOTS) return false;
    if (((uintptr_t)X % 16) || ((uintptr_t)P % 16) || ((uintptr_t)scales % 16) || ((uintptr_t)zeros % 16))
        return false;
    if (M > 1 && (ldx % 8 || ldx < K)) return false;
    const I1Cfg c = i4_gemv1_config(K, N, gs);
    return c.S <= I1_SMAX && i1_lds_bytes(M, i1_wave_bytes(M, c, wb)) <= 160 * 1024;
}

size_t i4_gemv1_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t gs) {
    const I1Cfg c = i4_gemv1_config(K, N, gs);
    if (c.S == 1) return 0;
    return COUNTER_BYTES + (size_t)(N / I1_TC) * c.S * std::max<int64_t>(M, 1) * I1_TC * sizeof(float) +
           (size_t)(N / I1_TC) * c.S * sizeof(uint32_t);
}

// The XCD-local exchange (default; MCQ4_XCD_LOCAL=0 selects the agent-scope
// one) needs K split, at most 4096 tiles per class of the padded grid, and the
// whole grid resident at once (split 0 waits for the other splits' flags): at
// most 256 workgroups.  Longer K on wide N can split further (K = 16384 at
// N = 32768: 1024 workgroups); those shapes take the agent-scope exchange,
// whose last arrival waits on nobody.
static bool use_xcd_local(int ntiles, int S) {
    return !opt_is("MCQ4_XCD_LOCAL", '0') && S > 1 && (ntiles + 7) / 8 <= 4096 && (ntiles + 7) / 8 * 8 * S <= 256;
}

template <int SZ, int ACT, bool XL, int RB, int WB, bool NORM = false>
static hipError_t launch_i1(const I4Gemv1Args &a, int ntiles, hipStream_t s) {
    const size_t lds = std::max(i1_lds_bytes(a.M, a.wave_bytes),
                                (size_t)I1_W * a.wave_bytes + (NORM ? RMS_WAVES * sizeof(float) : 0));
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)i4_gemv1_kernel<SZ, ACT, XL, RB, WB, NORM>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int gx = XL ? (ntiles + 7) / 8 * 8 : ntiles;
    hipLaunchKernelGGL((i4_gemv1_kernel<SZ, ACT, XL, RB, WB, NORM>), dim3(gx, a.S), dim3(I1_W * 64), lds, s, a);
    return hipGetLastError();
}

template <int SZ, int ACT, int WB>
static hipError_t launch_i1_xl(const I4Gemv1Args &a, int ntiles, hipStream_t s) {
    const bool xl = use_xcd_local(ntiles, a.S);
    if constexpr (WB == 4) {
        if (a.M > 16)
            return xl ? launch_i1<SZ, ACT, true, 2, WB>(a, ntiles, s) : launch_i1<SZ, ACT, false, 2, WB>(a, ntiles, s);
    } else {
        if (a.M > 16) return hipErrorInvalidValue;
    }
    if (a.M > 1) return xl ? launch_i1<SZ, ACT, true, 1, WB>(a, ntiles, s) : launch_i1<SZ, ACT, false, 1, WB>(a, ntiles, s);
    return xl ? launch_i1<SZ, ACT, true, 0, WB>(a, ntiles, s) : launch_i1<SZ, ACT, false, 0, WB>(a, ntiles, s);
}

template <int SZ, int WB>
static hipError_t launch_i1_act(const I4Gemv1Args &a, int ntiles, int act, hipStream_t s) {
    if (act == ACT_SILU) return launch_i1_xl<SZ, ACT_SILU, WB>(a, ntiles, s);
    if (act == ACT_GELU) return launch_i1_xl<SZ, ACT_GELU, WB>(a, ntiles, s);
    return launch_i1_xl<SZ, ACT_NONE, WB>(a, ntiles, s);
}

template <int SZ>
static hipError_t launch_i1_wb(const I4Gemv1Args &a, int ntiles, int act, int wb, hipStream_t s) {
    return wb == 8 ? launch_i1_act<SZ, 8>(a, ntiles, act, s) : launch_i1_act<SZ, 4>(a, ntiles, act, s);
}

// Arguments and LDS plan shared by the plain and the normalising launches.
static hipError_t i1_setup(I4Gemv1Args &a, const _Float16 *X, int64_t ldx, const uint8_t *P,
                           const void *scales, const void *zeros, _Float16 *Y, int64_t ldy, int M,
                           int K, int N, int gs, void *ws, int wb, bool norm) {
    const I1Cfg c = i4_gemv1_config(K, N, gs);
    a.X = X; a.P = P; a.scales = scales; a.zeros = zeros; a.Y = Y;
    a.K = K; a.N = N; a.nsteps = K / 32; a.spg = gs / 32; a.spw = c.spw; a.S = c.S;
    a.spg_log2 = -1;
    for (int b = 0; b < 30; ++b)
        if ((1 << b) == a.spg) a.spg_log2 = b;
    a.ngr_max = c.ngr_max;
    a.M = M; a.ldx = ldx; a.ldy = ldy;
    a.wave_bytes = (int)i1_wave_bytes(M, c, wb, norm);
    a.part = nullptr; a.flags = nullptr; a.counters = nullptr; a.foreign = split_foreign_mask();
    a.spin = split_spin();
    a.wn = nullptr; a.eps = 0.f;
    if (c.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.counters = (uint32_t *)ws;
        a.part = (float *)((char *)ws + COUNTER_BYTES);
        a.flags = (uint32_t *)(a.part + (int64_t)(N / I1_TC) * c.S * std::max(M, 1) * I1_TC);
    }
    if (i1_lds_bytes(M, a.wave_bytes) > 160 * 1024) return hipErrorInvalidValue;
    return hipSuccess;
}

hipError_t launch_i4_gemv1(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                           const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K, int N, int gs,
                           int act, void *ws, hipStream_t s, int wb) {
    if (wb != 4 && (wb != 8 || M > 16)) return hipErrorInvalidValue;
    I4Gemv1Args a;
    if (hipError_t e = i1_setup(a, X, ldx, P, scales, zeros, Y, ldy, M, K, N, gs, ws, wb, false)) return e;
    const int ntiles = N / I1_TC;
    if (sz_dt == DT_F32) return launch_i1_wb<DT_F32>(a, ntiles, act, wb, s);
    if (sz_dt == DT_F16) return launch_i1_wb<DT_F16>(a, ntiles, act, wb, s);
    return launch_i1_wb<DT_BF16>(a, ntiles, act, wb, s);
}

// fused_rmsnorm_linear_int4 at M == 1 in one launch: the shapes i4_gemv1 takes,
// a 16-byte aligned norm weight; MCQ4_I4_RMS_FUSE=0 keeps the two-kernel path.
bool i4_gemv1_rms_supported(int64_t K, int64_t N, int64_t gs, const void *X, const void *wn,
                            const void *P, const void *scales, const void *zeros) {
    if (opt_is("MCQ4_I4_RMS_FUSE", '0') || ((uintptr_t)wn % 16)) return false;
    if (!i4_gemv1_supported(1, K, N, gs, X, K, P, scales, zeros, 4)) return false;
    const I1Cfg c = i4_gemv1_config(K, N, gs);
    const size_t wave_bytes = i1_wave_bytes(1, c, 4, true);
    return std::max(i1_lds_bytes(1, wave_bytes), (size_t)I1_W * wave_bytes + RMS_WAVES * sizeof(float)) <=
           160 * 1024;
}

template <int SZ>
static hipError_t launch_i1_rms(const I4Gemv1Args &a, int ntiles, hipStream_t s) {
    return use_xcd_local(ntiles, a.S) ? launch_i1<SZ, ACT_NONE, true, 0, 4, true>(a, ntiles, s)
                                      : launch_i1<SZ, ACT_NONE, false, 0, 4, true>(a, ntiles, s);
}

hipError_t launch_i4_gemv1_rms(const _Float16 *X, const _Float16 *wn, float eps, const uint8_t *P,
                               const void *scales, const void *zeros, int sz_dt, _Float16 *Y, int K,
                               int N, int gs, void *ws, hipStream_t s) {
    I4Gemv1Args a;
    if (hipError_t e = i1_setup(a, X, K, P, scales, zeros, Y, N, 1, K, N, gs, ws, 4, true)) return e;
    a.wn = wn;
    a.eps = eps;
    const int ntiles = N / I1_TC;
    if (sz_dt == DT_F32) return launch_i1_rms<DT_F32>(a, ntiles, s);
    if (sz_dt == DT_F16) return launch_i1_rms<DT_F16>(a, ntiles, s);
    return launch_i1_rms<DT_BF16>(a, ntiles, s);
}

}  // namespace mcq4
