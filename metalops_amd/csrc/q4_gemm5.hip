// Prefill-shaped q4_0 matmul (M > 64) on gfx950 with the activation tile
// staged once per workgroup in LDS.
//
//   * WG = 256 threads = 4 waves in a 2x2 grid; WG tile BM x 256 (BM = 256 or
//     128); wave tile (BM/2) x 128 of v_mfma_f32_32x32x16_f16, fp32
//     accumulation.  K advances one q4_0 block (32) per step and two steps per
//     stage.
//   * Activations: one stage of the workgroup's A tile (BM rows x 64 halves =
//     128 bytes per row) is copied by global_load_lds_dwordx4, every row piece
//     a whole 128-byte line, into one of G5_NS LDS slots.  Each of the four
//     waves copies a quarter of the rows.  Chunk c (16 bytes) of row r lands at
//     position 8r + (c ^ (r & 7)), so the MFMA operand reads (ds_read_b128 of
//     one chunk for 32 consecutive rows) touch every bank group once per eight
//     lanes.
//   * Weights: as in q4_gemm4, each wave copies the raw q4_0 bytes of its 128
//     columns (2304 contiguous bytes per step) into a private LDS ring and
//     builds the fp16 B operands itself: natural-order unpack to 1024 + q,
//     minus 1032 (exact), times d (one rounding: the reference's fp16 dequant
//     value).  Step k+1's B operands are built during step k's MFMAs.
//   * One barrier per stage: after a wave's own copies of stage s have landed
//     (vmcnt), the barrier makes every wave's copies visible and guarantees
//     that all waves finished reading stage s-1, whose slot the copies of
//     stage s + G5_NS - 1, issued right after the barrier, overwrite.
//   * Stages past the end re-copy the last stage (valid memory, never read),
//     so each stage issues the same number of copies and the vmcnt waits are
//     exact.
//   * Tile numbering, split-K partials and the reduction kernel are shared
//     with q4_gemm4.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_gemm4.h"

namespace mcq4 {

constexpr int G5_NS = 3;                       // stages (A slots) in flight
constexpr int G5_ROWB = 128;                   // A bytes per row and stage (2 steps)
constexpr int G5_RAW_W = 18 * 128;             // raw weight bytes per wave and step
constexpr int G5_RAW_SLOT = G5_RAW_W + 64;     // + read overhang
constexpr int G5_RAW_N = 2 * G5_NS;            // raw ring slots per wave (steps)

template <int BM>
constexpr size_t gemm5_lds_bytes() {
    return (size_t)G5_NS * BM * G5_ROWB + (size_t)4 * G5_RAW_N * G5_RAW_SLOT;
}

// SCHED: the interleaved pipeline (dequant chunks and next-A reads between the
// MFMAs, barrier between the two steps of a stage); otherwise a plain loop
// with the barrier at the stage start.

template <int BM, bool SCHED>
__global__ void __launch_bounds__(256, 1)
q4_gemm5_kernel(Gemm4Args a) {
    constexpr int WM = BM / 2, WN = G4_BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int A_SLOT = BM * G5_ROWB;
    constexpr int A_LD = BM / 32;                // A copies per wave and stage (BM*8 chunks / 256 lanes)
    constexpr int GROUP = A_LD + 6;              // vector-memory instructions per wave and stage
    static_assert((G5_NS - 2) * GROUP < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    const int ntiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x;
    int tile_id = bid;
    if (ntiles % 8 == 0) tile_id = (bid % 8) * (ntiles / 8) + bid / 8;
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * BM, n0 = tn * G4_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nb * z / a.S);
    const int nk = (int)((int64_t)a.nb * (z + 1) / a.S) - k_lo;
    const int nst = (nk + 1) >> 1;

    uint8_t *const sA = smem;
    uint8_t *const ring = smem + G5_NS * A_SLOT + wave * (G5_RAW_N * G5_RAW_SLOT);

    // ---- A copies: instruction u of this wave covers positions 64(wave*A_LD+u) + lane,
    // i.e. row 8(wave*A_LD+u) + lane/8 and chunk (lane ^ lane/8) & 7 of it (the
    // chunk is the same for every u).
    const int a_c = (lane ^ (lane >> 3)) & 7;
    const int a_t = a_c >> 2;
    const int a_r0 = m0 + 8 * wave * A_LD + (lane >> 3);
    const _Float16 *a_col = a.X + (int64_t)k_lo * QK + 8 * (a_c & 3);
    auto copy_a = [&](int s_src, int s_dst) {
        uint8_t *dst = sA + (s_dst % G5_NS) * A_SLOT + wave * (A_LD * 1024);
        const int64_t koff = (int64_t)min(2 * s_src + a_t, nk - 1) * QK;
#pragma unroll
        for (int u = 0; u < A_LD; ++u) {
            const int m = min(a_r0 + 8 * u, a.M - 1);
            __builtin_amdgcn_global_load_lds(
                (void *)(a_col + (int64_t)m * a.ldx + koff),
                (__attribute__((address_space(3))) void *)(dst + 1024 * u), 16, 0, 0);
        }
    };

    // ---- raw weight copies: bytes 0..2047 of the wave's 2304-byte segment as two
    // 16-byte-per-lane copies, bytes 2048..2303 as one 4-byte-per-lane copy.  No
    // copy is lane-masked: a masked copy lets the compiler split the surrounding
    // copies over divergent branches, which changes the number of vector-memory
    // instructions the vmcnt waits count on.
    const int64_t row_bytes = (int64_t)a.N * BLOCK_BYTES;
    const uint8_t *w_k = a.W + (int64_t)k_lo * row_bytes;
    const bool wcols = n0 + wn * WN < a.N;
    const uint8_t *w_seg = wcols ? w_k + (int64_t)(n0 + wn * WN) * BLOCK_BYTES : w_k;
    auto copy_raw = [&](int k_src, int k_dst) {
        const uint8_t *src = w_seg + (int64_t)k_src * row_bytes;
        uint8_t *dst = ring + (k_dst % G5_RAW_N) * G5_RAW_SLOT;
#pragma unroll
        for (int c = 0; c < 2; ++c)
            __builtin_amdgcn_global_load_lds(
                (void *)(src + 1024 * c + 16 * lane),
                (__attribute__((address_space(3))) void *)(dst + 1024 * c), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(
            (void *)(src + 2048 + 4 * lane),
            (__attribute__((address_space(3))) void *)(dst + 2048), 4, 0, 0);
    };
    // Copy ci (0 .. GROUP-1) of stage s_dst's group: A copies first, then the
    // raw copies (3 per step), in the order issue_stage uses.
    auto issue_one = [&](int s_dst, int ci) {
        const int s_src = min(s_dst, nst - 1);
        if (ci < A_LD) {
            uint8_t *dst = sA + (s_dst % G5_NS) * A_SLOT + wave * (A_LD * 1024) + 1024 * ci;
            const int64_t koff = (int64_t)min(2 * s_src + a_t, nk - 1) * QK;
            const int m = min(a_r0 + 8 * ci, a.M - 1);
            __builtin_amdgcn_global_load_lds(
                (void *)(a_col + (int64_t)m * a.ldx + koff),
                (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
            return;
        }
        const int r = ci - A_LD, t = r / 3, c = r % 3;
        const uint8_t *src = w_seg + (int64_t)min(2 * s_src + t, nk - 1) * row_bytes;
        uint8_t *dst = ring + ((2 * s_dst + t) % G5_RAW_N) * G5_RAW_SLOT;
        if (c < 2)
            __builtin_amdgcn_global_load_lds(
                (void *)(src + 1024 * c + 16 * lane),
                (__attribute__((address_space(3))) void *)(dst + 1024 * c), 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds(
                (void *)(src + 2048 + 4 * lane),
                (__attribute__((address_space(3))) void *)(dst + 2048), 4, 0, 0);
    };
    // Stage s_dst's slots get stage min(s_dst, nst - 1)'s data.
    auto issue_stage = [&](int s_dst) {
        const int s_src = min(s_dst, nst - 1);
        copy_a(s_src, s_dst);
        copy_raw(min(2 * s_src, nk - 1), 2 * s_dst);
        copy_raw(min(2 * s_src + 1, nk - 1), 2 * s_dst + 1);
    };

    // ---- operand reads ----------------------------------------------------------
    const int lrow = lane & 31, lhi = lane >> 5;
    // A operand (i, ks) of step t of a stage: row wm*WM + 32 i + lrow, chunk 4t + 2ks + lhi.
    uint32_t a_off[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            a_off[t][ks] = (uint32_t)((wm * WM + lrow) * G5_ROWB + (((4 * t + 2 * ks + lhi) ^ (lrow & 7)) << 4));
    auto read_a = [&](int s, int t, half8_t (&av)[2][TM]) {
        const uint32_t base = lds_addr(sA + (s % G5_NS) * A_SLOT);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
                av[ks][i] = *(const lds_half8 *)(lds_ptr(base + a_off[t][ks]) + i * 32 * G5_ROWB);
    };
    const int qoff0 = 18 * lrow + 2 + 4 * lhi;
    const int q_al = qoff0 & ~3;
    const uint32_t q_sh = (uint32_t)(qoff0 & 3) * 8;
    const int d_off = 18 * lrow;
    auto load_b = [&](int k, half8_t (&bv)[2][TN]) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k % G5_RAW_N) * G5_RAW_SLOT));
        uint32_t qd[TN][4], dd[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const lds_u32 *qp = (const lds_u32 *)(Rs + q_al + j * 32 * 18);
#pragma unroll
            for (int t = 0; t < 4; ++t) qd[j][t] = qp[t];
            dd[j] = *(const lds_u16 *)(Rs + d_off + j * 32 * 18);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const half2_t d2 = bitcast<half2_t>(__builtin_amdgcn_perm(dd[j], dd[j], 0x01000100u));
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                bv[ks][j] = dequant8_nat(__builtin_amdgcn_alignbit(qd[j][2 * ks + 1], qd[j][2 * ks], q_sh), d2);
        }
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto mfmas = [&](const half8_t (&av)[2][TM], const half8_t (&bv)[2][TN]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[ks][i], bv[ks][j], acc[i][j], 0, 0, 0);
    };

    if constexpr (SCHED) {
        // Interleaved pipeline.  A half step runs the 32 (BM 256) or 16 (BM 128)
        // MFMAs of one K step; after each MFMA it issues either one LDS read of
        // the next A operands (first and last slots) or one chunk (4-8 VALU) of
        // the dequant of the next B operands, with scheduling fences between the
        // groups so the MFMA pipe never waits behind a block of VALU.  The
        // barrier sits between the two steps of a stage: after it, the next
        // stage's A is readable and the slot of the current stage is free for
        // the copies of stage s + 3.
        constexpr int NMF = 2 * TM * TN;         // MFMAs per step
        constexpr int NA = 2 * TM;               // A operand reads per step
        constexpr int NSLOT = NMF - NA;          // MFMA slots carrying dequant chunks
        // With copies: the GROUP copies of stage cs go out one per two MFMAs,
        // so the address unit works through them while the MFMAs run.
        auto half_step = [&](auto with_copies, int cs, const half8_t (&A)[2][TM], const half8_t (&B)[2][TN],
                             int k_next, half8_t (&Bn)[2][TN], int a_s, int a_t, half8_t (&An)[2][TM]) {
#pragma clang fp contract(off)
            const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k_next % G5_RAW_N) * G5_RAW_SLOT));
            uint32_t qd[TN][4], dd[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const lds_u32 *qp = (const lds_u32 *)(Rs + q_al + j * 32 * 18);
#pragma unroll
                for (int t = 0; t < 4; ++t) qd[j][t] = qp[t];
                dd[j] = *(const lds_u16 *)(Rs + d_off + j * 32 * 18);
            }
            const uint32_t abase = lds_addr(sA + (a_s % G5_NS) * A_SLOT);
            const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
            const uint32_t C64 = 0x64646464u;
            uint32_t lo[2 * TN], hi[2 * TN];
            uint4_t uu[2 * TN];
            half2_t d2[TN];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int idx = 0; idx < NMF; ++idx) {
                const int ks = idx / (TM * TN), i = (idx / TN) % TM, j = idx % TN;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B[ks][j], acc[i][j], 0, 0, 0);
                // Next A: reads 0 .. NA/2-1 after the first MFMAs, the rest after the last ones.
                const int ar = idx < NA / 2 ? idx : (idx >= NMF - NA / 2 ? idx - (NMF - NA) : -1);
                if (ar >= 0) {
                    const int aks = ar / TM, ai = ar % TM;
                    An[aks][ai] = *(const lds_half8 *)(lds_ptr(abase + a_off[a_t][aks]) + ai * 32 * G5_ROWB);
                }
                if constexpr (decltype(with_copies)::value) {
                    constexpr int STRIDE = NMF / GROUP >= 2 ? 2 : 1;
                    if (idx % STRIDE == 1 % STRIDE && idx / STRIDE < GROUP) issue_one(cs, idx / STRIDE);
                }
                // Dequant chunks (24 per step: 3 per 8-weight unit) over the middle slots.
#pragma unroll
                for (int c = 0; c < 24; ++c) {
                    if (NA / 2 + (c * NSLOT) / 24 != idx) continue;
                    const int unit = c / 3, part = c % 3, uj = unit >> 1, uk = unit & 1;
                    if (part == 0) {
                        if (uk == 0) d2[uj] = bitcast<half2_t>(__builtin_amdgcn_perm(dd[uj], dd[uj], 0x01000100u));
                        const uint32_t w = __builtin_amdgcn_alignbit(qd[uj][2 * uk + 1], qd[uj][2 * uk], q_sh);
                        lo[unit] = w & 0x0F0F0F0Fu;
                        hi[unit] = (w >> 4) & 0x0F0F0F0Fu;
                    } else if (part == 1) {
                        const uint32_t e03 = __builtin_amdgcn_perm(hi[unit], lo[unit], 0x05010400u);
                        const uint32_t e47 = __builtin_amdgcn_perm(hi[unit], lo[unit], 0x07030602u);
                        uu[unit] = uint4_t{__builtin_amdgcn_perm(C64, e03, 0x04010400u),
                                           __builtin_amdgcn_perm(C64, e03, 0x04030402u),
                                           __builtin_amdgcn_perm(C64, e47, 0x04010400u),
                                           __builtin_amdgcn_perm(C64, e47, 0x04030402u)};
                    } else {
                        uint4_t r;
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            r[t] = bitcast<uint32_t>((bitcast<half2_t>(uu[unit][t]) - off) * d2[uj]);
                        Bn[uk][uj] = bitcast<half8_t>(r);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // Prologue: stages 0, 1, 2 in flight; stage 0 landed for every wave.
        issue_stage(0);
        issue_stage(1);
        issue_stage(2);
        wait_vmcnt<2 * GROUP>();
        lds_barrier();
        half8_t A0[2][TM], A1[2][TM], B0[2][TN], B1[2][TN];
        read_a(0, 0, A0);
        load_b(0, B0);
        const int nfull = nk >> 1;
        for (int s = 0; s < nfull; ++s) {
            // Step 2s; builds B(2s+1) from stage s's raw bytes, reads A(s, step 1).
            half_step(std::false_type{}, 0, A0, B0, 2 * s + 1, B1, s, 1, A1);
            wait_vmcnt<GROUP>();                 // stage s+1 (own copies) landed
            lds_barrier();                       // stage s+1 visible; stage s's slot read by all
            // Step 2s+1 with stage s+3's copies; builds B(2s+2) (stage s+1), reads
            // A(s+1, step 0).  Past the last step both are clamped re-reads of
            // valid slots.
            half_step(std::true_type{}, s + 3, A1, B1, min(2 * s + 2, nk - 1), B0, s + 1, 0, A0);
        }
        if (nk & 1) mfmas(A0, B0);               // last step alone
    } else {
        // ---- prologue: stages 0 .. NS-2 in flight --------------------------------------
    #pragma unroll
        for (int p = 0; p < G5_NS - 1; ++p) issue_stage(p);
        wait_vmcnt<(G5_NS - 2) * GROUP>();           // stage 0 (own copies) landed
        half8_t b0[2][TN], b1[2][TN];
        load_b(0, b0);

        // Full stages (both steps valid); the loop body has no data-dependent
        // branches, so the accumulators stay in place.  B of the step after the
        // stage (clamped to the last step: its slot still holds valid data) is
        // built during the stage's second step.
        const int nfull = nk >> 1;
        for (int s = 0; s < nfull; ++s) {
            wait_vmcnt<(G5_NS - 2) * GROUP>();       // stage s (own copies) landed
            lds_barrier();                           // all copies of stage s landed; stage s-1 read
            issue_stage(s + G5_NS - 1);
            const int k0 = 2 * s;
            half8_t av[2][TM], av1[2][TM];
            read_a(s, 0, av);
            load_b(k0 + 1, b1);
            mfmas(av, b0);
            read_a(s, 1, av1);
            wait_vmcnt<(G5_NS - 2) * GROUP>();       // stage s+1 (own copies) landed
            load_b(min(k0 + 2, nk - 1), b0);
            mfmas(av1, b1);
        }
        if (nk & 1) {                                // last step alone (its B is in b0)
            wait_vmcnt<(G5_NS - 2) * GROUP>();
            lds_barrier();
            half8_t av[2][TM];
            read_a(nfull, 0, av);
            mfmas(av, b0);
        }
    }
    wait_vmcnt<0>();

    // ---- epilogue ----------------------------------------------------------------
    const int rsub = 4 * lhi;
    if (a.S == 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wn * WN + j * 32 + lrow;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                    if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)acc[i][j][r];
                }
            }
        return;
    }
    float *part = a.partials + ((int64_t)tile_id * a.S + z) * (BM * G4_BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nl = wn * WN + j * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                part[ml * G4_BN + nl] = acc[i][j][r];
            }
        }
}

template <int BM, bool SCHED>
static hipError_t launch_g5(const Gemm4Args &a, hipStream_t s) {
    constexpr size_t lds = gemm5_lds_bytes<BM>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm5_kernel<BM, SCHED>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((q4_gemm5_kernel<BM, SCHED>), dim3(a.tiles_m * a.tiles_n, 1, a.S), dim3(256), lds, s, a);
    if (a.S > 1) return launch_gemm4_reduce(a, BM, s);
    return hipGetLastError();
}

// Same requirements as q4_gemm4: N % 128 == 0, 16-byte aligned W and X rows.
bool gemm5_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t K, int64_t N) {
    return N % 128 == 0 && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 &&
           K >= QK;
}

// Plan: 256-row tiles, K split (powers of two, at least 16 steps per split)
// until about 192 workgroups have work.  A full-height tile with a split-K sum
// beats a 128-row tile on these shapes (2048x14336x4096: 262 vs 350 us; the
// fp32 partials cost one extra pass over M x N x S floats).
// MCQ4_GEMM2_BM=128 and MCQ4_GEMM4_SPLIT override (experiments, tests).
G4Cfg gemm5_config(int64_t M, int64_t K, int64_t N) {
    G4Cfg c{256, 1};
    if (const char *env = getenv("MCQ4_GEMM2_BM")) c.bm = atoi(env) == 128 ? 128 : 256;
    const int64_t t = ((M + c.bm - 1) / c.bm) * ((N + G4_BN - 1) / G4_BN);
    const int64_t nb = K / QK;
    while (t * c.S < 192 && nb / (c.S * 2) >= 16 && c.S < 16) c.S *= 2;
    if (const char *env = getenv("MCQ4_GEMM4_SPLIT")) c.S = std::max(1, std::min(16, atoi(env)));
    if (c.S > nb) c.S = 1;
    return c;
}

size_t gemm5_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const G4Cfg c = gemm5_config(M, K, N);
    if (c.S == 1) return 0;
    const int64_t t = ((M + c.bm - 1) / c.bm) * ((N + G4_BN - 1) / G4_BN);
    return COUNTER_BYTES + (size_t)t * c.S * c.bm * G4_BN * sizeof(float);
}

hipError_t launch_gemm5(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    const G4Cfg c = gemm5_config(M, K, N);
    Gemm4Args a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.tiles_n = (N + G4_BN - 1) / G4_BN;
    a.tiles_m = (M + c.bm - 1) / c.bm;
    a.S = c.S;
    a.partials = nullptr;
    if (c.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    bool sched = true;
    if (const char *env = getenv("MCQ4_GEMM5_SCHED")) sched = env[0] != '0';
    if (c.bm == 256) return sched ? launch_g5<256, true>(a, s) : launch_g5<256, false>(a, s);
    return sched ? launch_g5<128, true>(a, s) : launch_g5<128, false>(a, s);
}

}  // namespace mcq4
