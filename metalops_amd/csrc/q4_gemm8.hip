// Prefill-shaped q4_0 matmul for outputs with few tiles (M = 512, N = 4096:
// 64 tiles of 128 x 256) on gfx950: 128 x 128 workgroup tiles, one workgroup
// per CU, K split four ways inside the workgroup.
//
//   * Waves (wn, ph): CW = G8_CW column groups of 128 / CW columns times four
//     K phases.  A stage is four K blocks; phase ph computes block 4s + ph of
//     stage s.  CW = 2 (the default): eight waves, two per SIMD, each a
//     128 x 64 tile of v_mfma_f32_32x32x16_f16 (the wave tile of the 128 x 256
//     kernel); CW = 1: four waves of 128 x 128 (256 accumulators in AGPRs).
//     Measured at M = 512, 11008 x 4096: 55.7 against 60.4 us.
//   * Activations: one 128-row x 256-byte slot per stage (the four phases' K
//     blocks side by side), G8_NS slots, 16-byte chunk c of row r at position
//     c ^ (r & 7); the waves copy 128 / (4 CW) rows each.  A operands are
//     reloaded in place right after their last MFMA of the current stage.
//   * Weights: each wave copies the raw bytes of its columns in its K block
//     (18 per column, contiguous in the [K/32][N][18] layout) into a private
//     ring, and builds its B operands one stage ahead, spread over the stage's
//     MFMAs.  The weights of stage t go out with the activations of stage
//     t - G8_WD (G8_NS = 4 and G8_WD = -1: activations three stages ahead,
//     weights two; 54.9 against 55.7 us for 3 and +2).
//   * All copies are buffer loads into LDS: one add per activation copy (its
//     VGPR offset, which the resource's size bounds), scalar offsets for the
//     weights.
//   * One barrier per stage; stage s + G8_NS's activations go out during stage s.
//   * End: the four phases' accumulators are summed in LDS (reduce-scatter:
//     wave (wn, ph) ends with rows 32 ph .. 32 ph + 31 of its columns), so the
//     epilogue's stores spread over all waves.
//   * Two K splits across workgroups (grid.z) at most: both run on one XCD and
//     the second to finish adds the first's fp32 partial from that XCD's L2
//     (see xcd_ticket_inc) -- 64 KB of partials per workgroup, no reduction
//     kernel.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_prefill.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(q4_gemm8_split_fallbacks)

constexpr int G8_PH = 4;                          // K phases per workgroup
#ifdef G8_NS_SET
constexpr int G8_NS = G8_NS_SET;
#else
constexpr int G8_NS = 4;                          // activation stages in LDS
#endif
constexpr int G8_ROWB = 64 * G8_PH;               // activation bytes per row and stage
constexpr int G8_A_SLOT = G8_BM * G8_ROWB;        // 32 KB
#ifdef G8_WD_SET
constexpr int G8_WD = G8_WD_SET;
#else
constexpr int G8_WD = -1;                         // weight copies lead the activations' by this many stages
#endif
#ifdef G8_CW_SET
constexpr int G8_CW = G8_CW_SET;
#else
constexpr int G8_CW = 2;                          // column groups of waves per tile (1 or 2)
#endif
constexpr int G8_RAW_N = G8_NS + G8_WD;           // raw ring slots per wave
// Raw bytes per wave and K block: 18 per column of its 128 / CW columns; with 64
// columns the remainder copy's 32 idle lanes re-read into the slot's tail.
constexpr int g8_raw_slot(int cw) { return cw == 1 ? 18 * G8_BN : 1280; }
// + 16: the B operand reads of the last ring slot run up to 4 bytes past it.
constexpr size_t g8_lds(int cw) {
    const size_t pipe = (size_t)G8_NS * G8_A_SLOT + (size_t)G8_PH * cw * G8_RAW_N * g8_raw_slot(cw) + 16;
    // Phase sum: cw x 2 row blocks x 3 sources, each 64 lanes x 64 / cw floats.
    const size_t sum = (size_t)2 * 3 * 64 * 64 * 4;
    return pipe > sum ? pipe : sum;
}
static_assert(g8_lds(1) <= 160 * 1024 && g8_lds(2) <= 160 * 1024, "LDS budget: one workgroup per CU");

__global__ void __launch_bounds__(64 * G8_PH * G8_CW, 1)
q4_gemm8_kernel(Gemm6Args a) {
    constexpr int CW = G8_CW;
    constexpr int NW = G8_PH * CW;                // waves
    constexpr int WN = G8_BN / CW;                // columns per wave
    constexpr int TM = 4, TN = WN / 32;           // 128 x WN wave tiles
    constexpr int A_LD = G8_A_SLOT / (16 * 64 * NW);   // activation copies per wave and stage
    constexpr int W_LD = CW == 1 ? 3 : 2;         // weight copies per wave and stage
    constexpr int RAW_SLOT = g8_raw_slot(CW);
    constexpr int SUM_REGION = 64 * 16 * TN * 4;  // one wave's 32 x WN fp32 block
    constexpr int GROUP = A_LD + W_LD;            // vector-memory instructions per wave and stage
    constexpr int NMF = 2 * TM * TN;              // MFMAs per stage (16 at CW = 2)
    static_assert(2 * GROUP <= NMF, "copies ride on the stage's odd MFMAs");
    // Stage t's weights go out with stage t - G8_WD's activations, after them.
    // Copies still allowed in flight once the stage the next barrier admits has
    // landed (its activations and weights): with G8_WD > 0, the rest of the
    // activations' group and the later groups; otherwise the groups after the
    // one that carries its weights.  The prologue allows one group more.
    constexpr int WAIT_LOOP = G8_WD > 0 ? W_LD + (G8_NS - 2) * GROUP : (G8_NS - 2 + G8_WD) * GROUP;
    constexpr int WAIT_PRO = WAIT_LOOP + GROUP;
    static_assert(G8_NS + G8_WD >= 2 && WAIT_LOOP >= 0 && WAIT_PRO < 64, "copy schedule");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % CW, ph = wave / CW;

    const int ntiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x, gx = gridDim.x;
    int tile_id = bid;
    if (gx % 8 == 0) tile_id = (bid % 8) * (gx / 8) + bid / 8;
    if (tile_id >= ntiles) return;                // grid padding (XCD-local exchange)
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * G8_BM, n0 = tn * G8_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nb * z / a.S);
    const int nk = (int)((int64_t)a.nb * (z + 1) / a.S) - k_lo;
    const int nst = (nk + G8_PH - 1) / G8_PH;

    uint8_t *const sA = smem;
    uint8_t *const ring = smem + G8_NS * G8_A_SLOT + wave * (G8_RAW_N * RAW_SLOT);

    // Activation copy u of this wave covers rows 4 (A_LD wave + u) .. +3: lane l
    // fills row 4 (A_LD wave + u) + l/16 (A_LD even) at position l % 16 with chunk
    // (l % 16) ^ (row & 7) = (l % 16) ^ (4 (u & 1) + l/16).  Chunk c is K block
    // 4s + c/4 of the stage, halves 8 (c % 4) .. +7 of it.  Buffer loads: the
    // lane's byte offset plus the stage's K offset is the VGPR offset, which
    // the hardware checks against the resource's size (the activations' last
    // byte; the scalar offset is outside that check), so reads past the end
    // return zero.  K blocks past the split's end are read but used by no MFMA
    // (the phases they belong to skip their last stage).
    const int a_ce = (lane & 15) ^ (lane >> 4), a_co = a_ce ^ 4;
    const __amdgpu_buffer_rsrc_t a_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.X, (short)0, (int)(((int64_t)(a.M - 1) * a.ldx + (int64_t)a.nb * QK) * 2), 0x00020000);
    uint32_t a_vo[A_LD];
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
        const int c = (u & 1) ? a_co : a_ce;
        const int m = min(m0 + 4 * (A_LD * wave + u) + (lane >> 4), a.M - 1);
        a_vo[u] = ((uint32_t)m * (uint32_t)a.ldx + 8 * (c & 3)) * 2 + (c >> 2) * 64;
    }

    // Weights: one K block of the wave's WN columns is 18 WN contiguous bytes
    // at k * row_bytes + 18 (n0 + WN wn) (W below 2^31 bytes).
    const uint32_t row_bytes = (uint32_t)a.N * BLOCK_BYTES;
    const __amdgpu_buffer_rsrc_t w_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.W, (short)0, (int)0x7fffffff, 0x00020000);
    const uint32_t w_so0 = (uint32_t)k_lo * row_bytes + (uint32_t)(n0 + WN * wn) * BLOCK_BYTES;
    const uint32_t w_vo16 = 16 * lane, w_vo4 = 4 * (CW == 1 ? lane : min(lane, 31));

    // Copy ci (0 .. GROUP-1) issued for activation stage s_dst: A_LD activation
    // copies of stage s_dst, then this wave's K block of stage s_dst + G8_WD:
    // 128 columns, bytes 0..2047 (two copies of 16 per lane) and 2048..2303 (4
    // per lane); 64 columns, bytes 0..1023 and 1024..1151 (4 per lane for lanes
    // 0..31; lanes 32..63 re-read lane 31's dword into the slot's unused tail,
    // so no lane is masked and nothing past the segment is read).
    // Weight K blocks past the split's end re-copy its last block.
    auto issue_a = [&](int s_dst, int u) {
        uint8_t *dst = sA + (s_dst % G8_NS) * G8_A_SLOT + (A_LD * wave + u) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, (__attribute__((address_space(3))) void *)dst, 16,
                                                 a_vo[u] + (uint32_t)(k_lo + G8_PH * s_dst) * (QK * 2), 0, 0, 0);
    };
    auto issue_w = [&](int s_w, int r) {
        const uint32_t so = w_so0 + (uint32_t)min(G8_PH * s_w + ph, nk - 1) * row_bytes;
        uint8_t *dst = ring + (s_w % G8_RAW_N) * RAW_SLOT;
        // (The instruction's immediate offset would move the LDS destination
        // too, so the piece offsets go into the scalar offset.)
        if (r < W_LD - 1)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (__attribute__((address_space(3))) void *)(dst + 1024 * r),
                                                     16, w_vo16, so + 1024 * r, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (__attribute__((address_space(3))) void *)(dst + 1024 * r), 4,
                                                     w_vo4, so + 1024 * r, 0, 0);
    };
    auto issue_one = [&](int s_dst, int ci) {
        if (ci < A_LD) issue_a(s_dst, ci);
        else issue_w(s_dst + G8_WD, ci - A_LD);
    };

    const int lrow = lane & 31, lhi = lane >> 5;
    // A operand (i, ks): row 32 i + lrow, chunk 4 ph + 2 ks + lhi.
    uint32_t a_off[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        a_off[ks] = (uint32_t)(lrow * G8_ROWB + (((4 * ph + 2 * ks + lhi) ^ (lrow & 7)) << 4));
    auto read_a1 = [&](int s, int ks, int i) {
        const uint32_t base = lds_addr(sA + (s % G8_NS) * G8_A_SLOT);
        return *(const lds_half8 *)(lds_ptr(base + a_off[ks]) + i * 32 * G8_ROWB);
    };
    // B operand (ks, j): column 32 j + lrow, K elements 16 ks + 8 lhi .. +8 of
    // the block: qs bytes 2 + 8 ks + 4 lhi .. +4 of the column's 18-byte block,
    // byte q_b + u of the dword pair at q_al.  Dequant of one B dword (elements
    // 2u, 2u + 1 of the lane's eight): v_perm_b32 puts byte u into bytes 0 and
    // 2, v_and_or_b32 keeps the low nibble in byte 0 and the high nibble in
    // place in byte 2 and adds the exponent bytes 0x64 and 0x54, giving the
    // fp16 pair {1024 + q0, 64 + q1} exactly; minus {1032, 72} (exact) gives
    // q - 8, and one multiply by d the single rounding of the exact product --
    // the reference's fp16 dequant value.  4 VALU per two weights.
    const int qoff0 = 18 * lrow + 2 + 4 * lhi;
    const int q_al = qoff0 & ~3;
    const int q_b = qoff0 & 3;
    const int d_off = 18 * lrow;
    uint32_t bsel[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) bsel[u] = (uint32_t)(q_b + u) * 0x00010001u + 0x0C000C00u;
    const uint32_t nib_mask = opaque_sgpr(0x00F0000Fu), exp_bits = opaque_vgpr(0x54006400u);
    auto dq2 = [&](uint32_t hi_w, uint32_t lo_w, int u, half2_t d2) {
#pragma clang fp contract(off)
        const half2_t off = {(_Float16)1032.0f, (_Float16)72.0f};
        const half2_t h = bitcast<half2_t>(and_or(__builtin_amdgcn_perm(hi_w, lo_w, bsel[u]), nib_mask, exp_bits));
        return bitcast<uint32_t>((h - off) * d2);
    };
    auto load_b = [&](int s, half8_t (&bv)[2][TN]) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (s % G8_RAW_N) * RAW_SLOT));
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const lds_u32 *qp = (const lds_u32 *)(Rs + q_al + j * 32 * 18);
            uint32_t qd[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) qd[t] = qp[t];
            const uint32_t dd = *(const lds_u16 *)(Rs + d_off + j * 32 * 18);
            const half2_t d2 = bitcast<half2_t>(__builtin_amdgcn_perm(dd, dd, 0x01000100u));
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                uint4_t r;
#pragma unroll
                for (int u = 0; u < 4; ++u) r[u] = dq2(qd[2 * ks + 1], qd[2 * ks], u, d2);
                bv[ks][j] = bitcast<half8_t>(r);
            }
        }
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // One stage: the NMF MFMAs of (A, B), ordered ks, i, j.  The next stage's B
    // is NMF dwords (d = 4 unit + u, unit = 2 j + ks): after MFMA idx the
    // perm and and_or of dword idx - 1 and the subtract and multiply of dword
    // idx - 2 (so neither waits on the raw words just read nor on its own
    // first half), the rest after the last MFMA; also the in-place reload of
    // the A operand whose last use this was (stage s_next), and copy idx/2 of
    // stage cs after every odd MFMA.
    static_assert(NMF == 8 * TN, "one B dword per MFMA");
    half8_t A[2][TM];
    auto stage = [&](int cs, const half8_t (&B)[2][TN], int s_next, half8_t (&Bn)[2][TN]) {
#pragma clang fp contract(off)
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (s_next % G8_RAW_N) * RAW_SLOT));
        uint32_t qd[TN][4], dd[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const lds_u32 *qp = (const lds_u32 *)(Rs + q_al + j * 32 * 18);
#pragma unroll
            for (int t = 0; t < 4; ++t) qd[j][t] = qp[t];
            dd[j] = *(const lds_u16 *)(Rs + d_off + j * 32 * 18);
        }
        const half2_t off = {(_Float16)1032.0f, (_Float16)72.0f};
        half2_t d2[TN];
        uint32_t xw[NMF];
        uint4_t bb[2 * TN];
        auto first = [&](int d) {
            const int unit = d >> 2, u = d & 3, uj = unit >> 1, uk = unit & 1;
            if (u == 0 && uk == 0) d2[uj] = bitcast<half2_t>(__builtin_amdgcn_perm(dd[uj], dd[uj], 0x01000100u));
            xw[d] = and_or(__builtin_amdgcn_perm(qd[uj][2 * uk + 1], qd[uj][2 * uk], bsel[u]), nib_mask, exp_bits);
        };
        auto second = [&](int d) {
            const int unit = d >> 2, u = d & 3, uj = unit >> 1, uk = unit & 1;
            bb[unit][u] = bitcast<uint32_t>((bitcast<half2_t>(xw[d]) - off) * d2[uj]);
            if (u == 3) Bn[uk][uj] = bitcast<half8_t>(bb[unit]);
        };
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int idx = 0; idx < NMF; ++idx) {
            const int ks = idx / (TM * TN), i = (idx / TN) % TM, j = idx % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B[ks][j], acc[i][j], 0, 0, 0);
            if (j == TN - 1) A[ks][i] = read_a1(s_next, ks, i);
            if ((idx & 1) == 1 && (idx >> 1) < GROUP) issue_one(cs, idx >> 1);
            if (idx >= 2) second(idx - 2);
            if (idx >= 1) first(idx - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        second(NMF - 2);
        first(NMF - 1);
        second(NMF - 1);
    };

    // Prologue: the weights of stages 0 .. G8_WD-1, then activation stages
    // 0 .. G8_NS-1, each with the weights of stage s + G8_WD when that is one.
#pragma unroll
    for (int s = 0; s < G8_WD; ++s)
#pragma unroll
        for (int r = 0; r < W_LD; ++r) issue_w(s, r);
#pragma unroll
    for (int s = 0; s < G8_NS; ++s)
#pragma unroll
        for (int ci = 0; ci < GROUP; ++ci)
            if (ci < A_LD || s + G8_WD >= 0) issue_one(s, ci);
    wait_vmcnt<WAIT_PRO>();
    lds_barrier();
    half8_t B0[2][TN], B1[2][TN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < TM; ++i) A[ks][i] = read_a1(0, ks, i);
    load_b(0, B0);
    // Stage s: stage s+1 landed (own copies) and visible to all, and every
    // wave is past stage s-1, so slot s % G8_NS is free for stage s + G8_NS.
    int s = 0;
    for (; s + 2 < nst; s += 2) {
        wait_vmcnt<WAIT_LOOP>();
        lds_barrier();
        stage(s + G8_NS, B0, s + 1, B1);
        wait_vmcnt<WAIT_LOOP>();
        lds_barrier();
        stage(s + 1 + G8_NS, B1, s + 2, B0);
    }
    if (s + 1 < nst) {
        wait_vmcnt<WAIT_LOOP>();
        lds_barrier();
        stage(s + G8_NS, B0, s + 1, B1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int j = 0; j < TN; ++j) B0[ks][j] = B1[ks][j];
    }
    // The split's last stage (A and B loaded): phases past its last K block skip it.
    if (G8_PH * (nst - 1) + ph < nk) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B0[ks][j], acc[i][j], 0, 0, 0);
    }
    wait_vmcnt<0>();
    lds_barrier();                                // every copy landed; LDS free for the phase sum

    // Phase sum, two rounds of two 32-row blocks: every wave writes its
    // accumulators of the blocks other phases own, the owner adds the three
    // in phase order after its own.
    float4_t *const sum = (float4_t *)smem;
#pragma unroll
    for (int R = 0; R < 2; ++R) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int i = 2 * R + ii;
            if (ph != i) {
                const int k = (ph - i - 1) & 3;
                float4_t *dst = sum + ((wn * 2 + ii) * 3 + k) * (SUM_REGION / 16) + lane;
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4)
                        dst[(j * 4 + r4) * 64] = float4_t{acc[i][j][4 * r4], acc[i][j][4 * r4 + 1],
                                                          acc[i][j][4 * r4 + 2], acc[i][j][4 * r4 + 3]};
            }
        }
        lds_barrier();
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int i = 2 * R + ii;
            if (ph == i) {
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const float4_t *src = sum + ((wn * 2 + ii) * 3 + k) * (SUM_REGION / 16) + lane;
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            const float4_t v = src[(j * 4 + r4) * 64];
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc[i][j][4 * r4 + e] += v[e];
                        }
                }
            }
        }
        lds_barrier();
    }
    float16_t fin[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
        if (ph == i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) fin[j] = acc[i][j];
        }

    // Wave (wn, ph) holds rows 32 ph + 8 (r/4) + 4 lhi + r%4, columns WN wn + 32 j + lrow.
    const int rsub = 32 * ph + 4 * lhi;
    if (a.S == 1) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + WN * wn + j * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + rsub + 8 * (r >> 2) + (r & 3);
                if (m < a.M) a.Y[(int64_t)m * a.ldy + n] = (_Float16)fin[j][r];
            }
        }
        return;
    }
    constexpr int TILE = G8_BM * G8_BN;
    float *part = a.partials + ((int64_t)tile_id * 2 + z) * TILE;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int nl = WN * wn + j * 32 + lrow;
#pragma unroll
        for (int r = 0; r < 16; ++r) part[(rsub + 8 * (r >> 2) + (r & 3)) * G8_BN + nl] = fin[j][r];
    }
    // Both splits of this tile run on this XCD (same blockIdx.x, grid.x a
    // multiple of 8): the partials stay in its L2.  The second to arrive adds
    // the other's partial in split order and stores Y.
    wait_vmcnt<0>();
    __syncthreads();
    uint64_t *cnt = a.tickets + (bid & 7) * 4096 + (bid >> 3);
    const uint32_t xcc = xcc_id();
    uint32_t *last_flag = (uint32_t *)smem;
    if (tid == 0) {
        const uint64_t inc = xcd_ticket_inc(xcc, z);
        const uint64_t prev = __hip_atomic_fetch_add(cnt, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // 1: the other split ran on this XCD (read its partial from the L2);
        // 2: it did not (recompute it here).
        *last_flag = (prev & 0xFF) != 1 ? 0u : (xcd_ticket_local_mask(prev + inc, xcc, 2) & ~a.foreign) == 3u ? 1u : 2u;
        // Both splits have drawn: the slot is free for the next launch.
        if ((prev & 0xFF) == 1) __hip_atomic_store(cnt, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (*last_flag == 2u) note_split_fallback();
    }
    __syncthreads();
    const uint32_t lf = *last_flag;
    if (!lf) return;
    float *other = a.partials + ((int64_t)tile_id * 2 + (1 - z)) * TILE;
    if (lf == 2) {
        // The other split ran on another XCD: its partial is not in this L2.
        // Recompute it here into its slot, then read it back as usual.
        const int o_lo = (int)((int64_t)a.nb * (1 - z) / 2), o_hi = (int)((int64_t)a.nb * (2 - z) / 2);
#pragma unroll 1
        for (int v = tid; v < TILE; v += 64 * NW) {
            const int m = min(m0 + v / G8_BN, a.M - 1), n = n0 + v % G8_BN;
            other[v] = q4_dot_range(a.X + (int64_t)m * a.ldx, a.W, a.N, n, o_lo, o_hi);
        }
        wait_vmcnt<0>();
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int nl = WN * wn + j * 32 + lrow;
        float o[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) o[r] = load_l2_f32(other, ((rsub + 8 * (r >> 2) + (r & 3)) * G8_BN + nl) * 4);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + rsub + 8 * (r >> 2) + (r & 3), n = n0 + nl;
            const float v = z == 0 ? fin[j][r] + o[r] : o[r] + fin[j][r];   // p0 + p1 in split order
            if (m < a.M) a.Y[(int64_t)m * a.ldy + n] = (_Float16)v;
        }
    }
}

// Plan: two K splits when the 128 x 128 tiles alone fill at most half the
// CUs and each split keeps at least 16 K blocks; otherwise none.
// MCQ4_GEMM8_SPLIT=1|2 overrides (tests).
static int gemm8_splits(int64_t M, int64_t K, int64_t N) {
    const int64_t t = ((M + G8_BM - 1) / G8_BM) * (N / G8_BN);
    const int64_t nb = K / QK;
    int S = (t * 2 <= 256 && nb / 2 >= 16) ? 2 : 1;
    if (const char *env = opt("MCQ4_GEMM8_SPLIT")) S = atoi(env) == 2 ? 2 : 1;
    if (S > nb) S = 1;
    return S;
}

int gemm8_workgroups(int64_t M, int64_t K, int64_t N) {
    if (N % G8_BN) return 0;
    return (int)(((M + G8_BM - 1) / G8_BM) * (N / G8_BN) * gemm8_splits(M, K, N));
}

bool gemm8_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N) {
    if (!(N % G8_BN == 0 && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 && K >= QK &&
          M * ldx < ((int64_t)1 << 30) && (K / QK) * N * BLOCK_BYTES < ((int64_t)1 << 31)))
        return false;
    // Two splits exchange through the XCD's L2 only; MCQ4_XCD_LOCAL=0 leaves
    // such shapes to the other prefill kernels.
    if (gemm8_splits(M, K, N) == 2) {
        const int64_t t = ((M + G8_BM - 1) / G8_BM) * (N / G8_BN);
        if (opt_is("MCQ4_XCD_LOCAL", '0') || (t + 7) / 8 > 4096) return false;
    }
    return true;
}

size_t gemm8_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (N % G8_BN || gemm8_splits(M, K, N) == 1) return 0;
    const int64_t t = ((M + G8_BM - 1) / G8_BM) * (N / G8_BN);
    return COUNTER_BYTES + (size_t)t * 2 * G8_BM * G8_BN * sizeof(float);
}

hipError_t launch_gemm8(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    if (!gemm8_supported(X, ldx, W, M, K, N)) return hipErrorInvalidValue;
    Gemm6Args a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.tiles_n = N / G8_BN;
    a.tiles_m = (M + G8_BM - 1) / G8_BM;
    a.S = gemm8_splits(M, K, N);
    a.partials = nullptr;
    a.foreign = split_foreign_mask();
    if (a.S == 2) {
        if (!ws) return hipErrorInvalidValue;
        a.tickets = (uint64_t *)ws;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm8_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)g8_lds(G8_CW));
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int ntiles = a.tiles_m * a.tiles_n;
    const int gx = a.S == 2 ? (ntiles + 7) / 8 * 8 : ntiles;
    hipLaunchKernelGGL(q4_gemm8_kernel, dim3(gx, 1, a.S), dim3(64 * G8_PH * G8_CW), g8_lds(G8_CW), s, a);
    return hipGetLastError();
}

}  // namespace mcq4
