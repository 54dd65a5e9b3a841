// Prefill-shaped q4_0 matmul on gfx950: 256 x 64 wave tiles, one wave per SIMD.
//
//   * Workgroup = 4 waves along N, tile 256 (M) x 256 (N), one workgroup per
//     CU.  Each wave owns 64 columns and all 256 rows: 8 x 2 tiles of
//     v_mfma_f32_32x32x16_f16 (256 fp32 accumulators, in AGPRs), so each
//     dequantized B operand feeds 8 MFMAs -- half the dequant VALU per MFMA of a
//     128-row wave tile -- and each A operand read from LDS feeds 2.
//   * Activations: one stage = 2 K blocks (64 halves, 128 bytes per row) of the
//     256 rows, copied by global_load_lds_dwordx4 into one of 3 LDS slots
//     (32 KiB each); each wave copies 64 rows.  Chunk c (16 bytes) of row r is
//     stored at position c ^ ((r >> 1) & 7) of the row, so the operand reads
//     (ds_read_b128 of one chunk for 32 consecutive rows) hit 16 distinct bank
//     groups per 16 lanes.
//   * Weights: each wave copies the raw q4_0 bytes of its 64 columns (1152 per
//     K block: one 16-byte-per-lane and one 4-byte-per-lane copy) into a private
//     ring of 6 steps, and builds its B operands one step ahead: natural-order
//     unpack to 1024 + q, minus 1032, times d (the reference's fp16 dequant
//     value: one rounding of the exact product), in 12 chunks placed between the
//     step's 32 MFMAs.
//   * One barrier per stage, before its first step; the copies of A two stages
//     ahead and of the raw weights three stages ahead go out during that step,
//     and each step's raw words are read into registers one step before their
//     dequant, so no wait in the loop finds a recent LDS read outstanding.
//   * Split K (grid.z) for outputs with few tiles: fp32 partial tiles summed in
//     split order by q4_gemm7_reduce_kernel.  (An in-kernel sum by the second
//     workgroup of a tile to finish, through the XCD's L2, was measured slower
//     here: 230.5 against 223.1 us on the down projection at M = 2048, since it
//     serialises the epilogue of a 256 x 256 tile on one CU.)
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_prefill.h"

namespace mcq4 {

constexpr int G7_BM = 256, G7_BN = 256;
constexpr int G7_NS = 3;                        // stages (A slots) in flight
constexpr int G7_ROWB = 128;                    // A bytes per row and stage (2 steps)
constexpr int G7_A_SLOT = G7_BM * G7_ROWB;      // 32 KiB
constexpr int G7_WN = 64;                       // columns per wave
constexpr int G7_RAW_SLOT = 1280;               // 1152 raw bytes per step + the remainder copy's overhang
constexpr int G7_RAW_N = 8;                     // raw ring slots per wave (steps): 4 stages
constexpr size_t G7_LDS = (size_t)G7_NS * G7_A_SLOT + (size_t)4 * G7_RAW_N * G7_RAW_SLOT;
static_assert(G7_LDS <= 160 * 1024, "LDS budget");

struct Gemm7Args {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int tiles_m, tiles_n;
    int S;               // K splits (grid.z)
    float *partials;     // [tiles][S][256*256] when S > 1
};

__global__ void __launch_bounds__(256, 1)
q4_gemm7_kernel(Gemm7Args a) {
    constexpr int TM = G7_BM / 32, TN = G7_WN / 32;   // 8 x 2
    constexpr int A_LD = G7_BM * 8 / (64 * 4);         // A copies per wave and stage (8)
    constexpr int GROUP = A_LD + 4;                    // vector-memory instructions per wave and stage
    constexpr int NMF = 2 * TM * TN;                   // MFMAs per step (32)
    static_assert(2 * GROUP < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int bid = blockIdx.x, gx = gridDim.x;
    int tile_id = bid;
    if (gx % 8 == 0) tile_id = (bid % 8) * (gx / 8) + bid / 8;   // consecutive tiles on one XCD
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * G7_BM, n0 = tn * G7_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nb * z / a.S);
    const int nk = (int)((int64_t)a.nb * (z + 1) / a.S) - k_lo;
    const int nst = (nk + 1) >> 1;

    uint8_t *const sA = smem;
    uint8_t *const ring = smem + G7_NS * G7_A_SLOT + wave * (G7_RAW_N * G7_RAW_SLOT);

    // A copy ci of this wave: rows r = 64 wave + 8 ci + lane/8, position lane & 7,
    // source chunk (lane & 7) ^ ((r >> 1) & 7) = (lane & 7) ^ ((4 (ci & 1) + lane/16) & 7).
    // The copies are buffer loads: the stage's offset goes into the resource's
    // base address (SGPRs) and each lane's offset into the VGPR offset (one add
    // per A copy), and the resource's size bounds the reads (rows past M and
    // bytes past the end of W read as 0), so no address is clamped.
    const int a_c0 = (lane ^ (lane >> 4)) & 7, a_c1 = (lane ^ (4 + (lane >> 4))) & 7;
    // Byte counts fit 31 bits (launch_gemm7 checks X and W).
    const int x_row = (int)a.ldx * 2;
    const uint8_t *x_base = (const uint8_t *)(a.X + (int64_t)m0 * a.ldx + (int64_t)k_lo * QK);
    // Readable from x_base: up to the last row's K-th element (its row padding
    // past K need not be allocated).
    const int x_bytes = (int)((int64_t)(a.M - m0 - 1) * x_row + ((int64_t)a.nb - k_lo) * QK * 2);
    const int vo_a0 = (64 * wave + (lane >> 3)) * x_row + 16 * (a_c0 & 3) + 64 * (a_c0 >> 2);
    const int vo_a1 = (64 * wave + (lane >> 3)) * x_row + 16 * (a_c1 & 3) + 64 * (a_c1 >> 2);

    const int row_bytes = a.N * BLOCK_BYTES;
    const int w_off = k_lo * row_bytes + (n0 + wave * G7_WN) * BLOCK_BYTES;
    const uint8_t *w_base = a.W + w_off;
    const int w_bytes = a.nb * row_bytes - w_off;                                       // readable from w_base
    const int vo_w0 = 16 * lane, vo_w1 = 1024 + 4 * min(lane, 31);
    auto rsrc = [](const uint8_t *base, int off, int bytes) {
        return __builtin_amdgcn_make_buffer_rsrc((void *)(base + off), (short)0, max(0, bytes - off), 0x00020000);
    };

    // Copies of a stage: A copies ci = 0..7 of stage s_a, then the raw copies
    // ci = 8..11 of stage s_r: per step t the raw bytes 0..1023 (16 per lane)
    // and 1024..1151 (4 per lane for lanes 0..31; lanes 32..63 re-read lane 31's
    // dword into the slot's unused tail, so no lane is masked and nothing past
    // the segment is read: LDS-DMA copies of fewer than 4 bytes per lane still
    // fill 4 bytes per lane).  Stages past the end re-copy the last stage, so
    // every stage issues the same number of copies and the vmcnt waits are exact.
    // Copy ci of a t = 0 step: ci = 0..7 the A rows 8 ci .. of this wave's 64 of
    // stage s_a (into A slot as_), ci = 8..11 the raw copies of stage s_r (two
    // per K block: bytes 0..1023 at 16 per lane, 1024..1151 at 4 per lane for
    // lanes 0..31 with lanes 32..63 re-reading lane 31's dword into the slot's
    // unused tail -- no lane is masked and LDS-DMA copies of fewer than 4 bytes
    // per lane still fill 4 bytes per lane).  Stages past the end re-copy the
    // last stage, so every stage issues the same number of copies and the vmcnt
    // waits are exact.
    const __amdgpu_buffer_rsrc_t w_rs = rsrc(w_base, 0, w_bytes);
    auto issue_one = [&](int s_a, int as_, int s_r, int ci) {
        if (ci < A_LD) {
            const int s_src = min(s_a, nst - 1);
            uint8_t *dst = sA + as_ * G7_A_SLOT + G7_ROWB * (64 * wave + 8 * ci);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(x_base, 128 * s_src, x_bytes),
                                                     (__attribute__((address_space(3))) void *)dst, 16,
                                                     ((ci & 1) ? vo_a1 : vo_a0) + 8 * ci * x_row, 0, 0, 0);
            return;
        }
        const int s_src = min(s_r, nst - 1);
        const int r = ci - A_LD, t = r >> 1;
        // The K block is clamped to the split, so the weights' offset can be the
        // scalar one (outside the range check) of a single resource.
        const uint32_t so = (uint32_t)(min(2 * s_src + t, nk - 1) * row_bytes);
        uint8_t *dst = ring + ((2 * s_r + t) & (G7_RAW_N - 1)) * G7_RAW_SLOT;
        if ((r & 1) == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (__attribute__((address_space(3))) void *)dst, 16,
                                                     vo_w0, so, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (__attribute__((address_space(3))) void *)(dst + 1024),
                                                     4, vo_w1, so, 0, 0);
    };

    const int lrow = lane & 31, lhi = lane >> 5;
    // A operand (i, ks) of step t: row 32 i + lrow, chunk 4t + 2ks + lhi.
    uint32_t a_off[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            a_off[t][ks] = (uint32_t)(lrow * G7_ROWB + (((4 * t + 2 * ks + lhi) ^ ((lrow >> 1) & 7)) << 4));
    auto read_a1 = [&](int slot, int t, int ks, int i) {
        const uint32_t base = lds_addr(sA + slot * G7_A_SLOT);
        return *(const lds_half8 *)(lds_ptr(base + a_off[t][ks]) + i * 32 * G7_ROWB);
    };
    // B operand (ks, j): column 32 j + lrow, K elements 16 ks + 8 lhi .. +8 of
    // the block: qs bytes 2 + 8 ks + 4 lhi .. +4 of the column's 18-byte block.
    // A step's raw words: qd[j][0..3] (the dwords holding both ks halves) and
    // dd[j] (the scale), read one step before they are dequantized.
    const int qoff0 = 18 * lrow + 2 + 4 * lhi;
    const int q_al = qoff0 & ~3;
    const uint32_t q_sh = (uint32_t)(qoff0 & 3) * 8;
    const int d_off = 18 * lrow;
    struct Raw {
        uint32_t qd[TN][4], dd[TN];
    };
    auto read_raw_j = [&](int k, int j, Raw &rw) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k & (G7_RAW_N - 1)) * G7_RAW_SLOT));
        const lds_u32 *qp = (const lds_u32 *)(Rs + q_al + j * 32 * 18);
#pragma unroll
        for (int t = 0; t < 4; ++t) rw.qd[j][t] = qp[t];
        rw.dd[j] = *(const lds_u16 *)(Rs + d_off + j * 32 * 18);
    };
    auto read_raw = [&](int k, Raw &rw) {
#pragma unroll
        for (int j = 0; j < TN; ++j) read_raw_j(k, j, rw);
    };
    // Dequant of one B dword (K elements 2 u, 2 u + 1 of a lane's eight, from
    // byte u of its four qs bytes, which sit at byte q_b + u of the pair
    // (qd[2 ks + 1]:qd[2 ks])): v_perm_b32 puts the byte into bytes 0 and 2,
    // v_and_or_b32 keeps the low nibble in byte 0 and the high nibble in place
    // in byte 2 and adds the exponent bytes 0x64 and 0x54, giving the fp16 pair
    // {1024 + q0, 64 + q1} exactly; minus {1032, 72} (exact) gives q - 8, and
    // one multiply by d the single rounding of the exact product -- the
    // reference's fp16 dequant value.  4 VALU per two weights, no shifts.
    const int q_b = (int)(q_sh >> 3);
    uint32_t bsel[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) bsel[u] = (uint32_t)(q_b + u) * 0x00010001u + 0x0C000C00u;
    const uint32_t nib_mask = opaque_sgpr(0x00F0000Fu), exp_bits = opaque_vgpr(0x54006400u);
    auto dq2 = [&](uint32_t hi_w, uint32_t lo_w, int u, half2_t d2) {
#pragma clang fp contract(off)
        const half2_t off = {(_Float16)1032.0f, (_Float16)72.0f};
        const uint32_t x = __builtin_amdgcn_perm(hi_w, lo_w, bsel[u]);
        const half2_t h = bitcast<half2_t>(and_or(x, nib_mask, exp_bits));
        return bitcast<uint32_t>((h - off) * d2);
    };
    auto build_b = [&](const Raw &rw, half8_t (&bv)[2][TN]) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const half2_t d2 = bitcast<half2_t>(__builtin_amdgcn_perm(rw.dd[j], rw.dd[j], 0x01000100u));
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                uint4_t r;
#pragma unroll
                for (int u = 0; u < 4; ++u) r[u] = dq2(rw.qd[j][2 * ks + 1], rw.qd[j][2 * ks], u, d2);
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

    // One step: the 32 MFMAs of (A, B), ordered ks, i, j (16 MFMAs between the
    // two uses of an accumulator), with the rest of the step's work spread
    // evenly between them, since a wave issues in order and each MFMA keeps the
    // matrix pipe busy for a while: after MFMA idx, half of the dequant of one
    // dword of the next B (idx even: perm and and_or; odd: the subtract and the
    // multiply; dword idx/2, from the raw words rc read one step earlier), the
    // next step's A operand idx-1 (slot a_slot, step a_t) for idx 1..16, the raw
    // words of step k_read into rn at idx 17, 18 (after the A reads, so the wait
    // the compiler places before the next step's first MFMA finds nothing
    // recent outstanding), and with copies, copy idx/2 - 1 at the even idx 2..24.
    auto step = [&](auto with_copies, int s_a, int as_, int s_r, const half8_t (&A)[2][TM],
                    half8_t (&An)[2][TM], const half8_t (&B)[2][TN], half8_t (&Bn)[2][TN], const Raw &rc,
                    Raw &rn, int k_read, int a_slot, int a_t) {
#pragma clang fp contract(off)
        const half2_t off = {(_Float16)1032.0f, (_Float16)72.0f};
        half2_t d2[TN];
        uint32_t xw[16];
        uint4_t bb[2 * TN];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int idx = 0; idx < NMF; ++idx) {
            const int ks = idx / (TM * TN), i = (idx / TN) % TM, j = idx % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B[ks][j], acc[i][j], 0, 0, 0);
            {
                const int d = idx >> 1, unit = d >> 2, u = d & 3, uj = unit >> 1, uk = unit & 1;
                if ((idx & 1) == 0) {
                    if ((idx & 15) == 0)
                        d2[uj] = bitcast<half2_t>(__builtin_amdgcn_perm(rc.dd[uj], rc.dd[uj], 0x01000100u));
                    xw[d] = and_or(__builtin_amdgcn_perm(rc.qd[uj][2 * uk + 1], rc.qd[uj][2 * uk], bsel[u]),
                                   nib_mask, exp_bits);
                } else {
                    bb[unit][u] = bitcast<uint32_t>((bitcast<half2_t>(xw[d]) - off) * d2[uj]);
                    if (u == 3) Bn[uk][uj] = bitcast<half8_t>(bb[unit]);
                }
            }
            if (idx >= 1 && idx <= 2 * TM) {
                const int r = idx - 1;
                An[r / TM][r % TM] = read_a1(a_slot, a_t, r / TM, r % TM);
            }
            if (idx == 17) read_raw_j(k_read, 0, rn);
            if (idx == 18) read_raw_j(k_read, 1, rn);
            if constexpr (decltype(with_copies)::value) {
                if ((idx & 1) == 0 && idx >= 2 && idx / 2 - 1 < GROUP) issue_one(s_a, as_, s_r, idx / 2 - 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Pipeline (stage s = K blocks 2s, 2s+1).  During step 2s the MFMAs use A of
    // stage s and read A of stage s and the raw words of stage s+1; during step
    // 2s+1 they read A of stage s+1 and raw of stage s+1.  So the barrier before
    // step 2s makes A(s+1) and raw(s+1) visible (each wave waits for its own
    // copies, vmcnt), and also marks every wave done with step 2s-1 -- after it
    // nothing reads A(s-1) or raw(s-1), whose slots the copies issued during
    // step 2s overwrite: A(s+2) (2 steps of lookahead, from L2) and then
    // raw(s+3) (4 steps, from HBM).  vmcnt is in order, so waiting for all but
    // the 4 newest copies at the barrier covers A(s+1) and raw(s+1).
    // Prologue: A(0), raw(0), A(1), raw(1), raw(2).
#pragma unroll
    for (int ci = 0; ci < GROUP; ++ci) issue_one(0, 0, 0, ci);
#pragma unroll
    for (int ci = 0; ci < GROUP; ++ci) issue_one(1, 1, 1, ci);
#pragma unroll
    for (int ci = A_LD; ci < GROUP; ++ci) issue_one(2, 2, 2, ci);
    wait_vmcnt<GROUP - A_LD>();
    lds_barrier();
    half8_t A0[2][TM], A1[2][TM], B0[2][TN], B1[2][TN];
    Raw R0, R1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < TM; ++i) A0[ks][i] = read_a1(0, 0, ks, i);     // stage 0: slot 0
    read_raw(0, R0);
    read_raw(min(1, nk - 1), R1);
    build_b(R0, B0);
    const int nfull = nk >> 1;
    int slot0 = 0, slot1 = 1, slot2 = 2;         // A slots of stages s, s+1, s+2 (s mod 3, rotating)
    for (int s = 0; s < nfull; ++s) {
        if (s > 0) {
            wait_vmcnt<GROUP - A_LD>();          // A(s+1) and raw(s+1) (own copies) landed
            lds_barrier();                       // visible; every wave done with step 2s-1
        }
        // Step 2s: A(s, t=0); reads A(s, t=1), raw of step 2s+2; builds B(2s+1);
        // copies A(s+2) into the slot of stage s-1, and raw(s+3).
        step(std::true_type{}, s + 2, slot2, s + 3, A0, A1, B0, B1, R1, R0, min(2 * s + 2, nk - 1), slot0, 1);
        // Step 2s+1: A(s, t=1); reads A(s+1, t=0), raw of step 2s+3; builds B(2s+2).
        // Past the last step the reads are clamped re-reads of valid slots.
        step(std::false_type{}, 0, 0, 0, A1, A0, B1, B0, R0, R1, min(2 * s + 3, nk - 1), slot1, 0);
        const int t = slot0;
        slot0 = slot1; slot1 = slot2; slot2 = t;
    }
    if (nk & 1) {                                // last step alone (A and B already loaded)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0[ks][i], B0[ks][j], acc[i][j], 0, 0, 0);
    }
    wait_vmcnt<0>();

    const int rsub = 4 * lhi;
    if (a.S == 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wave * G7_WN + j * 32 + lrow;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                    if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)acc[i][j][r];
                }
            }
        return;
    }
    float *part = a.partials + ((int64_t)tile_id * a.S + z) * (G7_BM * G7_BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nl = wave * G7_WN + j * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                part[ml * G7_BN + nl] = acc[i][j][r];
            }
        }
}

// Sums the S fp32 partial tiles of every output tile in split order
// (deterministic) and stores fp16.  Each thread handles G7_RV float4 groups
// spaced a workgroup apart (all loads issued before the sums), non-temporal:
// the partials are read once.
constexpr int G7_RV = 4;
__global__ void __launch_bounds__(256)
q4_gemm7_reduce_kernel(Gemm7Args a) {
    constexpr int TILE = G7_BM * G7_BN;
    const int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n;
    const int64_t n4 = ntiles * (TILE / 4);
    const int64_t base = (int64_t)blockIdx.x * (256 * G7_RV) + threadIdx.x;
    float4_t sum[G7_RV];
#pragma unroll
    for (int u = 0; u < G7_RV; ++u) {
        const int64_t v4 = min(base + 256 * u, n4 - 1);
        const int64_t tile = v4 / (TILE / 4);
        const float4_t *p = (const float4_t *)(a.partials + tile * a.S * TILE) + v4 % (TILE / 4);
        sum[u] = __builtin_nontemporal_load(p);
    }
    for (int sp = 1; sp < a.S; ++sp) {
#pragma unroll
        for (int u = 0; u < G7_RV; ++u) {
            const int64_t v4 = min(base + 256 * u, n4 - 1);
            const int64_t tile = v4 / (TILE / 4);
            const float4_t *p = (const float4_t *)(a.partials + tile * a.S * TILE) + v4 % (TILE / 4);
            sum[u] += __builtin_nontemporal_load(p + (int64_t)sp * (TILE / 4));
        }
    }
#pragma unroll
    for (int u = 0; u < G7_RV; ++u) {
        const int64_t v4 = base + 256 * u;
        if (v4 >= n4) return;
        const int64_t tile = v4 / (TILE / 4);
        const int e = (int)(v4 % (TILE / 4)) * 4;
        const int tm = (int)(tile % a.tiles_m), tn = (int)(tile / a.tiles_m);
        const int m = tm * G7_BM + e / G7_BN, n = tn * G7_BN + e % G7_BN;
        if (m >= a.M) continue;
        if (n + 3 < a.N && (a.ldy & 3) == 0 && ((uintptr_t)a.Y & 7) == 0) {
            half4_t h;
#pragma unroll
            for (int c = 0; c < 4; ++c) h[c] = (_Float16)sum[u][c];
            *(half4_t *)(a.Y + (int64_t)m * a.ldy + n) = h;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (n + c < a.N) a.Y[(int64_t)m * a.ldy + n + c] = (_Float16)sum[u][c];
        }
    }
}

// Plan: S = the largest power of two (<= 8, at least 32 K blocks per split)
// that keeps the grid within 256 workgroups (one per CU).
static int gemm7_splits(int64_t M, int64_t K, int64_t N) {
    int S = 1;
    const int64_t t = ((M + G7_BM - 1) / G7_BM) * ((N + G7_BN - 1) / G7_BN);
    const int64_t nb = K / QK;
    while (t * S * 2 <= 256 && nb / (S * 2) >= 32 && S < 8) S *= 2;
    if (const char *env = opt("MCQ4_GEMM6_SPLIT")) S = std::max(1, std::min(16, atoi(env)));
    if (S > nb) S = 1;
    return S;
}

size_t gemm7_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const int S = gemm7_splits(M, K, N);
    if (S == 1) return 0;
    const int64_t t = ((M + G7_BM - 1) / G7_BM) * ((N + G7_BN - 1) / G7_BN);
    return COUNTER_BYTES + (size_t)t * S * G7_BM * G7_BN * sizeof(float);
}

// gemm6's shape rules, plus byte offsets that fit 31 bits (the copies address X
// and W through buffer resources with 32-bit offsets and sizes).
bool gemm7_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N) {
    return gemm6_supported(X, ldx, W, M, K, N) && M * ldx * 2 < ((int64_t)1 << 31) &&
           (K / QK) * N * BLOCK_BYTES < ((int64_t)1 << 31);
}

hipError_t launch_gemm7(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    Gemm7Args a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.tiles_n = (N + G7_BN - 1) / G7_BN;
    a.tiles_m = (M + G7_BM - 1) / G7_BM;
    a.S = gemm7_splits(M, K, N);
    a.partials = nullptr;
    if (a.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm7_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)G7_LDS);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int ntiles = a.tiles_m * a.tiles_n;
    hipLaunchKernelGGL(q4_gemm7_kernel, dim3(ntiles, 1, a.S), dim3(256), G7_LDS, s, a);
    if (a.S > 1) {
        const int64_t n4 = (int64_t)ntiles * (G7_BM * G7_BN / 4);
        hipLaunchKernelGGL(q4_gemm7_reduce_kernel, dim3((unsigned)((n4 + 256 * G7_RV - 1) / (256 * G7_RV))),
                           dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace mcq4
