// Prefill-shaped q4_0 matmul (M > 64) on gfx950: LDS-staged activations,
// per-wave dequantized weights, two waves per SIMD.
//
//   * Wave tile 128 x 64 of v_mfma_f32_32x32x16_f16 (128 fp32 accumulators), so
//     two waves share each SIMD and one wave's LDS, copy and barrier stalls are
//     covered by the other's MFMAs.  WG = 4 waves along N, WG tile 128 x 256,
//     two workgroups per CU, each barrier among 4 waves.
//   * Activations: one 128 x 128-byte stage per slot, 3 slots, swizzled chunk
//     positions 8r + (c ^ (r & 7)); each wave copies 32 rows.
//     A operands are reloaded in place: operand (ks, i) of the next step is
//     read right after the last MFMA of this step that uses it.
//   * Weights: each wave copies the raw bytes of its 64 columns (1152 bytes per
//     step: one 16-byte-per-lane and one 4-byte-per-lane copy, no lane masks)
//     into a private 6-slot ring and builds its B operands (natural-order
//     unpack to 1024 + q, minus 1032, times d: the reference's fp16 dequant
//     value) one step ahead, in 12 chunks spread over the step's 16 MFMAs.
//   * Barrier between the two steps of a stage; stage s+3's copies go out
//     during the second step, one per two MFMAs.
//   * Split K (grid.z): fp32 partial tiles in the caller's workspace, summed in
//     split order by q4_gemm6_reduce_kernel<S>; with two splits the second
//     workgroup of a tile to finish adds the first's partial itself, read from
//     their shared XCD's L2 (see xcd_ticket_inc), and stores Y.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_prefill.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(q4_gemm6_split_fallbacks)

constexpr int G6_NS = 3;                       // stages (A slots) in flight
constexpr int G6_ROWB = 128;                   // A bytes per row and stage (2 steps)
constexpr int G6_WN = 64;                      // columns per wave
constexpr int G6_RAW_W = 18 * G6_WN;           // raw weight bytes per wave and step (1152)
constexpr int G6_RAW_SLOT = 1280;              // 1024 + 256 (remainder copy); covers the read overhang
constexpr int G6_RAW_N = 2 * G6_NS;            // raw ring slots per wave (steps)
constexpr int WGM = 1;                         // rows of four waves per workgroup
constexpr size_t G6_LDS = (size_t)G6_NS * (128 * WGM) * G6_ROWB + (size_t)(4 * WGM) * G6_RAW_N * G6_RAW_SLOT;
static_assert(2 * G6_LDS <= 160 * 1024, "LDS budget: two workgroups per CU");
static_assert(G6_RAW_SLOT >= 1024 + 64 * 4 && G6_RAW_SLOT >= G6_RAW_W + 16, "raw slot covers the remainder copy and the read overhang");

__global__ void __launch_bounds__(256, 2)
q4_gemm6_kernel(Gemm6Args a) {
    constexpr int BM = 128 * WGM, NWAVES = 4 * WGM;
    constexpr int WM = BM / WGM, WN = G6_WN;   // 128 x 64 wave tiles
    constexpr int TM = WM / 32, TN = WN / 32;    // 4 x 2
    constexpr int A_SLOT = BM * G6_ROWB;
    constexpr int A_LD = BM * 8 / (64 * NWAVES);     // A copies per wave and stage (4)
    constexpr int GROUP = A_LD + 4;              // vector-memory instructions per wave and stage
    constexpr int NMF = 2 * TM * TN;             // MFMAs per step (16)
    static_assert(2 * GROUP < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;

    const int ntiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x, gx = gridDim.x;
    int tile_id = bid;
    if (gx % 8 == 0) tile_id = (bid % 8) * (gx / 8) + bid / 8;
    if (tile_id >= ntiles) return;                // grid padding (XCD-local exchange)
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * BM, n0 = tn * G6_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nb * z / a.S);
    const int nk = (int)((int64_t)a.nb * (z + 1) / a.S) - k_lo;

    uint8_t *const sA = smem;
    uint8_t *const ring = smem + G6_NS * A_SLOT + wave * (G6_RAW_N * G6_RAW_SLOT);

    // A copy u of this wave: positions 64(wave*A_LD+u) + lane = row 8(wave*A_LD+u) + lane/8,
    // chunk (lane ^ lane/8) & 7 (the same for every u): K step a_t = chunk/4 of
    // the stage, halves 8 (chunk % 4) .. +7 of it.  All copies are buffer loads
    // into LDS.  An activation copy's offset (lane part fixed, plus the stage's
    // K offset) is a VGPR, so the resource's size -- the activations' last byte
    // -- bounds it: the hardware's range check leaves out the scalar offset.
    // A weight copy's K block is clamped to the split and its offset is a
    // scalar.
    const int a_c = (lane ^ (lane >> 3)) & 7;
    const int a_t = a_c >> 2;
    const int a_r0 = m0 + 8 * wave * A_LD + (lane >> 3);
    const __amdgpu_buffer_rsrc_t a_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.X, (short)0, (int)(((int64_t)(a.M - 1) * a.ldx + (int64_t)a.nb * QK) * 2), 0x00020000);
    uint32_t a_vo[A_LD];
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
        const int m = min(a_r0 + 8 * u, a.M - 1);
        a_vo[u] = ((uint32_t)m * (uint32_t)a.ldx + 8 * (a_c & 3)) * 2 + a_t * (QK * 2);
    }

    const uint32_t row_bytes = (uint32_t)a.N * BLOCK_BYTES;
    const bool wcols = n0 + wn * WN < a.N;
    const __amdgpu_buffer_rsrc_t w_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.W, (short)0, (int)0x7fffffff, 0x00020000);
    const uint32_t w_so0 = (uint32_t)k_lo * row_bytes + (wcols ? (uint32_t)(n0 + wn * WN) * BLOCK_BYTES : 0u);
    const uint32_t w_vo16 = 16 * lane, w_vo4 = 4 * min(lane, 31);

    // Copy ci (0 .. GROUP-1) of stage s_dst: A copies, then per step t the raw
    // bytes 0..1023 (16 per lane) and 1024..1151 (4 per lane for lanes 0..31;
    // lanes 32..63 re-read lane 31's dword into the slot's unused tail, so no
    // lane is masked and nothing past the segment is read).  LDS-DMA copies of
    // fewer than 4 bytes per lane still fill 4 bytes per lane, so 2-byte copies
    // cannot pack the remainder.  Weight steps past the split's end re-copy its
    // last step; activation steps past it are read (zero past the activations'
    // last byte) but feed no MFMA.  The instruction's immediate offset would
    // move the LDS destination too, so the weights' piece offsets go into the
    // scalar offset.
    auto issue_one = [&](int s_dst, int ci) {
        if (ci < A_LD) {
            uint8_t *dst = sA + (s_dst % G6_NS) * A_SLOT + wave * (A_LD * 1024) + 1024 * ci;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, (__attribute__((address_space(3))) void *)dst, 16,
                                                     a_vo[ci] + (uint32_t)(k_lo + 2 * s_dst) * (QK * 2), 0, 0, 0);
            return;
        }
        const int r = ci - A_LD, t = r >> 1;
        const uint32_t so = w_so0 + (uint32_t)min(2 * s_dst + t, nk - 1) * row_bytes;
        uint8_t *dst = ring + ((2 * s_dst + t) % G6_RAW_N) * G6_RAW_SLOT;
        if ((r & 1) == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (__attribute__((address_space(3))) void *)dst, 16, w_vo16,
                                                     so, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (__attribute__((address_space(3))) void *)(dst + 1024), 4,
                                                     w_vo4, so + 1024, 0, 0);
    };
    auto issue_stage = [&](int s_dst) {
#pragma unroll
        for (int ci = 0; ci < GROUP; ++ci) issue_one(s_dst, ci);
    };

    const int lrow = lane & 31, lhi = lane >> 5;
    // A operand (i, ks) of step t: row wm*WM + 32 i + lrow, chunk 4t + 2ks + lhi.
    uint32_t a_off[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            a_off[t][ks] = (uint32_t)((wm * WM + lrow) * G6_ROWB + (((4 * t + 2 * ks + lhi) ^ (lrow & 7)) << 4));
    auto read_a1 = [&](int s, int t, int ks, int i) {
        const uint32_t base = lds_addr(sA + (s % G6_NS) * A_SLOT);
        return *(const lds_half8 *)(lds_ptr(base + a_off[t][ks]) + i * 32 * G6_ROWB);
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
    auto load_b = [&](int k, half8_t (&bv)[2][TN]) {
#pragma clang fp contract(off)
        const half2_t off = {(_Float16)1032.0f, (_Float16)72.0f};
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k % G6_RAW_N) * G6_RAW_SLOT));
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
                for (int u = 0; u < 4; ++u) {
                    const half2_t h = bitcast<half2_t>(
                        and_or(__builtin_amdgcn_perm(qd[2 * ks + 1], qd[2 * ks], bsel[u]), nib_mask, exp_bits));
                    r[u] = bitcast<uint32_t>((h - off) * d2);
                }
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

    // One step: the NMF MFMAs of (A, B).  The next B is NMF dwords (d = 4 unit
    // + u, unit = 2 j + ks): after MFMA idx the perm and and_or of dword idx - 1
    // and the subtract and multiply of dword idx - 2 (so neither waits on the
    // raw words just read nor on its own first half), the rest after the last
    // MFMA; also the in-place reload of the A operand whose last use this was
    // (next step's A: stage a_s, step a_t), and with copies, copy idx/2 of
    // stage cs after every odd MFMA.
    static_assert(NMF == 8 * TN, "one B dword per MFMA");
    half8_t A[2][TM];
    auto step = [&](auto with_copies, int cs, const half8_t (&B)[2][TN], int k_next,
                    half8_t (&Bn)[2][TN], int a_s, int a_t) {
#pragma clang fp contract(off)
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k_next % G6_RAW_N) * G6_RAW_SLOT));
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
            if (j == TN - 1) A[ks][i] = read_a1(a_s, a_t, ks, i);
            if constexpr (decltype(with_copies)::value) {
                if ((idx & 1) == 1 && (idx >> 1) < GROUP) issue_one(cs, idx >> 1);
            }
            if (idx >= 2) second(idx - 2);
            if (idx >= 1) first(idx - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        second(NMF - 2);
        first(NMF - 1);
        second(NMF - 1);
    };

    // Prologue: stages 0, 1, 2 in flight; stage 0 landed for every wave.
    issue_stage(0);
    issue_stage(1);
    issue_stage(2);
    wait_vmcnt<2 * GROUP>();
    lds_barrier();
    half8_t B0[2][TN], B1[2][TN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < TM; ++i) A[ks][i] = read_a1(0, 0, ks, i);
    load_b(0, B0);
    const int nfull = nk >> 1;
    for (int s = 0; s < nfull; ++s) {
        // Step 2s: builds B(2s+1) (stage s), reloads A(s, step 1).
        step(std::false_type{}, 0, B0, 2 * s + 1, B1, s, 1);
        wait_vmcnt<GROUP>();                     // stage s+1 (own copies) landed
        lds_barrier();                           // stage s+1 visible; stage s's slot read by all
        // Step 2s+1 with stage s+3's copies: builds B(2s+2) (stage s+1), reloads
        // A(s+1, step 0).  Past the last step both are clamped re-reads of valid slots.
        step(std::true_type{}, s + 3, B1, min(2 * s + 2, nk - 1), B0, s + 1, 0);
    }
    if (nk & 1) {                                // last step alone (A and B already loaded)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B0[ks][j], acc[i][j], 0, 0, 0);
    }
    wait_vmcnt<0>();

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
    float *part = a.partials + ((int64_t)tile_id * a.S + z) * (BM * G6_BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nl = wn * WN + j * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                part[ml * G6_BN + nl] = acc[i][j][r];
            }
        }
    if (!a.tickets) return;                       // the reduce kernel sums
    // Both splits of this tile run on this XCD (same blockIdx.x, grid.x a
    // multiple of 8): the partials stay in its L2.  The second to arrive adds
    // the other's partial, p0 + p1 (fp32 addition commutes, so the order of
    // arrival does not matter).
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
        if ((prev & 0xFF) == 1) {
            // Both splits have drawn: the slot is free for the next launch now, so
            // its reset overlaps the sum instead of trailing it.
            __hip_atomic_store(cnt, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (*last_flag == 2u) note_split_fallback();
    }
    __syncthreads();
    const uint32_t lf = *last_flag;
    if (!lf) return;
    float *other = a.partials + ((int64_t)tile_id * 2 + (1 - z)) * (BM * G6_BN);
    if (lf == 2) {
        // The other split ran on another XCD: its partial is not in this L2.
        // Recompute it here into its slot (plain stores, this L2), then read it
        // back as usual.  One output per thread and pass, nothing unrolled, so
        // the accumulators stay in their registers.
        const int o_lo = (int)((int64_t)a.nb * (1 - z) / 2), o_hi = (int)((int64_t)a.nb * (2 - z) / 2);
#pragma unroll 1
        for (int v = tid; v < BM * G6_BN; v += 256) {
            const int m = min(m0 + v / G6_BN, a.M - 1), n = min(n0 + v % G6_BN, a.N - 1);
            other[v] = q4_dot_range(a.X + (int64_t)m * a.ldx, a.W, a.N, n, o_lo, o_hi);
        }
        wait_vmcnt<0>();
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nl = wn * WN + j * 32 + lrow;
            float o[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                o[r] = load_l2_f32(other, (ml * G6_BN + nl) * 4);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3), n = n0 + nl;
                // p0 + p1 in split order
                const float v = z == 0 ? acc[i][j][r] + o[r] : o[r] + acc[i][j][r];
                if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)v;
            }
        }
}

// Sums the S fp32 partial tiles of every output tile in split order
// (deterministic) and stores fp16.  Thread t of block b owns float4 v = 256 b +
// t + 256 u of the [tiles][128 x 256] output for u < G6_RV; with S a template
// argument every split's loads of all its float4 go out before the first add
// (SC == 0: S read at run time, one split's loads at a time).
constexpr int G6_RV = 2;
template <int SC>
__global__ void __launch_bounds__(256)
q4_gemm6_reduce_kernel(Gemm6Args a) {
    constexpr int TILE = G6_BM * G6_BN;
    const int S = SC ? SC : a.S;
    const int64_t n4 = (int64_t)a.tiles_m * a.tiles_n * (TILE / 4);
    const int64_t base = (int64_t)blockIdx.x * (256 * G6_RV) + threadIdx.x;
    const float4_t *p[G6_RV];
#pragma unroll
    for (int u = 0; u < G6_RV; ++u) {
        const int64_t v4 = min(base + 256 * u, n4 - 1);
        const int64_t tile = v4 / (TILE / 4);
        p[u] = (const float4_t *)(a.partials + tile * S * TILE) + v4 % (TILE / 4);
    }
    float4_t sum[G6_RV];
    if constexpr (SC > 0) {
        float4_t v[G6_RV][SC];
#pragma unroll
        for (int sp = 0; sp < SC; ++sp)
#pragma unroll
            for (int u = 0; u < G6_RV; ++u) v[u][sp] = __builtin_nontemporal_load(p[u] + (int64_t)sp * (TILE / 4));
#pragma unroll
        for (int u = 0; u < G6_RV; ++u) {
            sum[u] = v[u][0];
#pragma unroll
            for (int sp = 1; sp < SC; ++sp) sum[u] += v[u][sp];
        }
    } else {
#pragma unroll
        for (int u = 0; u < G6_RV; ++u) sum[u] = __builtin_nontemporal_load(p[u]);
        for (int sp = 1; sp < S; ++sp) {
            float4_t v[G6_RV];
#pragma unroll
            for (int u = 0; u < G6_RV; ++u) v[u] = __builtin_nontemporal_load(p[u] + (int64_t)sp * (TILE / 4));
#pragma unroll
            for (int u = 0; u < G6_RV; ++u) sum[u] += v[u];
        }
    }
#pragma unroll
    for (int u = 0; u < G6_RV; ++u) {
        const int64_t v4 = base + 256 * u;
        if (v4 >= n4) break;
        const int64_t tile = v4 / (TILE / 4);
        const int e = (int)(v4 % (TILE / 4)) * 4;
        const int tm = (int)(tile % a.tiles_m), tn = (int)(tile / a.tiles_m);
        const int m = tm * G6_BM + e / G6_BN, n = tn * G6_BN + e % G6_BN;
        if (m >= a.M) continue;
        _Float16 *y = a.Y + (int64_t)m * a.ldy + n;
        if (n + 3 < a.N && ((uintptr_t)y & 7) == 0) {
            const half4_t h = {(_Float16)sum[u][0], (_Float16)sum[u][1], (_Float16)sum[u][2], (_Float16)sum[u][3]};
            *(half4_t *)y = h;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (n + c < a.N) y[c] = (_Float16)sum[u][c];
        }
    }
}

// Plan: 128-row tiles; K split S = the largest power of two (<= 16, at least
// 16 K blocks per split) that keeps the grid within 256 workgroups, one per
// CU; doubled once more when that stays within 512 (two per CU) and leaves at
// least 96 blocks per split, which pays on long K.  Measured over M =
// 128..2048 and the Llama shapes (graph replays): M=512 11008x4096 S=4 63.9 us
// (the previous "until 384 workgroups" plan, S=8: 78.5), M=512 4096x14336 S=1
// 72.7 (S=2: 81.6), M=2048 4096x4096 S=1 81.2 (S=2: 86.4), M=2048 14336x4096
// S=2 242.9 (S=1: 252.9).  MCQ4_GEMM6_SPLIT overrides (tests).
static int gemm6_splits(int64_t M, int64_t K, int64_t N) {
    int S = 1;
    const int64_t t = ((M + G6_BM - 1) / G6_BM) * ((N + G6_BN - 1) / G6_BN);
    const int64_t nb = K / QK;
    while (t * S * 2 <= 256 && nb / (S * 2) >= 16 && S < 16) S *= 2;
    if (t * S * 2 <= 512 && nb / (S * 2) >= 96 && S < 16) S *= 2;
    if (const char *env = opt("MCQ4_GEMM6_SPLIT")) S = std::max(1, std::min(16, atoi(env)));
    if (S > nb) S = 1;
    return S;
}

bool gemm6_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N) {
    // Buffer loads: activations below 2^31 bytes, W below 2^31 bytes.
    return N % 128 == 0 && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 &&
           K >= QK && M * ldx < ((int64_t)1 << 30) && (K / QK) * N * BLOCK_BYTES < ((int64_t)1 << 31);
}

size_t gemm6_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const int S = gemm6_splits(M, K, N);
    if (S == 1) return 0;
    const int64_t t = ((M + G6_BM - 1) / G6_BM) * ((N + G6_BN - 1) / G6_BN);
    return COUNTER_BYTES + (size_t)t * S * G6_BM * G6_BN * sizeof(float);
}

hipError_t launch_gemm6(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    Gemm6Args a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.tiles_n = (N + G6_BN - 1) / G6_BN;
    a.tiles_m = (M + G6_BM - 1) / G6_BM;
    a.S = gemm6_splits(M, K, N);
    a.partials = nullptr;
    a.foreign = split_foreign_mask();
    if (a.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
        // Two splits: summed in the kernel through the XCD's L2 (MCQ4_XCD_LOCAL=0:
        // by the reduction kernel).
        if (a.S == 2 && !opt_is("MCQ4_XCD_LOCAL", '0') && (a.tiles_m * a.tiles_n + 7) / 8 <= 4096)
            a.tickets = (uint64_t *)ws;
    }
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm6_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)G6_LDS);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int ntiles = a.tiles_m * a.tiles_n;
    const int gx = a.tickets ? (ntiles + 7) / 8 * 8 : ntiles;
    hipLaunchKernelGGL(q4_gemm6_kernel, dim3(gx, 1, a.S), dim3(256), G6_LDS, s, a);
    if (a.S > 1 && !a.tickets) {
        const int64_t n4 = (int64_t)ntiles * (G6_BM * G6_BN / 4);
        const dim3 grid((unsigned)((n4 + 256 * G6_RV - 1) / (256 * G6_RV)));
        switch (a.S) {
            case 2: hipLaunchKernelGGL(q4_gemm6_reduce_kernel<2>, grid, dim3(256), 0, s, a); break;
            case 4: hipLaunchKernelGGL(q4_gemm6_reduce_kernel<4>, grid, dim3(256), 0, s, a); break;
            case 8: hipLaunchKernelGGL(q4_gemm6_reduce_kernel<8>, grid, dim3(256), 0, s, a); break;
            default: hipLaunchKernelGGL(q4_gemm6_reduce_kernel<0>, grid, dim3(256), 0, s, a); break;
        }
    }
    return hipGetLastError();
}

}  // namespace mcq4
