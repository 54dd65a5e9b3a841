// Prefill-shaped (M > 16) per-group INT4 matmul on gfx950 with the activation
// tile staged in LDS and two waves per SIMD: the structure of q4_gemm6 with the
// packed[K/2][N] nibble format and 16-bit per-group scales/zeros.
//
//   * WG = 4 waves along N, WG tile 128 x 256, two workgroups per CU; wave tile
//     128 x 64 of v_mfma_f32_32x32x16_f16 (128 fp32 accumulators).  K advances
//     32 per step (16 byte rows), two steps per stage.
//   * Activations: one stage of the workgroup's 128 rows (128 bytes each) per
//     LDS slot, 3 slots, chunk c of row r at position 8r + (c ^ (r & 7)) so the
//     ds_read_b128 operand reads are free of bank conflicts; each wave copies
//     32 rows.  Operands are reloaded in place after their last use.
//   * Weights: per step each wave copies its 16 x 64 raw bytes (one
//     16-byte-per-lane copy, row-major [16][64]) and the step's group scale and
//     zero rows for its 64 columns (one 4-byte-per-lane copy: 64 scales, then
//     64 zeros) into a private ring of 6 step slots.  No copy is lane-masked.
//   * B operand: MFMA tile j column l%32 is the wave's column 2(l%32)+j, so one
//     ds_read_u16 of a byte row serves both tiles.  Per byte row r:
//     v_perm_b32 + v_and_or_b32 give the fp16 pair {1024 + q(2r), 1024 + q(2r+1)};
//     minus 1024 (exact) gives q; one fp16 FMA q*s + c with c = -z*s (fp32
//     product rounded to fp16) gives the weight (q - z)*s to fp16 precision
//     (the formula of i4_gemm).  The next step's operands are built in chunks
//     between this step's MFMAs.
//   * Barrier between the two steps of a stage; stage s+3's copies go out
//     during the second step, one per two MFMAs.  With two K splits the second
//     workgroup of a tile to finish sums both partials (XCD-local exchange, see
//     xcd_ticket_inc).  Otherwise split-K partials and their
//     reduction (with the fused activation) are i4_gemm's.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <stdlib.h>
#include <type_traits>

#include "i4_gemm.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(i4_gemm6_split_fallbacks)

constexpr int J6_NS = 3;                        // stages (A slots) in flight
constexpr int J6_ROWB = 128;                    // A bytes per row and stage (2 steps)
constexpr int J6_BM = 128;
constexpr int J6_WN = 64;                       // columns per wave
constexpr int J6_RAW = 16 * J6_WN;              // raw bytes per wave and step (1024)
constexpr int J6_SLOT = J6_RAW + 256;           // + 64 scales and 64 zeros (16-bit)
constexpr int J6_RAW_N = 2 * J6_NS;             // ring slots per wave (steps)
constexpr size_t J6_LDS = (size_t)J6_NS * J6_BM * J6_ROWB + (size_t)4 * J6_RAW_N * J6_SLOT;
static_assert(2 * J6_LDS <= 160 * 1024, "two workgroups per CU");

// One 16-byte-per-lane buffer copy into LDS from `base` (`bytes` readable) at
// the VGPR offset voff plus the scalar offset soff.  (A plain function: the host
// pass of a kernel template would instantiate the buffer builtins and drop the
// kernel.)
__device__ __forceinline__ void j6_copy16(const void *base, int bytes, uint32_t voff, uint32_t soff, uint8_t *dst) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, bytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, soff, 0, 0);
}

template <int SZ, int ACT>
__global__ void __launch_bounds__(256, 2)
i4_gemm6_kernel(I4GemmArgs a) {
    static_assert(SZ == DT_F16 || SZ == DT_BF16, "16-bit scales and zeros");
    constexpr int BM = J6_BM, WM = 128, WN = J6_WN;
    constexpr int TM = WM / 32, TN = WN / 32;     // 4 x 2
    constexpr int A_SLOT = BM * J6_ROWB;
    constexpr int A_LD = BM * 8 / (64 * 4);      // A copies per wave and stage (4)
    constexpr int GROUP = A_LD + 4;              // + per step: raw, scales/zeros
    constexpr int NMF = 2 * TM * TN;             // MFMAs per step (16)
    static_assert(2 * GROUP < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave;

    const int ntiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x, gx = gridDim.x;
    int tile_id = bid;
    if (gx % 8 == 0) tile_id = (bid % 8) * (gx / 8) + bid / 8;
    if (tile_id >= ntiles) return;                // grid padding (XCD-local exchange)
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * BM, n0 = tn * I4G_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nsteps * z / a.S);
    const int nk = (int)((int64_t)a.nsteps * (z + 1) / a.S) - k_lo;
    const int nst = (nk + 1) >> 1;
    const int N = a.N;

    uint8_t *const sA = smem;
    uint8_t *const ring = smem + J6_NS * A_SLOT + wave * (J6_RAW_N * J6_SLOT);

    // A copy u of this wave: row 8(wave*A_LD+u) + lane/8, chunk (lane ^ lane/8) & 7
    // (K step a_t of the stage, halves 8 (chunk % 4) .. +7 of it).  Buffer loads
    // (byte offsets fit 31 bits, i4_gemm6_supported): an activation copy's stage
    // offset goes into its VGPR offset, which the resource's size (the last
    // row's K-th element) bounds -- the scalar offset is outside the hardware's
    // range check; steps past the split are read but feed no MFMA.
    const int a_c = (lane ^ (lane >> 3)) & 7;
    const int a_t = a_c >> 2;
    const int a_r0 = m0 + 8 * wave * A_LD + (lane >> 3);
    const int x_bytes = (int)(((int64_t)(a.M - 1) * a.ldx + (int64_t)a.nsteps * 32) * 2);
    uint32_t a_vo[A_LD];
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
        const int m = min(a_r0 + 8 * u, a.M - 1);
        a_vo[u] = ((uint32_t)m * (uint32_t)a.ldx + 8 * (a_c & 3)) * 2 + a_t * 64;
    }

    // Weights: the lane's fixed offset, the K step (clamped to the split) as the
    // scalar offset; scale groups as a 32-bit scalar added to the lane's pointer.
    const int wcol0 = n0 + wn * WN;
    const int wcol = wcol0 < N ? wcol0 : 0;       // whole wave past N: copy column 0 instead
    const uint32_t w_vo = (uint32_t)(lane >> 2) * (uint32_t)N + (uint32_t)wcol + 16 * (lane & 3);
    const uint32_t w_so0 = (uint32_t)k_lo * 16 * (uint32_t)N;
    const uint8_t *sz_base = (const uint8_t *)(lane < 32 ? a.scales : a.zeros) + (int64_t)wcol * 2 + 4 * (lane & 31);

    // Copy ci (0 .. GROUP-1) of stage s_dst: the A copies, then per step t the raw
    // bytes and the scale/zero rows.  Stages past the end re-copy the last one.
    auto issue_one = [&](int s_dst, int ci) {
        const int s_src = min(s_dst, nst - 1);
        if (ci < A_LD) {
            uint8_t *dst = sA + (s_dst % J6_NS) * A_SLOT + wave * (A_LD * 1024) + 1024 * ci;
            j6_copy16(a.X, x_bytes, a_vo[ci] + (uint32_t)(k_lo + 2 * s_src) * 64, 0, dst);
            return;
        }
        const int r = ci - A_LD, t = r >> 1;
        const int step = min(2 * s_src + t, nk - 1);
        uint8_t *dst = ring + ((2 * s_dst + t) % J6_RAW_N) * J6_SLOT;
        if ((r & 1) == 0) {
            j6_copy16(a.P, 0x7fffffff, w_vo, w_so0 + (uint32_t)step * 16 * (uint32_t)N, dst);
        } else {
            const uint32_t grp = (uint32_t)i4_group_of(k_lo + step, a.spg_magic, a.spg_ident);
            __builtin_amdgcn_global_load_lds((void *)(sz_base + grp * (uint32_t)(2 * N)),
                                             (__attribute__((address_space(3))) void *)(dst + J6_RAW), 4, 0, 0);
        }
    };
    auto issue_stage = [&](int s_dst) {
#pragma unroll
        for (int ci = 0; ci < GROUP; ++ci) issue_one(s_dst, ci);
    };

    const int lrow = lane & 31, lhi = lane >> 5;
    uint32_t a_off[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            a_off[t][ks] = (uint32_t)(lrow * J6_ROWB + (((4 * t + 2 * ks + lhi) ^ (lrow & 7)) << 4));
    auto read_a1 = [&](int s, int t, int ks, int i) {
        const uint32_t base = lds_addr(sA + (s % J6_NS) * A_SLOT);
        return *(const lds_half8 *)(lds_ptr(base + a_off[t][ks]) + i * 32 * J6_ROWB);
    };

    const uint32_t c64 = opaque_vgpr(0x64006400u);
    const uint32_t mlo = opaque_sgpr(0x000F000Fu);
    const half2_t m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};

    // fp16 scale and offset pairs of the lane's two columns (2 lrow + j).
    auto scale_pairs = [&](const lds_u8 *Rs, half2_t (&s2)[TN], half2_t (&c2)[TN]) {
        const uint32_t sv = *(const lds_u32 *)(Rs + J6_RAW + 4 * lrow);
        const uint32_t zv = *(const lds_u32 *)(Rs + J6_RAW + 128 + 4 * lrow);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            float s, zz;
            if constexpr (SZ == DT_F16) {
                s = (float)bitcast<half2_t>(sv)[j];
                zz = (float)bitcast<half2_t>(zv)[j];
            } else {
                s = __uint_as_float(j ? (sv & 0xFFFF0000u) : (sv << 16));
                zz = __uint_as_float(j ? (zv & 0xFFFF0000u) : (zv << 16));
            }
            const _Float16 sh = (_Float16)s, ch = (_Float16)(-zz * s);
            s2[j] = half2_t{sh, sh};
            c2[j] = half2_t{ch, ch};
        }
    };
    // Pair of byte row r for tile j: {1024 + q(2r), 1024 + q(2r+1)} of column 2 lrow + j.
    auto b_pair = [&](uint32_t w, int j, half2_t s2, half2_t c2) {
        const uint32_t sel = (uint32_t)j | (uint32_t)j << 8 | (uint32_t)(4 + j) << 16 | (uint32_t)(4 + j) << 24;
        const half2_t q = bitcast<half2_t>(and_or(__builtin_amdgcn_perm(w >> 4, w, sel), mlo, c64)) + m1024;
        return bitcast<uint32_t>(__builtin_elementwise_fma(q, s2, c2));
    };
    auto load_b = [&](int k, half8_t (&bv)[2][TN]) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k % J6_RAW_N) * J6_SLOT));
        half2_t s2[TN], c2[TN];
        scale_pairs(Rs, s2, c2);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            uint32_t w[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) w[r] = *(const lds_u16 *)(Rs + (8 * ks + 4 * lhi + r) * J6_WN + 2 * lrow);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                uint4_t d;
#pragma unroll
                for (int r = 0; r < 4; ++r) d[r] = b_pair(w[r], j, s2[j], c2[j]);
                bv[ks][j] = bitcast<half8_t>(d);
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

    // One step: the NMF MFMAs of (A, B).  After MFMA idx: chunk idx of the next
    // B (chunk 0: raw reads and scale pairs; chunks 1..8: two byte rows of one
    // (ks, j) operand), the in-place reload of the A operand whose last use this
    // was, and with copies, copy idx/2 of stage cs after every odd MFMA.
    half8_t A[2][TM];
    auto step = [&](auto with_copies, int cs, const half8_t (&B)[2][TN], int k_next,
                    half8_t (&Bn)[2][TN], int a_s, int a_t) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k_next % J6_RAW_N) * J6_SLOT));
        uint32_t w[2][4];
        half2_t s2[TN], c2[TN];
        uint32_t d[2][TN][4];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int idx = 0; idx < NMF; ++idx) {
            const int ks = idx / (TM * TN), i = (idx / TN) % TM, j = idx % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B[ks][j], acc[i][j], 0, 0, 0);
            if (j == TN - 1) A[ks][i] = read_a1(a_s, a_t, ks, i);
            if constexpr (decltype(with_copies)::value) {
                if ((idx & 1) == 1 && (idx >> 1) < GROUP) issue_one(cs, idx >> 1);
            }
            if (idx == 0) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        w[kk][r] = *(const lds_u16 *)(Rs + (8 * kk + 4 * lhi + r) * J6_WN + 2 * lrow);
                scale_pairs(Rs, s2, c2);
            } else if (idx <= 8) {
                const int c = idx - 1, uk = c >> 2, uj = (c >> 1) & 1, rh = c & 1;
#pragma unroll
                for (int r = 2 * rh; r < 2 * rh + 2; ++r) d[uk][uj][r] = b_pair(w[uk][r], uj, s2[uj], c2[uj]);
                if (rh == 1) Bn[uk][uj] = bitcast<half8_t>(uint4_t{d[uk][uj][0], d[uk][uj][1], d[uk][uj][2], d[uk][uj][3]});
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
    half8_t B0[2][TN], B1[2][TN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < TM; ++i) A[ks][i] = read_a1(0, 0, ks, i);
    load_b(0, B0);
    const int nfull = nk >> 1;
    for (int s = 0; s < nfull; ++s) {
        step(std::false_type{}, 0, B0, 2 * s + 1, B1, s, 1);
        wait_vmcnt<GROUP>();                     // stage s+1 (own copies) landed
        lds_barrier();                           // stage s+1 visible; stage s's slot read by all
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

    // ---- epilogue: lane holds columns 2 lrow + j of the wave's 64 ----
    const int rsub = 4 * lhi;
    if (a.S == 1) {
        _Float16 *Y = (_Float16 *)a.Y;
        const int n = wcol0 + 2 * lrow;
        if (n >= N) return;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                if (m < a.M) {
                    half2_t v;
#pragma unroll
                    for (int j = 0; j < TN; ++j) v[j] = (_Float16)activate<ACT>(acc[i][j][r]);
                    *(half2_t *)(Y + (int64_t)m * a.ldy + n) = v;
                }
            }
        return;
    }
    float *part = a.partials + ((int64_t)tile_id * a.S + z) * (BM * I4G_BN);
    const int nl = wn * WN + 2 * lrow;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ml = i * 32 + 8 * (r >> 2) + rsub + (r & 3);
            float2 v;
            v.x = acc[i][0][r];
            v.y = acc[i][1][r];
            *(float2 *)(part + ml * I4G_BN + nl) = v;
        }
    if (!a.tickets) return;                       // the reduction kernel sums
    // Both splits of this tile run on this XCD (same blockIdx.x, grid.x a
    // multiple of 8): the second to arrive adds the other's partial from the
    // XCD's L2, p0 + p1 (fp32 addition commutes).
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
    float *other = a.partials + ((int64_t)tile_id * 2 + (1 - z)) * (BM * I4G_BN);
    if (lf == 2) {
        // The other split ran on another XCD: its partial is not in this L2.
        // Recompute it here into its slot (plain stores, this L2), then read it
        // back as usual.  One output per thread and pass, nothing unrolled, so
        // the accumulators stay in their registers.
        const int o_lo = (int)((int64_t)a.nsteps * (1 - z) / 2) * 32;
        const int o_hi = (int)((int64_t)a.nsteps * (2 - z) / 2) * 32;
#pragma unroll 1
        for (int v = tid; v < BM * I4G_BN; v += 256) {
            const int m = min(m0 + v / I4G_BN, a.M - 1), nn = min(n0 + v % I4G_BN, N - 1);
            other[v] = i4_dot_range<4>(a.X + (int64_t)m * a.ldx, a.P, a.scales, a.zeros, SZ, N, a.spg * 32, nn,
                                       o_lo, o_hi);
        }
        wait_vmcnt<0>();
        __syncthreads();
    }
    _Float16 *Y = (_Float16 *)a.Y;
    const int n = wcol0 + 2 * lrow;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        float o[16][2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ml = i * 32 + 8 * (r >> 2) + rsub + (r & 3);
            o[r][0] = load_l2_f32(other, (ml * I4G_BN + nl) * 4);
            o[r][1] = load_l2_f32(other, (ml * I4G_BN + nl + 1) * 4);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
            if (m < a.M && n < N) {
                half2_t v;
#pragma unroll
                for (int j = 0; j < TN; ++j)     // p0 + p1 in split order
                    v[j] = (_Float16)activate<ACT>(z == 0 ? acc[i][j][r] + o[r][j] : o[r][j] + acc[i][j][r]);
                *(half2_t *)(Y + (int64_t)m * a.ldy + n) = v;
            }
        }
    }
}

// Plan: 128-row tiles; K split S = the largest power of two (<= 16, at least 16
// steps per split) that keeps the grid within 256 workgroups, one per CU,
// doubled once more when that stays within 512 and leaves at least 64 steps per
// split (q4_gemm6 asks 96; INT4 gains from the extra split down to 64: M=1024
// 11008x4096 S=4 111 us vs S=2 122, M=512 4096x14336 S=2 80 vs S=1 84).  Against
// the previous "until 384 workgroups" plan: M=512 4096x4096 35 us (41), M=128
// 4096x14336 35 (39).  MCQ4_I4_GEMM6_SPLIT overrides.
struct J6Cfg {
    int S;
};
static J6Cfg i4_gemm6_config(int64_t M, int64_t K, int64_t N) {
    const int64_t t = ((M + J6_BM - 1) / J6_BM) * ((N + I4G_BN - 1) / I4G_BN);
    const int64_t ns = K / 32;
    int S = 1;
    while (t * S * 2 <= 256 && ns / (S * 2) >= 16 && S < 16) S *= 2;
    if (t * S * 2 <= 512 && ns / (S * 2) >= 64 && S < 16) S *= 2;
    if (S > ns) S = 1;
    return {S};
}

// 4-bit weights with 16-bit scales/zeros, plus i4_gemm's shape rules (N % 128,
// K % 32, group % 32, 16-byte aligned operands) and 4-byte aligned Y rows.
// MCQ4_I4_GEMM6=0 disables it.
bool i4_gemm6_supported(int wb, int sz_dt, int64_t M, int64_t K, int64_t N, int64_t gs, int64_t ldx, const void *Y,
                        int64_t ldy) {
    if (opt_is("MCQ4_I4_GEMM6", '0')) return false;
    // Buffer-load copies: activations and packed weights below 2^31 bytes.
    return wb == 4 && (sz_dt == DT_F16 || sz_dt == DT_BF16) && N % 128 == 0 && K % 32 == 0 && gs % 32 == 0 &&
           ((uintptr_t)Y % 4) == 0 && ldy % 2 == 0 && M * ldx < ((int64_t)1 << 30) &&
           (K / 2) * N < ((int64_t)1 << 31) && ((K + gs - 1) / gs) * N * 2 < ((int64_t)1 << 31);
}

size_t i4_gemm6_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const J6Cfg c = i4_gemm6_config(M, K, N);
    if (c.S == 1) return 0;
    const int64_t t = ((M + J6_BM - 1) / J6_BM) * ((N + I4G_BN - 1) / I4G_BN);
    return COUNTER_BYTES + (size_t)t * c.S * J6_BM * I4G_BN * sizeof(float);
}

template <int SZ, int ACT>
static hipError_t launch_j6(const I4GemmArgs &a, hipStream_t s) {
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)i4_gemm6_kernel<SZ, ACT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)J6_LDS);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int ntiles = a.tiles_m * a.tiles_n;
    const int gx = a.tickets ? (ntiles + 7) / 8 * 8 : ntiles;
    hipLaunchKernelGGL((i4_gemm6_kernel<SZ, ACT>), dim3(gx, 1, a.S), dim3(256), J6_LDS, s, a);
    if (a.S > 1 && !a.tickets) return launch_i4_gemm_reduce(a, J6_BM, ACT, s);
    return hipGetLastError();
}

template <int SZ>
static hipError_t launch_j6_act(const I4GemmArgs &a, int act, hipStream_t s) {
    if (act == ACT_SILU) return launch_j6<SZ, ACT_SILU>(a, s);
    if (act == ACT_GELU) return launch_j6<SZ, ACT_GELU>(a, s);
    return launch_j6<SZ, ACT_NONE>(a, s);
}

hipError_t launch_i4_gemm6(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                           const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K, int N,
                           int gs, int act, void *ws, hipStream_t s) {
    const J6Cfg c = i4_gemm6_config(M, K, N);
    I4GemmArgs a;
    a.foreign = split_foreign_mask();
    a.X = X; a.ldx = ldx; a.P = P; a.scales = scales; a.zeros = zeros; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nsteps = K / 32; a.N = N; a.spg = gs / 32; a.spg_magic = i4_spg_magic(a.spg); a.spg_ident = i4_spg_ident(a.spg);
    a.tiles_n = (N + I4G_BN - 1) / I4G_BN;
    a.tiles_m = (M + J6_BM - 1) / J6_BM;
    a.S = c.S;
    a.partials = nullptr;
    if (c.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
        // Two splits: summed in the kernel through the XCD's L2 (MCQ4_XCD_LOCAL=0:
        // by the reduction kernel).
        if (c.S == 2 && !opt_is("MCQ4_XCD_LOCAL", '0') && (a.tiles_m * a.tiles_n + 7) / 8 <= 4096)
            a.tickets = (uint64_t *)ws;
    }
    if (sz_dt == DT_F16) return launch_j6_act<DT_F16>(a, act, s);
    return launch_j6_act<DT_BF16>(a, act, s);
}

}  // namespace mcq4
