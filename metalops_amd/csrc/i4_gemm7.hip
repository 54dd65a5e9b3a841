// Prefill-shaped per-group INT4 matmul on gfx950: 256 x 64 wave tiles, one
// wave per SIMD -- q4_gemm7's structure with the packed[K/2][N] nibble format
// and 16-bit per-group scales/zeros (W = (q - z) * s).
//
//   * Workgroup = 4 waves along N, tile 256 (M) x 256 (N), one workgroup per
//     CU.  Each wave owns 64 columns and all 256 rows: 8 x 2 tiles of
//     v_mfma_f32_32x32x16_f16 (256 fp32 accumulators), so each B operand feeds
//     8 MFMAs, half the dequant per MFMA of i4_gemm6's 128-row wave tiles.
//   * Activations: q4_gemm7's stages (2 steps of 32 K, 128 bytes per row, 3
//     LDS slots of 32 KiB, buffer-resource copies, chunk c of row r at position
//     c ^ ((r >> 1) & 7)).
//   * Weights: per step each wave copies its 16 byte rows x 64 columns (one
//     16-byte-per-lane copy, row-major [16][64]) and the step's group scale and
//     zero rows for its 64 columns (one 4-byte-per-lane copy: 64 scales, then
//     64 zeros) into a private ring of 8 step slots, and reads each step's words
//     into registers one step before it dequantizes them.
//   * B operand: MFMA tile j column l%32 is the wave's column 2(l%32)+j, so one
//     ds_read_u16 of a byte row serves both tiles.  Per byte row and tile:
//     v_perm_b32 puts byte j into bytes 0 and 2, v_and_or_b32 keeps the low
//     nibble in byte 0 and the high nibble in place in byte 2 with the exponent
//     bytes 0x64 and 0x54 -- the fp16 pair {1024 + q(2r), 64 + q(2r+1)} exactly;
//     minus {1024, 64} (exact) gives q, and one fp16 FMA q*s + c with
//     c = -z*s (fp32 product rounded to fp16) gives (q - z)*s as i4_gemm6 does.
//     4 VALU per two weights, spread over the step's 32 MFMAs.
//   * Split K (grid.z) for outputs with few tiles: fp32 partial tiles summed in
//     split order, with the fused activation, by i4_gemm_reduce_kernel.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "i4_gemm.h"

namespace mcq4 {

constexpr int J7_BM = 256;
constexpr int J7_NS = 3;                        // stages (A slots) in flight
constexpr int J7_ROWB = 128;                    // A bytes per row and stage (2 steps)
constexpr int J7_A_SLOT = J7_BM * J7_ROWB;      // 32 KiB
constexpr int J7_WN = 64;                       // columns per wave
constexpr int J7_RAW = 16 * J7_WN;              // raw bytes per wave and step (1024)
constexpr int J7_SLOT = J7_RAW + 256;           // + 64 scales and 64 zeros (16-bit)
constexpr int J7_RAW_N = 8;                     // ring slots per wave (steps): 4 stages
constexpr size_t J7_LDS = (size_t)J7_NS * J7_A_SLOT + (size_t)4 * J7_RAW_N * J7_SLOT;
static_assert(J7_LDS <= 160 * 1024, "LDS budget");

// One 16-byte-per-lane buffer copy into LDS: bytes [off, bytes) of `base`
// readable, lane offset voff.  (A plain function: the host pass of a kernel
// template would instantiate the buffer builtins and drop the kernel.)
__device__ __forceinline__ void j7_copy16(const uint8_t *base, int off, int bytes, uint8_t *dst, int voff) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(base + off), (short)0, max(0, bytes - off), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, 0, 0, 0);
}

// One 16-byte-per-lane weight copy into LDS: P's bytes at the scalar offset
// `so` (the K step, clamped to the split) plus the lane's fixed offset.
__device__ __forceinline__ void j7_copy_w(const uint8_t *P, uint32_t so, uint8_t *dst, uint32_t voff) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)P, (short)0, 0x7fffffff, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, so, 0, 0);
}

template <int SZ, int ACT>
__global__ void __launch_bounds__(256, 1)
i4_gemm7_kernel(I4GemmArgs a) {
    static_assert(SZ == DT_F16 || SZ == DT_BF16, "16-bit scales and zeros");
    constexpr int TM = J7_BM / 32, TN = J7_WN / 32;   // 8 x 2
    constexpr int A_LD = J7_BM * 8 / (64 * 4);         // A copies per wave and stage (8)
    constexpr int GROUP = A_LD + 4;                    // + per step: raw, scales/zeros
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
    const int m0 = tm * J7_BM, n0 = tn * I4G_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nsteps * z / a.S);
    const int nk = (int)((int64_t)a.nsteps * (z + 1) / a.S) - k_lo;
    const int nst = (nk + 1) >> 1;
    const int N = a.N;

    uint8_t *const sA = smem;
    uint8_t *const ring = smem + J7_NS * J7_A_SLOT + wave * (J7_RAW_N * J7_SLOT);

    // A copies: as q4_gemm7 (buffer resource per stage; rows past M read 0).
    const int a_c0 = (lane ^ (lane >> 4)) & 7, a_c1 = (lane ^ (4 + (lane >> 4))) & 7;
    const int x_row = (int)a.ldx * 2;
    const uint8_t *x_base = (const uint8_t *)(a.X + (int64_t)m0 * a.ldx + (int64_t)k_lo * 32);
    // Readable from x_base: up to the last row's K-th element (its row padding
    // past K need not be allocated).
    const int x_bytes = (int)((int64_t)(a.M - m0 - 1) * x_row + ((int64_t)a.nsteps - k_lo) * 32 * 2);
    const int vo_a0 = (64 * wave + (lane >> 3)) * x_row + 16 * (a_c0 & 3) + 64 * (a_c0 >> 2);
    const int vo_a1 = (64 * wave + (lane >> 3)) * x_row + 16 * (a_c1 & 3) + 64 * (a_c1 >> 2);

    // Weight copies: byte row lane/4, 16-byte piece lane%4 of the wave's 64
    // columns; scales (lanes 0..31) and zeros (lanes 32..63), 4 bytes a lane.  A
    // wave wholly past N (N % 256 == 128) copies column 0 instead.
    const int wcol0 = n0 + wave * J7_WN;
    const int wcol = wcol0 < N ? wcol0 : 0;
    // Byte offsets fit 31 bits (i4_gemm7_supported): the weights' K step is a
    // scalar offset, a scale group a 32-bit scalar added to the lane's pointer.
    const uint32_t w_vo = (uint32_t)(lane >> 2) * (uint32_t)N + 16 * (lane & 3);
    const uint32_t w_so0 = (uint32_t)k_lo * 16 * (uint32_t)N + (uint32_t)wcol;
    const uint8_t *sz_base = (const uint8_t *)(lane < 32 ? a.scales : a.zeros) + (int64_t)wcol * 2 + 4 * (lane & 31);

    // Copy ci of a t = 0 step: ci = 0..7 the A rows 8 ci .. of this wave's 64 of
    // stage s_a (into A slot as_), ci = 8..11 the raw and scale/zero copies of
    // the two steps of stage s_r.  Stages past the end re-copy the last stage,
    // so every stage issues the same number of copies and the vmcnt waits are
    // exact.  No copy is lane-masked.
    auto issue_one = [&](int s_a, int as_, int s_r, int ci) {
        if (ci < A_LD) {
            const int s_src = min(s_a, nst - 1);
            uint8_t *dst = sA + as_ * J7_A_SLOT + J7_ROWB * (64 * wave + 8 * ci);
            j7_copy16(x_base, 128 * s_src, x_bytes, dst, ((ci & 1) ? vo_a1 : vo_a0) + 8 * ci * x_row);
            return;
        }
        const int s_src = min(s_r, nst - 1);
        const int r = ci - A_LD, t = r >> 1;
        const int step = min(2 * s_src + t, nk - 1);
        uint8_t *dst = ring + ((2 * s_r + t) & (J7_RAW_N - 1)) * J7_SLOT;
        if ((r & 1) == 0) {
            j7_copy_w(a.P, w_so0 + (uint32_t)step * 16 * (uint32_t)N, dst, w_vo);
        } else {
            const uint32_t grp = (uint32_t)i4_group_of(k_lo + step, a.spg_magic, a.spg_ident);
            __builtin_amdgcn_global_load_lds((void *)(sz_base + grp * (uint32_t)(2 * N)),
                                             (__attribute__((address_space(3))) void *)(dst + J7_RAW), 4, 0, 0);
        }
    };

    const int lrow = lane & 31, lhi = lane >> 5;
    // A operand (i, ks) of step t: row 32 i + lrow, chunk 4t + 2ks + lhi.
    uint32_t a_off[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            a_off[t][ks] = (uint32_t)(lrow * J7_ROWB + (((4 * t + 2 * ks + lhi) ^ ((lrow >> 1) & 7)) << 4));
    auto read_a1 = [&](int slot, int t, int ks, int i) {
        const uint32_t base = lds_addr(sA + slot * J7_A_SLOT);
        return *(const lds_half8 *)(lds_ptr(base + a_off[t][ks]) + i * 32 * J7_ROWB);
    };
    // A step's words: w[ks][r] = bytes (2 lrow, 2 lrow + 1) of byte row
    // 8 ks + 4 lhi + r, and the scale and zero pairs of those two columns.
    struct Raw {
        uint32_t w[2][4], sv, zv;
    };
    auto read_raw_k = [&](int k, int ks, Raw &rw) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k & (J7_RAW_N - 1)) * J7_SLOT));
#pragma unroll
        for (int r = 0; r < 4; ++r) rw.w[ks][r] = *(const lds_u16 *)(Rs + (8 * ks + 4 * lhi + r) * J7_WN + 2 * lrow);
        if (ks == 0) {
            rw.sv = *(const lds_u32 *)(Rs + J7_RAW + 4 * lrow);
            rw.zv = *(const lds_u32 *)(Rs + J7_RAW + 128 + 4 * lrow);
        }
    };
    // fp16 scale and offset pair of tile j's column (2 lrow + j): s and
    // c = fp16(-z * s) (fp32 product).
    auto scale_pair = [&](const Raw &rw, int j, half2_t &s2, half2_t &c2) {
        float s, zz;
        if constexpr (SZ == DT_F16) {
            s = (float)bitcast<half2_t>(rw.sv)[j];
            zz = (float)bitcast<half2_t>(rw.zv)[j];
        } else {
            s = __uint_as_float(j ? (rw.sv & 0xFFFF0000u) : (rw.sv << 16));
            zz = __uint_as_float(j ? (rw.zv & 0xFFFF0000u) : (rw.zv << 16));
        }
        const _Float16 sh = (_Float16)s, ch = (_Float16)(-zz * s);
        s2 = half2_t{sh, sh};
        c2 = half2_t{ch, ch};
    };
    uint32_t bsel[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) bsel[j] = (uint32_t)j * 0x00010001u + 0x0C000C00u;
    const uint32_t nib_mask = opaque_sgpr(0x00F0000Fu), exp_bits = opaque_vgpr(0x54006400u);
    auto build_b = [&](const Raw &rw, half8_t (&bv)[2][TN]) {
#pragma clang fp contract(off)
        const half2_t off = {(_Float16)1024.0f, (_Float16)64.0f};
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            half2_t s2, c2;
            scale_pair(rw, j, s2, c2);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                uint4_t d;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const half2_t h = bitcast<half2_t>(and_or(__builtin_amdgcn_perm(rw.w[ks][r], rw.w[ks][r], bsel[j]),
                                                              nib_mask, exp_bits));
                    d[r] = bitcast<uint32_t>(__builtin_elementwise_fma(h - off, s2, c2));
                }
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

    // One step: the 32 MFMAs of (A, B), ordered ks, i, j, with the rest of the
    // step's work spread evenly between them (a wave issues in order): after MFMA
    // idx, half of the dequant of one dword of the next B (idx even: perm and
    // and_or; odd: the subtract and the FMA; dword idx/2 = (j, ks, row), from the
    // words rc read one step earlier, the tile's scale pair built at idx 0 and
    // 16), the next step's A operand idx-1 for idx 1..16, the words of step
    // k_read into rn at idx 17, 18, and with copies, copy idx/2 - 1 at the even
    // idx 2..24.
    auto step = [&](auto with_copies, int s_a, int as_, int s_r, const half8_t (&A)[2][TM],
                    half8_t (&An)[2][TM], const half8_t (&B)[2][TN], half8_t (&Bn)[2][TN], const Raw &rc,
                    Raw &rn, int k_read, int a_slot, int a_t) {
#pragma clang fp contract(off)
        const half2_t off = {(_Float16)1024.0f, (_Float16)64.0f};
        half2_t s2[TN], c2[TN];
        uint32_t xw[16];
        uint4_t bb[2 * TN];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int idx = 0; idx < NMF; ++idx) {
            const int ks = idx / (TM * TN), i = (idx / TN) % TM, j = idx % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks][i], B[ks][j], acc[i][j], 0, 0, 0);
            {
                const int d = idx >> 1, unit = d >> 2, r = d & 3, uj = unit >> 1, uk = unit & 1;
                if ((idx & 1) == 0) {
                    if ((idx & 15) == 0) scale_pair(rc, uj, s2[uj], c2[uj]);
                    xw[d] = and_or(__builtin_amdgcn_perm(rc.w[uk][r], rc.w[uk][r], bsel[uj]), nib_mask, exp_bits);
                } else {
                    bb[unit][r] = bitcast<uint32_t>(__builtin_elementwise_fma(bitcast<half2_t>(xw[d]) - off,
                                                                               s2[uj], c2[uj]));
                    if (r == 3) Bn[uk][uj] = bitcast<half8_t>(bb[unit]);
                }
            }
            if (idx >= 1 && idx <= 2 * TM) {
                const int r = idx - 1;
                An[r / TM][r % TM] = read_a1(a_slot, a_t, r / TM, r % TM);
            }
            if (idx == 17) read_raw_k(k_read, 0, rn);
            if (idx == 18) read_raw_k(k_read, 1, rn);
            if constexpr (decltype(with_copies)::value) {
                if ((idx & 1) == 0 && idx >= 2 && idx / 2 - 1 < GROUP) issue_one(s_a, as_, s_r, idx / 2 - 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Pipeline (stage s = steps 2s, 2s+1), as q4_gemm7: the barrier before step
    // 2s makes A(s+1) and the words of stage s+1 visible and marks every wave
    // done with step 2s-1; the copies issued during step 2s overwrite the slots
    // of stage s-1: A(s+2), then the weights of stage s+3.  vmcnt is in order,
    // so waiting for all but the 4 newest copies covers A(s+1) and raw(s+1).
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
    read_raw_k(0, 0, R0);
    read_raw_k(0, 1, R0);
    read_raw_k(min(1, nk - 1), 0, R1);
    read_raw_k(min(1, nk - 1), 1, R1);
    build_b(R0, B0);
    const int nfull = nk >> 1;
    int slot0 = 0, slot1 = 1, slot2 = 2;         // A slots of stages s, s+1, s+2 (rotating)
    for (int s = 0; s < nfull; ++s) {
        if (s > 0) {
            wait_vmcnt<GROUP - A_LD>();          // A(s+1) and raw(s+1) (own copies) landed
            lds_barrier();                       // visible; every wave done with step 2s-1
        }
        step(std::true_type{}, s + 2, slot2, s + 3, A0, A1, B0, B1, R1, R0, min(2 * s + 2, nk - 1), slot0, 1);
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

    // Epilogue: lane holds columns 2 lrow + j of the wave's 64.  Element-wise
    // stores straight from the accumulators (packing column pairs first made
    // the compiler spill 32 accumulators to scratch here).
    const int rsub = 4 * lhi;
    if (a.S == 1) {
        _Float16 *Y = (_Float16 *)a.Y;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = wcol0 + 2 * lrow + j;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                    if (m < a.M && n < N) Y[(int64_t)m * a.ldy + n] = (_Float16)activate<ACT>(acc[i][j][r]);
                }
            }
        return;
    }
    float *part = a.partials + ((int64_t)tile_id * a.S + z) * (J7_BM * I4G_BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nl = wave * J7_WN + 2 * lrow + j;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                part[ml * I4G_BN + nl] = acc[i][j][r];
            }
        }
}

// Plan: S = the largest power of two (<= 8, at least 32 steps per split) that
// keeps the grid within 256 workgroups (one per CU).
static int i4_gemm7_splits(int64_t M, int64_t K, int64_t N) {
    int S = 1;
    const int64_t t = ((M + J7_BM - 1) / J7_BM) * ((N + I4G_BN - 1) / I4G_BN);
    const int64_t ns = K / 32;
    while (t * S * 2 <= 256 && ns / (S * 2) >= 32 && S < 8) S *= 2;
    if (S > ns) S = 1;
    return S;
}

// i4_gemm6's shape rules, a grid that nearly fills the CUs (at least 160 tiles
// of 256 x 256, or 96 with K >= 8192; us, i4_gemm6 / this kernel: M=1024
// 4096x11008 113.1 / 103.2, M=768 4096x14336 112.1 / 100.7, M=1280 4096x8192
// 110.9 / 99.9, M=640 4096x11008 (129 tiles) 74.9 / 95.2), and byte offsets of X, the packed
// weights and the scales that fit 31 bits (its copies use buffer resources and
// 32-bit scalar offsets).
// MCQ4_I4_GEMM7=0 disables it, =1 takes it whatever the grid (tests).
bool i4_gemm7_supported(int wb, int sz_dt, int64_t M, int64_t K, int64_t N, int64_t gs, const _Float16 *X,
                        int64_t ldx, const void *Y, int64_t ldy) {
    if (opt_is("MCQ4_I4_GEMM7", '0')) return false;
    const bool force = opt_is("MCQ4_I4_GEMM7", '1');
    const int64_t t = ((M + J7_BM - 1) / J7_BM) * ((N + I4G_BN - 1) / I4G_BN);
    return wb == 4 && (sz_dt == DT_F16 || sz_dt == DT_BF16) && N % 128 == 0 && K % 32 == 0 && gs % 32 == 0 &&
           ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 && ((uintptr_t)Y % 4) == 0 && ldy % 2 == 0 &&
           M * ldx * 2 < ((int64_t)1 << 31) && (K / 2) * N < ((int64_t)1 << 31) &&
           ((K + gs - 1) / gs) * N * 2 < ((int64_t)1 << 31) && (force || t >= 160 || (t >= 96 && K >= 8192));
}

size_t i4_gemm7_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const int S = i4_gemm7_splits(M, K, N);
    if (S == 1) return 0;
    const int64_t t = ((M + J7_BM - 1) / J7_BM) * ((N + I4G_BN - 1) / I4G_BN);
    return COUNTER_BYTES + (size_t)t * S * J7_BM * I4G_BN * sizeof(float);
}

template <int SZ, int ACT>
static hipError_t launch_j7(const I4GemmArgs &a, hipStream_t s) {
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)i4_gemm7_kernel<SZ, ACT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)J7_LDS);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    const int ntiles = a.tiles_m * a.tiles_n;
    hipLaunchKernelGGL((i4_gemm7_kernel<SZ, ACT>), dim3(ntiles, 1, a.S), dim3(256), J7_LDS, s, a);
    if (a.S > 1) return launch_i4_gemm_reduce(a, J7_BM, ACT, s);
    return hipGetLastError();
}

template <int SZ>
static hipError_t launch_j7_act(const I4GemmArgs &a, int act, hipStream_t s) {
    if (act == ACT_SILU) return launch_j7<SZ, ACT_SILU>(a, s);
    if (act == ACT_GELU) return launch_j7<SZ, ACT_GELU>(a, s);
    return launch_j7<SZ, ACT_NONE>(a, s);
}

hipError_t launch_i4_gemm7(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                           const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K, int N,
                           int gs, int act, void *ws, hipStream_t s) {
    I4GemmArgs a;
    a.X = X; a.ldx = ldx; a.P = P; a.scales = scales; a.zeros = zeros; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nsteps = K / 32; a.N = N; a.spg = gs / 32; a.spg_magic = i4_spg_magic(a.spg); a.spg_ident = i4_spg_ident(a.spg);
    a.tiles_n = (N + I4G_BN - 1) / I4G_BN;
    a.tiles_m = (M + J7_BM - 1) / J7_BM;
    a.S = i4_gemm7_splits(M, K, N);
    a.partials = nullptr;
    if (a.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    if (sz_dt == DT_F16) return launch_j7_act<DT_F16>(a, act, s);
    return launch_j7_act<DT_BF16>(a, act, s);
}

}  // namespace mcq4
