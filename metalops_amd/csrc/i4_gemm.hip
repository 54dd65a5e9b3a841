// Prefill-shaped (M > 16) per-group INT4 / INT8 matmul on gfx950: barrier-free
// MFMA GEMM.  The description is for INT4; INT8 (int8 [K][N], quantization.py
// :242-286) differs only in the raw step (32 byte rows, four copies) and the
// unpack (byte pairs of rows 2r, 2r+1 -> fp16 1152 + q).
//
//   * WG = 256 threads = 4 waves in a 2x2 grid; WG tile BM x 256 (BM = 256 or
//     128); wave tile (BM/2) x 128 of v_mfma_f32_32x32x16_f16 tiles, fp32
//     accumulation.  K advances 32 rows (16 byte rows of packed[K/2][N]) per step.
//   * Every wave fetches what it consumes itself (no workgroup barrier):
//       - activations: the wave's MFMA A operands straight into a register ring
//         I4G_P steps ahead;
//       - weights: the wave's 16 x 128 raw bytes of the step, two
//         global_load_lds_dwordx4 per step (row-major [16][128] in a private
//         LDS ring of I4G_P + 1 slots), I4G_P steps ahead;
//       - scales/zeros of the step's group for the wave's 128 columns, one
//         more global_load_lds_dwordx4 into the same ring slot (L2 hits).
//     Every step issues the same loads (steps past the end are clamped), so
//     one explicit vmcnt wait per step covers the LDS copies.
//   * B operand: MFMA tile j (0..3) column l%32 is the wave's column 4*(l%32) + j,
//     so one ds_read_b32 of a byte row serves all four tiles.  Lane half l/32
//     takes K elements 8*(l/32)..+8 of each 16-wide K half (byte rows
//     8ks + 4(l/32) + r).  Per byte row: v_perm_b32 + v_and_or_b32 give the fp16
//     pair {1024 + q(2r), 1024 + q(2r+1)}; minus 1024 (exact) gives q; one fp16
//     FMA gives q*s + c with c = -z*s (fp32 product rounded to fp16): the
//     dequantized weight (q - z)*s to fp16 precision.  The operands are built
//     while earlier MFMAs run (a step ahead for BM = 128, a 32-column tile
//     ahead for BM = 256).
//   * Outputs with few tiles split K over grid.z; the splits' fp32 partial
//     tiles are summed in split order by a second kernel on the same stream.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "i4_gemm.h"

namespace mcq4 {

constexpr int I4G_P = 3;                       // steps in flight ahead of the MFMAs
constexpr int I4G_R = I4G_P + 1;               // raw ring slots per wave

// Per weight format (WB = bits per weight): 32 K per step either way; INT4 packs
// two rows per byte (16 byte rows per step), INT8 one (32 rows).
template <int WB>
struct I4gFmt {
    static constexpr int ROWS = WB == 4 ? 16 : 32;          // byte rows per step
    static constexpr int RAW = ROWS * 128;                   // raw bytes per wave and step
    static constexpr int SLOT = RAW + 1024;                  // + scales/zeros of 128 columns (fp32)
    static constexpr int COPIES = RAW / 1024;                // global_load_lds_dwordx4 per step
    static constexpr size_t LDS = (size_t)4 * I4G_R * SLOT;  // 4 waves
};



template <int BM, int SZ, int ACT, int WB>
__global__ void __launch_bounds__(256, 1)
i4_gemm_kernel(I4GemmArgs a) {
    constexpr int I4G_RAW = I4gFmt<WB>::RAW, I4G_SLOT = I4gFmt<WB>::SLOT;
    constexpr int ROWS = I4gFmt<WB>::ROWS, COPIES = I4gFmt<WB>::COPIES;
    constexpr int RPL = ROWS / 4;                // byte rows per lane and K half (4 or 8)
    constexpr int WM = BM / 2, WN = I4G_BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;   // TN = 4
    static_assert(TN == 4, "four 32-column tiles per wave");
    constexpr int A_LD = 2 * TM;
    constexpr int GROUP = A_LD + COPIES + 1;    // vector-memory instructions per step
    static_assert((I4G_P - 1) * GROUP < 64, "vmcnt range");
    constexpr int ESZ = SZ == DT_F32 ? 4 : 2;
    constexpr int SZ_LANES = 128 * ESZ / 16;    // lanes per scale (or zero) row copy
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
    const int m0 = tm * BM, n0 = tn * I4G_BN;
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nsteps * z / a.S);
    const int nk = (int)((int64_t)a.nsteps * (z + 1) / a.S) - k_lo;

    const int lrow = lane & 31, lhi = lane >> 5;
    const int N = a.N;
    // A operand (i, ks) of step k: row m0 + wm*WM + 32 i + lrow, halves 32k + 16ks + 8lhi.
    const _Float16 *a_src[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = min(m0 + wm * WM + 32 * i + lrow, a.M - 1);
        a_src[i] = a.X + (int64_t)m * a.ldx + (int64_t)k_lo * 32 + 8 * lhi;
    }
    // Raw copies: copy c of a step = byte rows 8c .. 8c+7 (lane: row 8c + l/8, 16-byte piece l%8).
    uint8_t *ring = smem + wave * (I4G_R * I4G_SLOT);
    const int wcol = n0 + wn * WN;
    const bool wcols = wcol < N;                 // whole wave past N: copy column 0 instead
    const uint8_t *w_base = a.P + (int64_t)k_lo * ROWS * N + (int64_t)(lane >> 3) * N +
                            (wcols ? wcol : 0) + 16 * (lane & 7);
    // Scale/zero copy: lanes 0..SZ_LANES-1 copy the scale row, the next
    // SZ_LANES lanes the zero row (16 bytes each) of the wave's 128 columns.
    const bool sz_lane = lane < 2 * SZ_LANES;
    const int sz_li = lane < SZ_LANES ? lane : lane - SZ_LANES;
    const uint8_t *sz_src = (const uint8_t *)(lane < SZ_LANES ? a.scales : a.zeros) +
                            (int64_t)((wcols ? wcol : 0) * ESZ + 16 * sz_li);

    half8_t av[I4G_P][2][TM];
    auto load_a = [&](int k, half8_t (&dst)[2][TM]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
                dst[ks][i] = *(const half8_t *)(a_src[i] + (int64_t)k * 32 + 16 * ks);
    };
    auto copy_raw = [&](int k) {
        const uint8_t *src = w_base + (int64_t)k * ROWS * N;
        uint8_t *dst = ring + (k % I4G_R) * I4G_SLOT;
#pragma unroll
        for (int c = 0; c < COPIES; ++c)
            __builtin_amdgcn_global_load_lds(
                (void *)(src + (int64_t)8 * c * N),
                (__attribute__((address_space(3))) void *)(dst + 1024 * c), 16, 0, 0);
        const int64_t grp = i4_group_of(k_lo + k, a.spg_magic, a.spg_ident);
        if (sz_lane)
            __builtin_amdgcn_global_load_lds(
                (void *)(sz_src + grp * N * ESZ),
                (__attribute__((address_space(3))) void *)(dst + I4G_RAW), 16, 0, 0);
    };

    const uint32_t c64 = opaque_vgpr(0x64006400u);
    const uint32_t mlo = opaque_sgpr(0x000F000Fu);
    // fp16 value of code 0 in the unpacked pair: 1024 (INT4) or 1152 (INT8, q + 128).
    const half2_t m1024 = WB == 4 ? half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f}
                                  : half2_t{(_Float16)-1152.0f, (_Float16)-1152.0f};
    // B source of a step: the lane's eight raw dwords and the fp16 scale and
    // offset pairs of its four columns.
    struct BSrc {
        uint32_t raw[2][RPL];
        half2_t s2[4], c2[4];
    };
    auto fetch_b = [&](int k, BSrc &b) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k % I4G_R) * I4G_SLOT));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int r = 0; r < RPL; ++r)
                b.raw[ks][r] = *(const lds_u32 *)(Rs + (2 * RPL * ks + RPL * lhi + r) * 128 + 4 * lrow);
        float s[4], zz[4];
        typedef __attribute__((address_space(3))) float4_t lds_f4;
        typedef __attribute__((address_space(3))) u32x2 lds_u2;
        if constexpr (SZ == DT_F32) {
            const float4_t s_f = *(const lds_f4 *)(Rs + I4G_RAW + 16 * lrow);
            const float4_t z_f = *(const lds_f4 *)(Rs + I4G_RAW + 512 + 16 * lrow);
#pragma unroll
            for (int j = 0; j < 4; ++j) { s[j] = s_f[j]; zz[j] = z_f[j]; }
        } else {
            const u32x2 s_in = *(const lds_u2 *)(Rs + I4G_RAW + 8 * lrow);
            const u32x2 z_in = *(const lds_u2 *)(Rs + I4G_RAW + 256 + 8 * lrow);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (SZ == DT_F16) {
                    s[j] = (float)bitcast<half2_t>(s_in[j >> 1])[j & 1];
                    zz[j] = (float)bitcast<half2_t>(z_in[j >> 1])[j & 1];
                } else {
                    s[j] = __uint_as_float((j & 1) ? (s_in[j >> 1] & 0xFFFF0000u) : (s_in[j >> 1] << 16));
                    zz[j] = __uint_as_float((j & 1) ? (z_in[j >> 1] & 0xFFFF0000u) : (z_in[j >> 1] << 16));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const _Float16 sh = (_Float16)s[j], ch = (_Float16)(-zz[j] * s[j]);
            b.s2[j] = half2_t{sh, sh};
            b.c2[j] = half2_t{ch, ch};
        }
    };
    // B operands (both K halves) of 32-column MFMA tile j.
    auto build_b = [&](const BSrc &b, int j, half8_t (&bv)[2]) {
        const uint32_t sel = (uint32_t)j | (uint32_t)j << 8 | (uint32_t)(4 + j) << 16 |
                             (uint32_t)(4 + j) << 24;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            uint4_t d;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t pair;
                if constexpr (WB == 4) {
                    const uint32_t w = b.raw[ks][r];
                    pair = and_or(__builtin_amdgcn_perm(w >> 4, w, sel), mlo, c64);
                } else {
                    // bytes of K rows 2r, 2r+1 to positions 0 and 2; the xor flips
                    // the sign bit (q + 128) and sets the 0x64 exponent bytes.
                    const uint32_t sel8 = (uint32_t)j | 0x0Cu << 8 | (uint32_t)(4 + j) << 16 | 0x0Cu << 24;
                    pair = __builtin_amdgcn_perm(b.raw[ks][2 * r + 1], b.raw[ks][2 * r], sel8) ^ 0x64806480u;
                }
                const half2_t q = bitcast<half2_t>(pair) + m1024;
                d[r] = bitcast<uint32_t>(__builtin_elementwise_fma(q, b.s2[j], b.c2[j]));
            }
            bv[ks] = bitcast<half8_t>(d);
        }
    };
    auto load_b = [&](int k, half8_t (&bv)[2][TN]) {
        BSrc b;
        fetch_b(k, b);
        half8_t t[2];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            build_b(b, j, t);
            bv[0][j] = t[0];
            bv[1][j] = t[1];
        }
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

#pragma unroll
    for (int p = 0; p < I4G_P; ++p) {
        const int kp = min(p, nk - 1);
        load_a(kp, av[p]);
        copy_raw(kp);
    }
    // Double-buffered B (BM = 128): step k+1's operands are built during step
    // k's MFMAs.  Tile-ahead B (BM = 256, where the accumulators leave no room
    // for a second full set): within a step, tile j+1's operands are built
    // while tile j's MFMAs run.
    constexpr bool DB = BM == 128;
    half8_t bcur[2][TN];
    if constexpr (DB) {
        wait_vmcnt<(I4G_P - 1) * GROUP>();       // step 0 (and everything older) landed
        load_b(0, bcur);
    }

    // Step k uses A ring slot u = k % P; afterwards slot u is refilled with step k+P.
    auto step = [&](int k, int u) {
        if constexpr (DB) {
            wait_vmcnt<(I4G_P - 2) * GROUP>();   // step k+1's raw copies landed
            half8_t bnxt[2][TN];
            load_b(min(k + 1, nk - 1), bnxt);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[u][ks][i], bcur[ks][j],
                                                                            acc[i][j], 0, 0, 0);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int j = 0; j < TN; ++j) bcur[ks][j] = bnxt[ks][j];
        } else {
            wait_vmcnt<(I4G_P - 1) * GROUP>();   // step k's raw copies landed
            BSrc b;
            fetch_b(k, b);
            half8_t bj[2];
            build_b(b, 0, bj);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                half8_t bn[2];
                if (j + 1 < TN) build_b(b, j + 1, bn);
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[u][ks][i], bj[ks],
                                                                            acc[i][j], 0, 0, 0);
                if (j + 1 < TN) { bj[0] = bn[0]; bj[1] = bn[1]; }
            }
        }
        const int kn = min(k + I4G_P, nk - 1);
        load_a(kn, av[u]);
        copy_raw(kn);
    };

    int k = 0;
    for (; k + I4G_P <= nk; k += I4G_P) {
#pragma unroll
        for (int u = 0; u < I4G_P; ++u) step(k + u, u);
    }
#pragma unroll
    for (int u = 0; u < I4G_P; ++u)
        if (k + u < nk) step(k + u, u);
    wait_vmcnt<0>();

    // ---- epilogue: lane holds columns 4*lrow + j (j = 0..3) of the wave's 128 ----
    const int rsub = 4 * lhi;
    if (a.S == 1) {
        _Float16 *Y = (_Float16 *)a.Y;
        const int n = wcol + 4 * lrow;
        if (n >= N) return;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                if (m < a.M) {
                    half4_t v;
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = (_Float16)activate<ACT>(acc[i][j][r]);
                    *(half4_t *)(Y + (int64_t)m * a.ldy + n) = v;
                }
            }
        return;
    }
    float *part = a.partials + ((int64_t)tile_id * a.S + z) * (BM * I4G_BN);
    const int nl = wn * WN + 4 * lrow;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ml = wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
            float4_t v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = acc[i][j][r];
            *(float4_t *)(part + ml * I4G_BN + nl) = v;
        }
}

// Sums the S fp32 partial tiles of every output tile in split order and stores
// act(sum) as fp16; four consecutive columns per thread.
template <int BM, int ACT>
__global__ void __launch_bounds__(256)
i4_gemm_reduce_kernel(I4GemmArgs a) {
    constexpr int TILE = BM * I4G_BN;
    const int64_t v4 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n;
    if (v4 >= ntiles * (TILE / 4)) return;
    const int64_t tile = v4 / (TILE / 4);
    const int e = (int)(v4 % (TILE / 4)) * 4;
    const int tm = (int)(tile % a.tiles_m), tn = (int)(tile / a.tiles_m);
    const float4_t *p = (const float4_t *)(a.partials + tile * a.S * TILE + e);
    float4_t sum = p[0];
    for (int sp = 1; sp < a.S; ++sp) sum += p[(int64_t)sp * (TILE / 4)];
    const int m = tm * BM + e / I4G_BN, n = tn * I4G_BN + e % I4G_BN;
    if (m >= a.M || n >= a.N) return;
    half4_t v;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = (_Float16)activate<ACT>(sum[c]);
    *(half4_t *)((_Float16 *)a.Y + (int64_t)m * a.ldy + n) = v;
}

hipError_t launch_i4_gemm_reduce(const I4GemmArgs &a, int bm, int act, hipStream_t s) {
    const int64_t n4 = (int64_t)a.tiles_m * a.tiles_n * (bm * I4G_BN / 4);
    const dim3 grid((unsigned)((n4 + 255) / 256));
    if (bm == 256) {
        if (act == ACT_SILU) hipLaunchKernelGGL((i4_gemm_reduce_kernel<256, ACT_SILU>), grid, dim3(256), 0, s, a);
        else if (act == ACT_GELU) hipLaunchKernelGGL((i4_gemm_reduce_kernel<256, ACT_GELU>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((i4_gemm_reduce_kernel<256, ACT_NONE>), grid, dim3(256), 0, s, a);
    } else {
        if (act == ACT_SILU) hipLaunchKernelGGL((i4_gemm_reduce_kernel<128, ACT_SILU>), grid, dim3(256), 0, s, a);
        else if (act == ACT_GELU) hipLaunchKernelGGL((i4_gemm_reduce_kernel<128, ACT_GELU>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((i4_gemm_reduce_kernel<128, ACT_NONE>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

template <int BM, int SZ, int ACT, int WB>
static hipError_t launch_i4g(const I4GemmArgs &a, hipStream_t s) {
    constexpr size_t lds = I4gFmt<WB>::LDS;
    if (lds > 64 * 1024) {
        // Raise the kernel's dynamic-LDS limit once per device.
        static std::atomic<uint64_t> done{0};
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        const uint64_t bit = 1ull << (dev & 63);
        if (!(done.load(std::memory_order_acquire) & bit)) {
            e = hipFuncSetAttribute((const void *)i4_gemm_kernel<BM, SZ, ACT, WB>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
            done.fetch_or(bit, std::memory_order_acq_rel);
        }
    }
    hipLaunchKernelGGL((i4_gemm_kernel<BM, SZ, ACT, WB>), dim3(a.tiles_m * a.tiles_n, 1, a.S),
                       dim3(256), lds, s, a);
    if (a.S > 1) return launch_i4_gemm_reduce(a, BM, ACT, s);
    return hipGetLastError();
}

template <int BM, int SZ, int WB>
static hipError_t launch_i4g_act(const I4GemmArgs &a, int act, hipStream_t s) {
    if (act == ACT_SILU) return launch_i4g<BM, SZ, ACT_SILU, WB>(a, s);
    if (act == ACT_GELU) return launch_i4g<BM, SZ, ACT_GELU, WB>(a, s);
    return launch_i4g<BM, SZ, ACT_NONE, WB>(a, s);
}

template <int BM, int WB>
static hipError_t launch_i4g_sz(const I4GemmArgs &a, int sz_dt, int act, hipStream_t s) {
    if (sz_dt == DT_F32) return launch_i4g_act<BM, DT_F32, WB>(a, act, s);
    if (sz_dt == DT_F16) return launch_i4g_act<BM, DT_F16, WB>(a, act, s);
    return launch_i4g_act<BM, DT_BF16, WB>(a, act, s);
}

// Needs N % 128 == 0 (whole 128-column wave strips),
// group_size % 32 == 0, K % 32 == 0, 16-byte aligned packed weights, scales,
// zeros and activation rows, and Y rows that take 8-byte stores.
bool i4_gemm_supported(int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                       const void *P, const void *scales, const void *zeros, const void *Y,
                       int64_t ldy) {
    return N % 128 == 0 && K % 32 == 0 && K >= 32 && gs % 32 == 0 && ldx % 8 == 0 &&
           ((uintptr_t)X % 16) == 0 && ((uintptr_t)P % 16) == 0 &&
           ((uintptr_t)scales % 16) == 0 && ((uintptr_t)zeros % 16) == 0 &&
           ((uintptr_t)Y % 8) == 0 && ldy % 4 == 0 && K / 32 < (1 << 24);
}

struct I4GCfg {
    int bm, S;
};

static I4GCfg i4_gemm_config(int64_t M, int64_t K, int64_t N) {
    const int64_t tn = (N + I4G_BN - 1) / I4G_BN;
    I4GCfg c{256, 1};
    if (((M + 255) / 256) * tn < 192) c.bm = 128;
    const int64_t t = ((M + c.bm - 1) / c.bm) * tn;
    const int64_t ns = K / 32;
    while (t * c.S < 192 && ns / (c.S * 2) >= 16 && c.S < 16) c.S *= 2;
    if (c.S > ns) c.S = 1;
    return c;
}

bool i4_gemm6_supported(int wb, int sz_dt, int64_t M, int64_t K, int64_t N, int64_t gs, int64_t ldx, const void *Y,
                        int64_t ldy);
size_t i4_gemm6_workspace_bytes(int64_t M, int64_t K, int64_t N);
hipError_t launch_i4_gemm6(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                           const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K, int N,
                           int gs, int act, void *ws, hipStream_t s);

bool i4_gemm7_supported(int wb, int sz_dt, int64_t M, int64_t K, int64_t N, int64_t gs, const _Float16 *X,
                        int64_t ldx, const void *Y, int64_t ldy);
size_t i4_gemm7_workspace_bytes(int64_t M, int64_t K, int64_t N);
hipError_t launch_i4_gemm7(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                           const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K, int N,
                           int gs, int act, void *ws, hipStream_t s);

// Covers the three prefill kernels (i4_gemm7 and i4_gemm6 for 4-bit weights
// with 16-bit scales/zeros, this one otherwise).
size_t i4_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const I4GCfg c = i4_gemm_config(M, K, N);
    const int64_t t = ((M + c.bm - 1) / c.bm) * ((N + I4G_BN - 1) / I4G_BN);
    const size_t own = c.S == 1 ? 0 : COUNTER_BYTES + (size_t)t * c.S * c.bm * I4G_BN * sizeof(float);
    return std::max({own, i4_gemm6_workspace_bytes(M, K, N), i4_gemm7_workspace_bytes(M, K, N)});
}

hipError_t launch_i4_gemm(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                          const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K,
                          int N, int gs, int act, void *ws, hipStream_t s, int wb) {
    if (i4_gemm7_supported(wb, sz_dt, M, K, N, gs, X, ldx, Y, ldy))
        return launch_i4_gemm7(X, ldx, P, scales, zeros, sz_dt, Y, ldy, M, K, N, gs, act, ws, s);
    if (i4_gemm6_supported(wb, sz_dt, M, K, N, gs, ldx, Y, ldy))
        return launch_i4_gemm6(X, ldx, P, scales, zeros, sz_dt, Y, ldy, M, K, N, gs, act, ws, s);
    const I4GCfg c = i4_gemm_config(M, K, N);
    I4GemmArgs a;
    a.X = X; a.ldx = ldx; a.P = P; a.scales = scales; a.zeros = zeros; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nsteps = K / 32; a.N = N; a.spg = gs / 32; a.spg_magic = i4_spg_magic(a.spg); a.spg_ident = i4_spg_ident(a.spg);
    a.tiles_n = (N + I4G_BN - 1) / I4G_BN;
    a.tiles_m = (M + c.bm - 1) / c.bm;
    a.S = c.S;
    a.partials = nullptr;
    if (c.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    if (wb == 8) {
        if (c.bm == 256) return launch_i4g_sz<256, 8>(a, sz_dt, act, s);
        return launch_i4g_sz<128, 8>(a, sz_dt, act, s);
    }
    if (c.bm == 256) return launch_i4g_sz<256, 4>(a, sz_dt, act, s);
    return launch_i4g_sz<128, 4>(a, sz_dt, act, s);
}

}  // namespace mcq4
