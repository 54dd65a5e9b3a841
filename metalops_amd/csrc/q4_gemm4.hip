// Prefill-shaped q4_0 matmul (M > 64) on gfx950: barrier-free MFMA GEMM.
//
//   * WG = 256 threads = 4 waves in a 2x2 grid; WG tile BM x 256 (BM = 256 or
//     128); wave tile (BM/2) x 128 of v_mfma_f32_32x32x16_f16 tiles, fp32
//     accumulation.  K advances one q4_0 block (32) per step.
//   * Every wave fetches everything it consumes itself, so waves never wait for
//     each other and no workgroup barrier is needed:
//       - activations: the wave's MFMA A operands (16 bytes per lane and
//         operand) are loaded from global memory (L2-resident; the workgroup's
//         two waves of a row half read the same lines) straight into registers,
//         G4_P steps ahead, in a register ring of G4_P slots;
//       - weights: the raw q4_0 bytes of the wave's 128 columns for one step
//         (2304 contiguous bytes) are copied with three global_load_lds_dwordx4
//         into a private LDS ring of G4_P + 1 slots, G4_P steps ahead.
//   * B operand of lane l (column n = l%32 of a 32-column MFMA tile, K elements
//     8*(l/32)..+8 of a 16-wide K half): the qs dword of those 8 elements and
//     the column's scale d from the raw slot, unpacked in natural order to fp16
//     1024+q, minus 1032 (exact) and times d (one rounding: the reference's fp16
//     dequant value).  Step k+1's B operands are built while the MFMAs of step k
//     run.
//   * Per step a wave issues the same number of loads and copies (steps past the
//     end are clamped to the last), so one explicit vmcnt wait per step covers
//     the copies; the compiler's own waits cover the register loads.
//   * Workgroup ids are remapped so each XCD works on a contiguous range of
//     tiles.
//   * Outputs with few tiles split K over grid.z: each split writes an fp32
//     partial tile to the caller's workspace, and a second small kernel on the
//     same stream sums the partials in split order and writes fp16 (the kernel
//     boundary orders the two; no fences or atomics).
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>

#include "q4_gemm4.h"

namespace mcq4 {

#ifndef MCQ4_G4_P
#define MCQ4_G4_P 3
#endif
constexpr int G4_P = MCQ4_G4_P;                // steps in flight ahead of the MFMAs
constexpr int G4_R = G4_P + 1;                 // raw ring slots per wave
constexpr int G4_RAW_W = 18 * 128;             // raw bytes per wave and step (2304)
constexpr int G4_RAW_SLOT = G4_RAW_W + 64;     // + read overhang



template <int BM, int WGM>
__global__ void __launch_bounds__(WGM * 128, 1)
q4_gemm4_kernel(Gemm4Args a) {
    // WGM waves along M x 2 along N.  WGM = 2: one wave per SIMD, B operands
    // double-buffered in registers.  WGM = 4: two waves per SIMD (<= 256
    // registers each), B built just in time per 32-column tile.
    constexpr bool JIT_B = WGM == 4;
    constexpr int WM = BM / WGM, WN = G4_BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int A_LD = 2 * TM;                 // register loads per step
    constexpr int GROUP = A_LD + 3;              // vector-memory instructions per step
    static_assert((G4_P - 1) * GROUP < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;     // wm < WGM

    const int ntiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x;
    int tile_id = bid;
    if (ntiles % 8 == 0) tile_id = (bid % 8) * (ntiles / 8) + bid / 8;
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * BM, n0 = tn * G4_BN;
    // K range of this split: steps [k_lo, k_lo + nk).
    const int z = (int)blockIdx.z;
    const int k_lo = (int)((int64_t)a.nb * z / a.S);
    const int nk = (int)((int64_t)a.nb * (z + 1) / a.S) - k_lo;

    const int lrow = lane & 31, lhi = lane >> 5;
    // A operand (i, ks) of step k: row m0 + wm*WM + 32 i + lrow, halves 32k + 16ks + 8lhi.
    const _Float16 *a_src[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = min(m0 + wm * WM + 32 * i + lrow, a.M - 1);
        a_src[i] = a.X + (int64_t)m * a.ldx + (int64_t)k_lo * QK + 8 * lhi;
    }
    // Raw copies: chunk q = lane + 64 c (q < 144) of the wave's 2304-byte segment.
    uint8_t *ring = smem + wave * (G4_R * G4_RAW_SLOT);
    const int64_t row_bytes = (int64_t)a.N * BLOCK_BYTES;
    const uint8_t *w_k = a.W + (int64_t)k_lo * row_bytes;
    const uint8_t *w_src = w_k + (int64_t)(n0 + wn * WN) * BLOCK_BYTES + 16 * lane;
    const bool wcols = n0 + wn * WN < a.N;       // whole wave past N: copy column 0 instead
    const uint8_t *w_base = wcols ? w_src : w_k + 16 * lane;

    half8_t av[G4_P][2][TM];
    auto load_a = [&](int k, half8_t (&dst)[2][TM]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
                dst[ks][i] = *(const half8_t *)(a_src[i] + (int64_t)k * QK + 16 * ks);
    };
    auto copy_raw = [&](int k) {
        const uint8_t *src = w_base + (int64_t)k * row_bytes;
        uint8_t *dst = ring + (k % G4_R) * G4_RAW_SLOT;
#pragma unroll
        for (int c = 0; c < 3; ++c)
            if (c < 2 || lane < 16)
                __builtin_amdgcn_global_load_lds(
                    (void *)(src + 1024 * c),
                    (__attribute__((address_space(3))) void *)(dst + 1024 * c), 16, 0, 0);
    };

    // B operand addresses within a raw slot (columns relative to the wave's 128).
    const int qoff0 = 18 * lrow + 2 + 4 * lhi;   // + 18*32 j + 8 ks
    const int q_al = qoff0 & ~3;
    const uint32_t q_sh = (uint32_t)(qoff0 & 3) * 8;
    const int d_off = 18 * lrow;
    auto load_b = [&](int k, half8_t (&bv)[2][TN]) {
        const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k % G4_R) * G4_RAW_SLOT));
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

    // ---- prologue: steps 0..P-1 in flight (A then raw per step) ----------------
#pragma unroll
    for (int p = 0; p < G4_P; ++p) {
        const int kp = min(p, nk - 1);
        load_a(kp, av[p]);
        copy_raw(kp);
    }
    half8_t bcur[2][TN];
    if constexpr (!JIT_B) {
        wait_vmcnt<(G4_P - 1) * GROUP>();         // step 0 (and everything older) landed
        load_b(0, bcur);
    }

    // One step: MFMAs of step k (A ring slot S), then step k+P's loads into the
    // freed slot S.  Double-buffered B: step k+1's B is built during step k's
    // MFMAs.  Just-in-time B: each 32-column tile's B is built right before its
    // MFMAs (the other wave on the SIMD covers the latency).
    auto step = [&](int k, half8_t (&a_cur)[2][TM]) {
        if constexpr (JIT_B) {
            wait_vmcnt<(G4_P - 1) * GROUP>();     // step k's raw copies landed
            const lds_u8 *Rs = lds_ptr(lds_addr(ring + (k % G4_R) * G4_RAW_SLOT));
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const lds_u32 *qp = (const lds_u32 *)(Rs + q_al + j * 32 * 18);
                uint32_t qd[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) qd[t] = qp[t];
                const uint32_t dd = *(const lds_u16 *)(Rs + d_off + j * 32 * 18);
                const half2_t d2 = bitcast<half2_t>(__builtin_amdgcn_perm(dd, dd, 0x01000100u));
                half8_t bv[2];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    bv[ks] = dequant8_nat(__builtin_amdgcn_alignbit(qd[2 * ks + 1], qd[2 * ks], q_sh), d2);
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_cur[ks][i], bv[ks],
                                                                            acc[i][j], 0, 0, 0);
            }
        } else {
            wait_vmcnt<(G4_P - 2) * GROUP>();     // step k+1's raw copies landed
            half8_t bnxt[2][TN];
            load_b(min(k + 1, nk - 1), bnxt);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_cur[ks][i], bcur[ks][j],
                                                                            acc[i][j], 0, 0, 0);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int j = 0; j < TN; ++j) bcur[ks][j] = bnxt[ks][j];
        }
        const int kn = min(k + G4_P, nk - 1);
        load_a(kn, a_cur);
        copy_raw(kn);
    };

    int k = 0;
    for (; k + G4_P <= nk; k += G4_P) {
#pragma unroll
        for (int u = 0; u < G4_P; ++u) step(k + u, av[u]);
    }
#pragma unroll
    for (int u = 0; u < G4_P; ++u)
        if (k + u < nk) step(k + u, av[u]);
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
    // Split-K: this split's fp32 partial tile (dense BM x 256, row-major); the
    // reduction kernel launched right after sums the splits in order.
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

// Sums the S fp32 partial tiles of every output tile in split order
// (deterministic) and stores fp16; four consecutive columns per thread.
template <int BM>
__global__ void __launch_bounds__(256)
q4_gemm4_reduce_kernel(Gemm4Args a) {
    constexpr int TILE = BM * G4_BN;
    const int64_t v4 = (int64_t)blockIdx.x * 256 + threadIdx.x;     // float4 index
    const int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n;
    if (v4 >= ntiles * (TILE / 4)) return;
    const int64_t tile = v4 / (TILE / 4);
    const int e = (int)(v4 % (TILE / 4)) * 4;
    const int tm = (int)(tile % a.tiles_m), tn = (int)(tile / a.tiles_m);
    const float4_t *p = (const float4_t *)(a.partials + tile * a.S * TILE + e);
    float4_t sum = p[0];
    for (int sp = 1; sp < a.S; ++sp) sum += p[(int64_t)sp * (TILE / 4)];
    const int m = tm * BM + e / G4_BN, n = tn * G4_BN + e % G4_BN;
    if (m >= a.M) return;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (n + c < a.N) a.Y[(int64_t)m * a.ldy + n + c] = (_Float16)sum[c];
}

hipError_t launch_gemm4_reduce(const Gemm4Args &a, int bm, hipStream_t s) {
    const int64_t n4 = (int64_t)a.tiles_m * a.tiles_n * (bm * G4_BN / 4);
    const dim3 grid((unsigned)((n4 + 255) / 256));
    if (bm == 256) hipLaunchKernelGGL((q4_gemm4_reduce_kernel<256>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((q4_gemm4_reduce_kernel<128>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int BM, int WGM>
static hipError_t launch_g4(const Gemm4Args &a, hipStream_t s) {
    constexpr size_t lds = (size_t)(2 * WGM) * G4_R * G4_RAW_SLOT;
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm4_kernel<BM, WGM>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((q4_gemm4_kernel<BM, WGM>), dim3(a.tiles_m * a.tiles_n, 1, a.S),
                       dim3(WGM * 128), lds, s, a);
    if (a.S > 1) return launch_gemm4_reduce(a, BM, s);
    return hipGetLastError();
}

// Needs N % 128 == 0 (every wave's 128 columns are whole, 16-byte aligned raw
// segments), a 16-byte aligned weight base, and 16-byte aligned activation rows.
bool gemm4_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t K, int64_t N) {
    return N % 128 == 0 && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 &&
           K >= QK;
}

// Row-tile height and K splits: BM = 128 when 256-row tiles would leave fewer
// than 192 tiles; K is split (powers of two, at least 16 steps per split) until
// about 192 workgroups have work.
G4Cfg gemm4_config(int64_t M, int64_t K, int64_t N) {
    const int64_t tn = (N + G4_BN - 1) / G4_BN;
    G4Cfg c{256, 1};
    if (((M + 255) / 256) * tn < 192) c.bm = 128;
    if (const char *env = getenv("MCQ4_GEMM2_BM")) c.bm = atoi(env) == 128 ? 128 : 256;
    const int64_t t = ((M + c.bm - 1) / c.bm) * tn;
    const int64_t nb = K / QK;
    while (t * c.S < 192 && nb / (c.S * 2) >= 16 && c.S < 16) c.S *= 2;
    if (const char *env = getenv("MCQ4_GEMM4_SPLIT")) c.S = std::max(1, std::min(16, atoi(env)));
    if (c.S > nb) c.S = 1;
    return c;
}

size_t gemm4_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const G4Cfg c = gemm4_config(M, K, N);
    if (c.S == 1) return 0;
    const int64_t t = ((M + c.bm - 1) / c.bm) * ((N + G4_BN - 1) / G4_BN);
    // Partials follow the workspace's counter area, which stays untouched (zero)
    // for the kernels that use it.
    return COUNTER_BYTES + (size_t)t * c.S * c.bm * G4_BN * sizeof(float);
}

hipError_t launch_gemm4(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    const G4Cfg c = gemm4_config(M, K, N);
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
    int wgm = 2;
    if (const char *env = getenv("MCQ4_GEMM4_WGM")) wgm = atoi(env) == 4 ? 4 : 2;
    if (c.bm == 256) return wgm == 4 ? launch_g4<256, 4>(a, s) : launch_g4<256, 2>(a, s);
    return wgm == 4 ? launch_g4<128, 4>(a, s) : launch_g4<128, 2>(a, s);
}

}  // namespace mcq4
