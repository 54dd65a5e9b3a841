// Prefill-shaped q4_0 matmul (M > 64) on gfx950: asynchronous-copy MFMA GEMM
// with the weights dequantized per wave, straight from the raw q4_0 bytes in
// LDS into MFMA operand registers.
//
//   * WG = 256 threads = 4 waves in a 2x2 grid; WG tile BM x 256 (BM = 256 or
//     128); wave tile (BM/2) x 128 of v_mfma_f32_32x32x16_f16 tiles, fp32
//     accumulation.  K advances one q4_0 block (32) per step.
//   * A G3_STAGES-slot LDS ring receives, per K step, the activation tile (BM
//     rows x 64 bytes, 16-byte chunks XOR-swizzled per row) and the raw q4_0
//     bytes of the step's 256 columns (one contiguous 4608-byte row segment)
//     through global_load_lds_dwordx4 copies issued G3_STAGES-1 steps ahead.
//   * B operand of lane l (column n = l%32 of a 32-column MFMA tile, K elements
//     8*(l/32)..+8 of a 16-wide K half): the qs dword of those 8 elements and
//     the column's scale d, read from the raw slot, unpacked in natural order to
//     fp16 1024+q, minus 1032 (exact) and times d (one rounding: the
//     reference's fp16 dequant value).  Compared with a shared fp16 B tile this
//     moves 2.3 KB of raw bytes per wave and step through LDS instead of
//     writing and re-reading 16 KB of fp16 weights.
//   * Software pipeline: while the MFMAs of step k run on operands held in
//     registers, the wave reads and dequantizes step k+1's operands (landed and
//     made visible by the previous iteration's barrier).  One barrier per step.
//   * Workgroup ids are remapped so each XCD works on a contiguous range of
//     tiles.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>

#include "q4_common.h"

namespace mcq4 {

constexpr int G3_THREADS = 256;
constexpr int G3_BN = 256;
#ifndef MCQ4_G3_STAGES
#define MCQ4_G3_STAGES 5
#endif
constexpr int G3_STAGES = MCQ4_G3_STAGES;
constexpr int G3_RAW = 18 * G3_BN;    // raw q4 bytes of one K step (288 16-byte chunks)
#ifndef MCQ4_G3_VPM
#define MCQ4_G3_VPM 6
#endif
constexpr int G3_VALU_PER_MFMA = MCQ4_G3_VPM;   // dequant VALU slots after each MFMA


struct Gemm3Args {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int tiles_m, tiles_n;
    int64_t w_last_chunk;  // byte offset of the last 16-byte chunk of W
};

template <int BM>
struct G3Layout {
    static constexpr int A_STAGE = BM * 64;
    static constexpr int A_OFF = 0;
    static constexpr int RAW_OFF = A_OFF + G3_STAGES * A_STAGE;
    static constexpr int BYTES = RAW_OFF + G3_STAGES * (G3_RAW + 64);   // + read overhang
    static constexpr int A_LOADS = BM * 4 / 64 / 4;   // 1 KiB copies per wave per step
};

template <int BM>
__global__ void __launch_bounds__(G3_THREADS, 1)
q4_gemm3_kernel(Gemm3Args a) {
    using L = G3Layout<BM>;
    constexpr int WM = BM / 2, WN = G3_BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LOADS_PER_STEP = L::A_LOADS + 2;  // + raw main + raw tail
    constexpr int RAW_SLOT = G3_RAW + 64;
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
    const int m0 = tm * BM, n0 = tn * G3_BN;
    const int nk = a.nb;

    // ---- per-lane async-copy sources ------------------------------------------
    // A copy i of this wave fills LDS chunk p = 64*(wave + 4i) + lane of the slot:
    // row r = p/4, stored chunk p%4 holds logical chunk (p%4) ^ (((r>>1) ^ (r>>3)) & 3).
    const _Float16 *a_src[L::A_LOADS];
#pragma unroll
    for (int i = 0; i < L::A_LOADS; ++i) {
        const int p = 64 * (wave + 4 * i) + lane;
        const int r = p >> 2;
        const int q = (p & 3) ^ (((r >> 1) ^ (r >> 3)) & 3);
        const int m = min(m0 + r, a.M - 1);
        a_src[i] = a.X + (int64_t)m * a.ldx + 8 * q;
    }
    // Raw q4 copies: main chunk 64*wave + lane, tail chunk 256 + 8*wave + lane (lanes < 8).
    const int64_t row_bytes = (int64_t)a.N * BLOCK_BYTES;
    const int64_t raw0 = (int64_t)n0 * BLOCK_BYTES;
    const int64_t rc_main = raw0 + 16 * (64 * wave + lane);
    const int64_t rc_tail = raw0 + 16 * (256 + 8 * wave + (lane & 7));

    auto issue = [&](int k) {
        const int slot = k % G3_STAGES;
#pragma unroll
        for (int i = 0; i < L::A_LOADS; ++i)
            __builtin_amdgcn_global_load_lds(
                (void *)(a_src[i] + (int64_t)k * QK),
                (__attribute__((address_space(3))) void *)(smem + L::A_OFF + slot * L::A_STAGE +
                                                           1024 * (wave + 4 * i)),
                16, 0, 0);
        const int64_t rb = (int64_t)k * row_bytes;
        __builtin_amdgcn_global_load_lds(
            (void *)(a.W + imin64(rb + rc_main, a.w_last_chunk)),
            (__attribute__((address_space(3))) void *)(smem + L::RAW_OFF + slot * RAW_SLOT +
                                                       1024 * wave),
            16, 0, 0);
        if (lane < 8)
            __builtin_amdgcn_global_load_lds(
                (void *)(a.W + imin64(rb + rc_tail, a.w_last_chunk)),
                (__attribute__((address_space(3))) void *)(smem + L::RAW_OFF + slot * RAW_SLOT +
                                                           4096 + 128 * wave),
                16, 0, 0);
    };

    // ---- operand addresses -------------------------------------------------------
    const int lrow = lane & 31, lhi = lane >> 5;
    const int swz = ((lrow >> 1) ^ (lrow >> 3)) & 3;
    int a_rd[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) a_rd[ks] = (wm * WM + lrow) * 64 + 16 * ((2 * ks + lhi) ^ swz);
    // B: column c_j = wn*128 + 32 j + lrow; its block at 18 c_j; the qs dword of
    // half ks at 18 c_j + 2 + 8 ks + 4 lhi, read as the aligned dword pair around it.
    const int qoff0 = 18 * (wn * WN + lrow) + 2 + 4 * lhi;     // + 18*32 j + 8 ks
    const int q_al = qoff0 & ~3;                               // 18*32 j and 8 ks keep alignment
    const uint32_t q_sh = (uint32_t)(qoff0 & 3) * 8;
    const int d_off = 18 * (wn * WN + lrow);

    struct Ops {
        half8_t av[2][TM], bv[2][TN];
    };
    // Reads step k's operands from its slot and dequantizes B.
    auto load_ops = [&](int k, Ops &o) {
        const int slot = k % G3_STAGES;
        const lds_u8 *As = lds_ptr(lds_addr(smem + L::A_OFF + slot * L::A_STAGE));
        const lds_u8 *Rs = lds_ptr(lds_addr(smem + L::RAW_OFF + slot * RAW_SLOT));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i) o.av[ks][i] = *(const lds_half8 *)(As + a_rd[ks] + i * 32 * 64);
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
            for (int ks = 0; ks < 2; ++ks) {
                const uint32_t w = __builtin_amdgcn_alignbit(qd[j][2 * ks + 1], qd[j][2 * ks], q_sh);
                o.bv[ks][j] = dequant8_nat(w, d2);
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

    // ---- prologue: steps 0..S-2 in flight; steps 0 and 1 landed; step 0 loaded --
    // Steps past the last are clamped to it, so every wait counts the same
    // number of copies per step.
#pragma unroll
    for (int k = 0; k < G3_STAGES - 1; ++k) issue(min(k, nk - 1));
    wait_vmcnt<(G3_STAGES - 3) * LOADS_PER_STEP>();
    lds_barrier();
    Ops cur;
    load_ops(0, cur);

    for (int k = 0; k < nk; ++k) {
        issue(min(k + G3_STAGES - 1, nk - 1));
        Ops nxt;
        load_ops(min(k + 1, nk - 1), nxt);      // landed and visible since the last barrier
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.av[ks][i], cur.bv[ks][j],
                                                                        acc[i][j], 0, 0, 0);
        // Schedule: next step's LDS reads first, then each MFMA followed by a
        // slice of the next step's dequant arithmetic, so the matrix core never
        // waits behind a block of VALU work (one wave per SIMD, in-order issue).
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * TM + 3 * TN, 0);      // DS reads
#pragma unroll
        for (int i = 0; i < 2 * TM * TN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, G3_VALU_PER_MFMA, 0); // VALU
        }
        // Step k+2 must have landed (and every wave be past its reads of the slot
        // the next iteration's copies refill) before the next iteration.
        wait_vmcnt<(G3_STAGES - 3) * LOADS_PER_STEP>();
        lds_barrier();
        cur = nxt;
    }
    wait_vmcnt<0>();

    // ---- epilogue ----------------------------------------------------------------
    const int col_l = lane & 31, rsub = 4 * lhi;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn * WN + j * 32 + col_l;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)acc[i][j][r];
            }
        }
}

template <int BM>
static hipError_t launch_g3(const Gemm3Args &a, hipStream_t s) {
    using L = G3Layout<BM>;
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm3_kernel<BM>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::BYTES);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((q4_gemm3_kernel<BM>), dim3(a.tiles_m * a.tiles_n), dim3(G3_THREADS),
                       L::BYTES, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm3(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, hipStream_t s) {
    Gemm3Args a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.w_last_chunk = (int64_t)a.nb * N * BLOCK_BYTES - 16;
    a.tiles_n = (N + G3_BN - 1) / G3_BN;
    int bm = 256;
    if (((int64_t)(M + 255) / 256) * a.tiles_n < 192) bm = 128;
    if (const char *env = getenv("MCQ4_GEMM2_BM")) bm = atoi(env) == 128 ? 128 : 256;
    a.tiles_m = (M + bm - 1) / bm;
    if (bm == 256) return launch_g3<256>(a, s);
    return launch_g3<128>(a, s);
}

}  // namespace mcq4
