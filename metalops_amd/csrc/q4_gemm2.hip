// Prefill-shaped q4_0 matmul (M > 64) on gfx950: asynchronous-copy MFMA GEMM.
//
//   * WG = 256 threads = 4 waves in a 2x2 grid; WG tile BM x 256 (BM = 256 or
//     128); wave tile (BM/2) x 128 of v_mfma_f32_32x32x16_f16 tiles, fp32
//     accumulation.  K advances one q4_0 block (32) per step.
//   * A G2_STAGES-slot LDS ring receives, per K step, the activation tile (BM rows x
//     64 bytes) and the raw q4_0 bytes of the step's 256 columns (one 4608-byte
//     contiguous row segment) through global_load_lds_dwordx4: 16-byte async
//     copies that bypass registers.  Copies run G2_STAGES-1 steps ahead.
//   * Each K step the 256 threads dequantize the *next* step's raw blocks (one
//     column each: fp16 (q-8)*d, the reference's fp16 dequant value) into one of
//     two fp16 B buffers, while the MFMAs consume the current one.
//   * Activation rows are 64 bytes in LDS with the 16-byte chunk index XORed by
//     ((row >> 1) ^ (row >> 3)) & 3, so the 16-byte operand reads of 8 (and of
//     16) consecutive rows hit disjoint banks; the fp16 B rows are padded to 80
//     bytes for the same reason.
//   * One barrier per K step.  Workgroup ids are remapped so each XCD works on a
//     contiguous range of tiles.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include <algorithm>
#include <atomic>

#include "q4_common.h"

namespace mcq4 {

constexpr int G2_THREADS = 256;
constexpr int G2_BN = 256;
#ifndef MCQ4_G2_STAGES
#define MCQ4_G2_STAGES 4
#endif
constexpr int G2_STAGES = MCQ4_G2_STAGES;   // async-copy ring slots (prefetch G2_STAGES-1 steps)
constexpr int G2_RAW = 18 * G2_BN;    // raw q4 bytes of one K step (288 16-byte chunks)
constexpr int G2_DQ_ROW = 80;         // bytes per fp16 B row (32 halves + 16 pad)
constexpr int G2_DQ = G2_BN * G2_DQ_ROW;

struct Gemm2Args {
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
struct G2Layout {
    static constexpr int A_STAGE = BM * 64;
    static constexpr int A_OFF = 0;
    static constexpr int RAW_OFF = A_OFF + G2_STAGES * A_STAGE;
    static constexpr int DQ_OFF = RAW_OFF + G2_STAGES * G2_RAW;
    static constexpr int BYTES = DQ_OFF + 2 * G2_DQ;
    static constexpr int A_LOADS = BM * 4 / 64 / 4;   // 1 KiB copies per wave per step
};

template <int BM>
__global__ void __launch_bounds__(G2_THREADS, 1)
q4_gemm2_kernel(Gemm2Args a) {
    using L = G2Layout<BM>;
    constexpr int WM = BM / 2, WN = G2_BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LOADS_PER_STEP = L::A_LOADS + 2;  // + raw main + raw tail
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
    const int m0 = tm * BM, n0 = tn * G2_BN;
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

    auto issue_main = [&](int k) {
        const int slot = k % G2_STAGES;
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
            (__attribute__((address_space(3))) void *)(smem + L::RAW_OFF + slot * G2_RAW +
                                                       1024 * wave),
            16, 0, 0);
    };
    auto issue_tail = [&](int k) {  // lanes 0..7 only
        const int slot = k % G2_STAGES;
        const int64_t rb = (int64_t)k * row_bytes;
            __builtin_amdgcn_global_load_lds(
                (void *)(a.W + imin64(rb + rc_tail, a.w_last_chunk)),
                (__attribute__((address_space(3))) void *)(smem + L::RAW_OFF + slot * G2_RAW +
                                                           4096 + 128 * wave),
                16, 0, 0);
    };

    auto issue = [&](int k) {
        issue_main(k);
        if (lane < 8) issue_tail(k);
    };

    // ---- dequant: thread t -> column t of step k into fp16 buffer (k & 1) -----
    const bool t_even = (tid & 1) == 0;
    const uint32_t dq_sel = t_even ? 0x05040302u : 0x03020100u;  // qs dwords from the pair
    const int raw_q = (18 * tid + 2) & ~3;                         // aligned start of the qs run
    struct RawBlk {
        uint32_t d, dw[5];
    };
    auto dq_read = [&](int k) {
        const int slot = k % G2_STAGES;
        const lds_u8 *raw = lds_ptr(lds_addr(smem + L::RAW_OFF + slot * G2_RAW));
        RawBlk r;
        r.d = *(const lds_u16 *)(raw + 18 * tid);
        const lds_u32 *qp = (const lds_u32 *)(raw + raw_q);
#pragma unroll
        for (int j = 0; j < 5; ++j) r.dw[j] = qp[j];
        return r;
    };
    auto dq_math = [&](const RawBlk &r, uint4_t (&nat)[4]) {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const uint32_t w = __builtin_amdgcn_perm(r.dw[h + 1], r.dw[h], dq_sel);
            const half8_t p = dequant8_perm(w, r.d);   // [e0,e2,e4,e6,e1,e3,e5,e7]
            const uint4_t u = bitcast<uint4_t>(p);
            nat[h][0] = __builtin_amdgcn_perm(u[2], u[0], 0x05040100u);  // e0, e1
            nat[h][1] = __builtin_amdgcn_perm(u[2], u[0], 0x07060302u);  // e2, e3
            nat[h][2] = __builtin_amdgcn_perm(u[3], u[1], 0x05040100u);  // e4, e5
            nat[h][3] = __builtin_amdgcn_perm(u[3], u[1], 0x07060302u);  // e6, e7
        }
    };
    auto dq_write = [&](int k, const uint4_t (&nat)[4]) {
        uint8_t *dst = smem + L::DQ_OFF + (k & 1) * G2_DQ + tid * G2_DQ_ROW;
#pragma unroll
        for (int h = 0; h < 4; ++h) *(uint4_t *)(dst + 16 * h) = nat[h];
    };
    auto dequant = [&](int k) {
        uint4_t nat[4];
        dq_math(dq_read(k), nat);
        dq_write(k, nat);
    };

    // ---- MFMA operand addresses ------------------------------------------------
    const int lrow = lane & 31, lhi = lane >> 5;
    const int swz = ((lrow >> 1) ^ (lrow >> 3)) & 3;
    int a_rd[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) a_rd[ks] = (wm * WM + lrow) * 64 + 16 * ((2 * ks + lhi) ^ swz);
    const int b_rd = (wn * WN + lrow) * G2_DQ_ROW + 16 * lhi;

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // ---- prologue: steps 0..G2_STAGES-2 in flight, step 0 dequantized ----------
    // Steps past the last are clamped to it, so every wait below counts the same
    // number of copies per step.
#pragma unroll
    for (int k = 0; k < G2_STAGES - 1; ++k) issue(min(k, nk - 1));
    wait_vmcnt<(G2_STAGES - 2) * LOADS_PER_STEP>();     // step 0 landed
    lds_barrier();
    dequant(0);
    wait_vmcnt<(G2_STAGES - 3) * LOADS_PER_STEP>();     // step 1 landed
    lds_barrier();

    for (int k = 0; k < nk; ++k) {
        // Copies for step k+G2_STAGES-1 (clamped to the last step near the end, so
        // every iteration issues the same number of copies and the waits stay exact).
        const int kk = min(k + G2_STAGES - 1, nk - 1);
        issue_main(kk);
        if (lane < 8) issue_tail(kk);
        // ---- one basic block: operands, dequant of step k+1, MFMAs of step k ----
        const int kn = min(k + 1, nk - 1);
        const RawBlk raw = dq_read(kn);   // landed and visible since the last barrier
        const lds_u8 *As = lds_ptr(lds_addr(smem + L::A_OFF + (k % G2_STAGES) * L::A_STAGE));
        const lds_u8 *Bs = lds_ptr(lds_addr(smem + L::DQ_OFF + (k & 1) * G2_DQ));
        half8_t av[2][TM], bv[2][TN];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
                av[ks][i] = *(const lds_half8 *)(As + a_rd[ks] + i * 32 * 64);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bv[ks][j] = *(const lds_half8 *)(Bs + b_rd + j * 32 * G2_DQ_ROW + 32 * ks);
        }
        uint4_t nat[4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[ks][i], bv[ks][j],
                                                                        acc[i][j], 0, 0, 0);
        dq_math(raw, nat);
        dq_write(kn, nat);
        // Schedule: raw + first-half operand reads, then MFMAs interleaved 1:3
        // with the dequant arithmetic; second-half operand reads and the dequant
        // stores slot in between.
        __builtin_amdgcn_sched_group_barrier(0x100, 4 + TM + TN, 0);          // DS reads
#pragma unroll
        for (int i = 0; i < TM * TN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);               // VALU
            if (i < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        }
#pragma unroll
        for (int i = 0; i < TM * TN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);               // VALU
            if (i < 4) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);    // DS write
        }
        // Step k+2 must have landed before the next iteration dequantizes it.
        wait_vmcnt<(G2_STAGES - 3) * LOADS_PER_STEP>();
        lds_barrier();
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
static hipError_t launch_g2(const Gemm2Args &a, hipStream_t s) {
    using L = G2Layout<BM>;
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemm2_kernel<BM>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::BYTES);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((q4_gemm2_kernel<BM>), dim3(a.tiles_m * a.tiles_n), dim3(G2_THREADS),
                       L::BYTES, s, a);
    return hipGetLastError();
}

// The async-copy GEMM needs 16-byte aligned raw rows (N % 8 == 0), a 16-byte
// aligned weight base and activation rows, and at least one full 16-byte chunk.
bool gemm2_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t K, int64_t N) {
    return N % 8 == 0 && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && ldx % 8 == 0 &&
           (K / QK) * N * BLOCK_BYTES >= 16;
}

hipError_t launch_gemm2(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, hipStream_t s) {
    Gemm2Args a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.w_last_chunk = (int64_t)a.nb * N * BLOCK_BYTES - 16;
    a.tiles_n = (N + G2_BN - 1) / G2_BN;
    int bm = 256;
    if (((int64_t)(M + 255) / 256) * a.tiles_n < 192) bm = 128;
    if (const char *env = opt("MCQ4_GEMM2_BM")) bm = atoi(env) == 128 ? 128 : 256;
    a.tiles_m = (M + bm - 1) / bm;
    if (bm == 256) return launch_g2<256>(a, s);
    return launch_g2<128>(a, s);
}

}  // namespace mcq4
