// Prefill-shaped q4_0 matmul (M > 64) on gfx950: MFMA-bound GEMM.
//
//   * WG = 256 threads = 4 waves in a 2x2 grid; WG tile BM x BN; wave tile
//     (BM/2) x (BN/2) built from v_mfma_f32_32x32x16_f16 tiles (fp32 accumulate).
//   * K advances one q4_0 block (32) per stage.  Per stage each thread owning a
//     column loads that column's 18-byte block, dequantizes it to fp16
//     (q-8)*d -- the reference's fp16 dequant value -- and writes the 32 weights
//     as one LDS row of the transposed B tile; the activation tile is copied to
//     LDS 16 bytes per load.  LDS rows are padded to 40 halves (80 bytes) so the
//     16-byte operand reads of 8 consecutive rows hit disjoint banks.
//   * Two LDS stages: global loads for stage s+1 are issued before the MFMAs of
//     stage s and stored after them; one barrier per stage.
//   * Workgroup ids are remapped so that consecutive tiles land on the same XCD
//     (WGs are dispatched round-robin over the 8 XCDs), grouping tiles that
//     share activation rows in one XCD's L2.
//   * Optional split-K (grid.z) with fp32 partials reduced in a fixed order by
//     the last-arriving WG of each output tile.
//
// MFMA 32x32 output layout: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
#include "q4_common.h"

namespace mcq4 {

constexpr int GEMM_THREADS = 256;
constexpr int LDS_ROW = 40;  // halves per LDS row (32 + 8 padding)

struct GemmArgs {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int tiles_m, tiles_n;
    int S;
    float *partials;     // [tiles][S][BM*BN] when S > 1
    uint32_t *counters;  // [tiles]
};

// Natural-order dequant of 8 nibbles: returns fp16 weights e0..e7 as 4 dwords.
__device__ __forceinline__ uint4_t dequant8_natural(uint32_t w, uint32_t dbits) {
    const half8_t p = dequant8_perm(w, dbits);  // [e0,e2,e4,e6,e1,e3,e5,e7]
    const uint4_t u = bitcast<uint4_t>(p);
    uint4_t r;
    r[0] = __builtin_amdgcn_perm(u[2], u[0], 0x05040100u);  // e0, e1
    r[1] = __builtin_amdgcn_perm(u[2], u[0], 0x07060302u);  // e2, e3
    r[2] = __builtin_amdgcn_perm(u[3], u[1], 0x05040100u);  // e4, e5
    r[3] = __builtin_amdgcn_perm(u[3], u[1], 0x07060302u);  // e6, e7
    return r;
}

template <int BM, int BN>
__global__ void __launch_bounds__(GEMM_THREADS, 1)
q4_gemm_kernel(GemmArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int A_CHUNKS = BM * 4 / GEMM_THREADS;  // 16-byte chunks per thread
    static_assert(BN <= GEMM_THREADS, "one B column per thread");
    static_assert(A_CHUNKS >= 1, "tile too small");

    __shared__ __attribute__((aligned(16))) _Float16 lds_a[2][BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 lds_b[2][BN * LDS_ROW];
    __shared__ uint32_t last_flag;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware tile mapping: hardware sends WG i to XCD i % 8.  Give each XCD a
    // contiguous range of tile ids, walked M-fastest inside column strips.
    const int ntiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x;
    int tile_id = bid;
    if (ntiles % 8 == 0) tile_id = (bid % 8) * (ntiles / 8) + bid / 8;
    const int tm = tile_id % a.tiles_m;
    const int tn = tile_id / a.tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    // Split-K range.
    const int per = (a.nb + a.S - 1) / a.S;
    const int kb_beg = blockIdx.z * per;
    const int kb_end = min(a.nb, kb_beg + per);

    // ---- per-thread global load assignments --------------------------------
    // A: chunk c covers row c/4, halves 8*(c%4) .. +8 of the 32-wide K slice.
    const _Float16 *a_src[A_CHUNKS];
    bool a_ok[A_CHUNKS];
    int a_lds[A_CHUNKS];
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
        const int c = tid + i * GEMM_THREADS;
        const int r = c >> 2, q = c & 3;
        const int m = m0 + r;
        a_ok[i] = m < a.M;
        a_src[i] = a.X + (int64_t)(a_ok[i] ? m : 0) * a.ldx + 8 * q;
        a_lds[i] = r * LDS_ROW + 8 * q;
    }
    // B: thread tid < BN owns column n0 + tid.
    const bool b_own = tid < BN;
    const int bn = n0 + tid;
    const bool b_ok = b_own && bn < a.N;
    const int64_t row_bytes = (int64_t)a.N * BLOCK_BYTES;
    const uint8_t *b_src = a.W + (int64_t)(b_ok ? bn : 0) * BLOCK_BYTES;

    uint4_t ra[A_CHUNKS];
    uint16_t rb[9];

    auto load_stage = [&](int kb) {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i)
            ra[i] = a_ok[i] ? *(const uint4_t *)(a_src[i] + (int64_t)kb * QK)
                            : uint4_t{0u, 0u, 0u, 0u};
        if (b_own) {
            const uint16_t *p = (const uint16_t *)(b_src + (int64_t)kb * row_bytes);
#pragma unroll
            for (int j = 0; j < 9; ++j) rb[j] = b_ok ? p[j] : (uint16_t)0;
        }
    };
    auto store_stage = [&](int st) {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) *(uint4_t *)(&lds_a[st][a_lds[i]]) = ra[i];
        if (b_own) {
            _Float16 *dst = &lds_b[st][tid * LDS_ROW];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t w = (uint32_t)rb[1 + 2 * h] | ((uint32_t)rb[2 + 2 * h] << 16);
                *(uint4_t *)(dst + 8 * h) = dequant8_natural(w, rb[0]);
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

    // Operand read offsets (halves) inside a stage.
    const int lrow = lane & 31, lk = 8 * (lane >> 5);
    const int a_rd = (wm * WM + lrow) * LDS_ROW + lk;
    const int b_rd = (wn * WN + lrow) * LDS_ROW + lk;

    if (kb_beg < kb_end) {
        load_stage(kb_beg);
        store_stage(0);
    }
    __syncthreads();
    int st = 0;
    for (int kb = kb_beg; kb < kb_end; ++kb) {
        const bool more = kb + 1 < kb_end;
        if (more) load_stage(kb + 1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            half8_t av[TM], bv[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                av[i] = *(const half8_t *)(&lds_a[st][a_rd + i * 32 * LDS_ROW + 16 * ks]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bv[j] = *(const half8_t *)(&lds_b[st][b_rd + j * 32 * LDS_ROW + 16 * ks]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j],
                                                                        0, 0, 0);
        }
        if (more) store_stage(st ^ 1);
        __syncthreads();
        st ^= 1;
    }

    // ---- epilogue ------------------------------------------------------------
    const int col_l = lane & 31, rsub = 4 * (lane >> 5);
    if (a.S == 1) {
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
        return;
    }
    // Split-K: write this WG's partial tile (dense BM x BN, row-major), then the
    // last WG to arrive sums all S partials in order and writes fp16.
    float *part = a.partials + ((int64_t)tile_id * a.S + blockIdx.z) * (BM * BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nl = wn * WN + j * 32 + col_l;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = wm * WM + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
                part[ml * BN + nl] = acc[i][j][r];
            }
        }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.counters[tile_id], 1u);
        last_flag = (prev == (uint32_t)(a.S - 1)) ? 1u : 0u;
        if (last_flag) __hip_atomic_store(&a.counters[tile_id], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    const float *base = a.partials + (int64_t)tile_id * a.S * (BM * BN);
    for (int v = tid; v < BM * BN; v += GEMM_THREADS) {
        float s = 0.f;
        for (int sp = 0; sp < a.S; ++sp)
            s += __hip_atomic_load(base + (int64_t)sp * (BM * BN) + v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        const int m = m0 + v / BN, n = n0 + v % BN;
        if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)s;
    }
}

// ---- configuration ----------------------------------------------------------

struct GemmCfg {
    int BM, BN, S;
};

static GemmCfg gemm_config(int64_t M, int64_t K, int64_t N) {
    GemmCfg c{256, 256, 1};
    const int64_t nb = K / QK;
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if (tiles(256, 256) < 192) {
        c.BN = 128;
        if (tiles(256, 128) < 192) c.BM = 128;
    }
    const int64_t t = tiles(c.BM, c.BN);
    int64_t S = 1;
    while (t * S < 192 && nb / (S * 2) >= 32) S *= 2;
    c.S = (int)S;
    if (((M + c.BM - 1) / c.BM) * ((N + c.BN - 1) / c.BN) > COUNTER_SLOTS) c.S = 1;
    return c;
}

size_t gemm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const GemmCfg c = gemm_config(M, K, N);
    if (c.S == 1) return 0;
    const int64_t t = ((M + c.BM - 1) / c.BM) * ((N + c.BN - 1) / c.BN);
    return COUNTER_BYTES + (size_t)t * c.S * c.BM * c.BN * sizeof(float);
}

template <int BM, int BN>
static hipError_t launch_g(GemmArgs a, hipStream_t s) {
    dim3 grid(a.tiles_m * a.tiles_n, 1, a.S), block(GEMM_THREADS);
    hipLaunchKernelGGL((q4_gemm_kernel<BM, BN>), grid, block, 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                       int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    const GemmCfg c = gemm_config(M, K, N);
    GemmArgs a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.tiles_m = (M + c.BM - 1) / c.BM;
    a.tiles_n = (N + c.BN - 1) / c.BN;
    a.S = c.S;
    a.partials = nullptr; a.counters = nullptr;
    if (c.S > 1) {
        a.counters = (uint32_t *)ws;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    if (c.BM == 256 && c.BN == 256) return launch_g<256, 256>(a, s);
    if (c.BM == 256) return launch_g<256, 128>(a, s);
    if (c.BN == 256) return launch_g<128, 256>(a, s);
    return launch_g<128, 128>(a, s);
}

}  // namespace mcq4
