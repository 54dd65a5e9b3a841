// Decode-shaped q4_0 matmul (M <= 64) on gfx950: HBM-bound weight streaming
// feeding v_mfma_f32_16x16x32_f16.
//
// Work decomposition
//   * One MFMA 16x16x32 consumes exactly one q4_0 block per output column: the
//     32 weights of block (kb, n) form the K=32 slice of the B operand.
//   * A wave owns NT column tiles of 16 columns and MT row tiles of 16 rows, and
//     a contiguous range of K blocks.  The WG's WAVES waves split the WG's block
//     range; WGs along grid.y split K further (split-K = S).
//   * Lane l (column c = l%16, k-group g = l/16) reads, per block and column
//     tile, the fp16 scale and qs bytes 4g..4g+3 (elements 8g..8g+7) with 2-byte
//     loads (blocks are only 2-byte aligned); across the wave that is one
//     contiguous 288-byte run per column tile.  dequant8_perm turns them into
//     fp16 (q-8)*d in registers; the activations are loaded 16 bytes per lane
//     and permuted to the same slot order.
//   * Reduction over waves goes through LDS; across split-K WGs through fp32
//     partials in the workspace, summed in a fixed order by the last-arriving WG
//     of each column tile (per-tile arrival counter, reset to zero by that WG).
//
// MFMA 16x16 output layout: lane l holds D[4*(l/16) + i][l%16], i = 0..3.
#include "q4_common.h"

#ifndef MCQ4_SKINNY_LOADS
#define MCQ4_SKINNY_LOADS 0
#endif

namespace mcq4 {

struct SkinnyArgs {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int n_begin;        // first output column handled (columns before it are skipped)
    int S;              // split-K factor (grid.y)
    float *partials;    // [tiles][S][MT*NT*256] when S > 1
    uint32_t *counters; // [tiles] when S > 1
};

template <int MT, int NT, int WAVES, int U>
__global__ void __launch_bounds__(WAVES * 64)
q4_skinny_kernel(SkinnyArgs a) {
    constexpr int NFRAG = MT * NT;
    __shared__ float red[WAVES][256];
    __shared__ uint32_t last_flag;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int tile = blockIdx.x;
    const int n0 = a.n_begin + tile * (16 * NT);

    // K-block range of this wave.
    const int per_wg = (a.nb + a.S - 1) / a.S;
    const int wg_beg = blockIdx.y * per_wg;
    const int wg_end = min(a.nb, wg_beg + per_wg);
    const int per_wave = (max(0, wg_end - wg_beg) + WAVES - 1) / WAVES;
    const int kbeg = min(wg_end, wg_beg + wave * per_wave);
    const int kend = min(wg_end, kbeg + per_wave);

    // Per-lane byte offsets within one K-block row of W (row = 18*N bytes).
    int boff[NT];
    bool bvalid[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int n = n0 + t * 16 + c;
        bvalid[t] = n < a.N;
        boff[t] = (bvalid[t] ? n : 0) * BLOCK_BYTES;
    }
    // Per-lane activation row pointers (nullptr rows contribute zero).
    const _Float16 *xrow[MT];
    bool xvalid[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + c;
        xvalid[mt] = m < a.M;
        xrow[mt] = a.X + (int64_t)(xvalid[mt] ? m : 0) * a.ldx + 8 * g;
    }

    float4_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int64_t row_bytes = (int64_t)a.N * BLOCK_BYTES;

    auto step = [&](int kb_first, int count) {
        // Issue every load of `count` blocks first, then compute.
        uint16_t dq[U][NT], q0[U][NT], q1[U][NT];
        uint4_t xv[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u < count) {
                const uint8_t *rb = a.W + (int64_t)(kb_first + u) * row_bytes;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint16_t *p = (const uint16_t *)(rb + boff[t]);
#if MCQ4_SKINNY_LOADS == 1
                    dq[u][t] = __builtin_nontemporal_load(p);
                    q0[u][t] = __builtin_nontemporal_load(p + 1 + 2 * g);
                    q1[u][t] = __builtin_nontemporal_load(p + 2 + 2 * g);
#elif MCQ4_SKINNY_LOADS == 2
                    dq[u][t] = p[0];
                    const uintptr_t o = (uintptr_t)(p + 1 + 2 * g);
                    const uint32_t *pa = (const uint32_t *)(o & ~(uintptr_t)3);
                    const uint32_t sh = (uint32_t)(o & 3) * 8;
                    const uint32_t lo = pa[0];
                    const uint32_t hi = pa[sh ? 1 : 0];
                    const uint32_t w = __builtin_amdgcn_alignbit(hi, lo, sh);
                    q0[u][t] = (uint16_t)w;
                    q1[u][t] = (uint16_t)(w >> 16);
#else
                    dq[u][t] = p[0];
                    q0[u][t] = p[1 + 2 * g];
                    q1[u][t] = p[2 + 2 * g];
#endif
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    if (xvalid[mt])
                        xv[u][mt] = *(const uint4_t *)(xrow[mt] + (int64_t)(kb_first + u) * QK);
                    else
                        xv[u][mt] = uint4_t{0u, 0u, 0u, 0u};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u < count) {
                half8_t av[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) av[mt] = perm_act8(xv[u][mt]);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint32_t w = (uint32_t)q0[u][t] | ((uint32_t)q1[u][t] << 16);
                    half8_t bv = dequant8_perm(w, dq[u][t]);
                    if (!bvalid[t]) bv = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[mt], bv, acc[mt][t],
                                                                            0, 0, 0);
                }
            }
        }
    };

    int kb = kbeg;
    for (; kb + U <= kend; kb += U) step(kb, U);
    if (kb < kend) step(kb, kend - kb);

    // ---- reduce over the WG's waves, one 16x16 fragment at a time ----------
    const int tid = threadIdx.x;
    float *part = nullptr;
    if (a.S > 1)
        part = a.partials + ((int64_t)tile * a.S + blockIdx.y) * (NFRAG * 256);
#pragma unroll
    for (int f = 0; f < NFRAG; ++f) {
        const int mt = f / NT, t = f % NT;
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][lane * 4 + i] = acc[mt][t][i];
        __syncthreads();
        for (int v = tid; v < 256; v += WAVES * 64) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) s += red[w][v];
            const int l = v >> 2, i = v & 3;
            const int m = mt * 16 + 4 * (l >> 4) + i;
            const int n = n0 + t * 16 + (l & 15);
            if (a.S == 1) {
                if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)s;
            } else {
                part[f * 256 + v] = s;
            }
        }
        __syncthreads();
    }
    // Without counters the partials are summed by q4_skinny_reduce_kernel (the
    // kernel boundary orders it after this one).
    if (a.S == 1 || !a.counters) return;

    // ---- split-K: the last WG to arrive for this tile sums the partials ----
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.counters[tile], 1u);
        last_flag = (prev == (uint32_t)(a.S - 1)) ? 1u : 0u;
        if (last_flag) __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    const float *base = a.partials + (int64_t)tile * a.S * (NFRAG * 256);
    for (int v = tid; v < NFRAG * 256; v += WAVES * 64) {
        float s = 0.f;
        for (int sp = 0; sp < a.S; ++sp)
            s += __hip_atomic_load(base + (int64_t)sp * (NFRAG * 256) + v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        const int f = v >> 8, r = v & 255;
        const int mt = f / NT, t = f % NT;
        const int l = r >> 2, i = r & 3;
        const int m = mt * 16 + 4 * (l >> 4) + i;
        const int n = n0 + t * 16 + (l & 15);
        if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (_Float16)s;
    }
}

// Sums the S fp32 partials of the tiles from n_begin on in split order (the
// fragment layout above: lane l of fragment (mt, t) holds rows 4 (l / 16) + i,
// column l % 16) and stores fp16.
__global__ void __launch_bounds__(256) q4_skinny_reduce_kernel(SkinnyArgs a, int MT, int NT) {
    const int ncols = a.N - a.n_begin;
    const int64_t v0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (v0 >= (int64_t)a.M * ncols) return;
    const int m = (int)(v0 / ncols), nn = (int)(v0 % ncols);
    const int tile = nn / (16 * NT), tn = nn % (16 * NT);
    const int f = (m / 16) * NT + tn / 16;
    const int v = (((m % 16) / 4) * 16 + tn % 16) * 4 + m % 4;
    const int nfrag = MT * NT;
    const float *p = a.partials + (int64_t)tile * a.S * (nfrag * 256) + f * 256 + v;
    float s = 0.f;
    for (int sp = 0; sp < a.S; ++sp) s += p[(int64_t)sp * nfrag * 256];
    a.Y[(int64_t)m * a.ldy + a.n_begin + nn] = (_Float16)s;
}

// ---- launch configuration ---------------------------------------------------

struct SkinnyCfg {
    int NT, WAVES, S, U;
};

template <int MT, int NT, int WAVES, int U>
static hipError_t launch_t(const SkinnyArgs &a, int tiles, hipStream_t s) {
    dim3 grid(tiles, a.S), block(WAVES * 64);
    hipLaunchKernelGGL((q4_skinny_kernel<MT, NT, WAVES, U>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int MT, int NT, int WAVES>
static hipError_t launch_w(const SkinnyArgs &a, const SkinnyCfg &c, int tiles, hipStream_t s) {
    if (c.U == 4) return launch_t<MT, NT, WAVES, 4>(a, tiles, s);
    if (c.U == 8) return launch_t<MT, NT, WAVES, 8>(a, tiles, s);
    return launch_t<MT, NT, WAVES, 16>(a, tiles, s);
}

template <int MT, int NT>
static hipError_t launch_nt(const SkinnyArgs &a, const SkinnyCfg &c, int tiles, hipStream_t s) {
    if (c.WAVES == 4) return launch_w<MT, NT, 4>(a, c, tiles, s);
    if (c.WAVES == 8) return launch_w<MT, NT, 8>(a, c, tiles, s);
    return launch_w<MT, NT, 16>(a, c, tiles, s);
}

template <int MT>
static hipError_t launch_mt(const SkinnyArgs &a, const SkinnyCfg &c, int tiles, hipStream_t s) {
    if (c.NT == 1) return launch_nt<MT, 1>(a, c, tiles, s);
    if (c.NT == 2) return launch_nt<MT, 2>(a, c, tiles, s);
    return launch_nt<MT, 4>(a, c, tiles, s);
}

// Default: no cross-workgroup split-K.  Publishing partials across
// workgroups needs device-scope release/acquire fences, which on this
// multi-XCD part write back / invalidate the whole L2 of each XCD and cost
// ~100 us per launch; K is split across the waves of one workgroup instead.
SkinnyCfg skinny_config(int64_t M, int64_t K, int64_t N) {
    SkinnyCfg c;
    const int64_t nb = K / QK;
    c.NT = (N >= 8192) ? 2 : 1;
    c.WAVES = nb >= 256 ? 16 : 8;
    c.S = 1;
    c.U = 8;
    if ((N + 16 * c.NT - 1) / (16 * c.NT) > COUNTER_SLOTS) c.S = 1;
    (void)M;
    return c;
}

size_t gemvm_workspace_bytes(int64_t M, int64_t K, int64_t N);

// Tail split: the columns past the last whole 16-column tile, which the other
// decode kernels leave to this one (N % 16 != 0), are one or two tiles; walking
// all of K in one workgroup took 8-22 us there (M = 1 11008 x 4104: 22.5 us
// against ~7 for 4096 columns), so their K is split over up to 32 workgroups
// whose fp32 partials a second kernel sums.
constexpr int SK_TAIL_SMAX = 32;
static int skinny_tail_splits(int64_t K) {
    const int64_t nb = K / QK;
    return nb >= 64 ? (int)std::min<int64_t>(SK_TAIL_SMAX, nb / 16) : 1;
}

// The larger of this kernel's split-K needs and the small-batch GEMV's.
size_t skinny_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    const SkinnyCfg c = skinny_config(M, K, N);
    size_t need = 0;
    if (N % 16 && skinny_tail_splits(K) > 1)
        need = COUNTER_BYTES + (size_t)2 * skinny_tail_splits(K) * ((M + 15) / 16) * c.NT * 256 * sizeof(float);
    if (c.S > 1) {
        const int MT = (int)((M + 15) / 16);
        const int64_t tiles = (N + 16 * c.NT - 1) / (16 * c.NT);
        need = COUNTER_BYTES + (size_t)tiles * c.S * MT * c.NT * 256 * sizeof(float);
    }
    return std::max(need, gemvm_workspace_bytes(M, K, N));
}

bool decode_lds_supported(const uint8_t *W, int64_t N, int64_t ldx);
hipError_t launch_decode_lds(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                             int64_t ldy, int M, int K, int N, int *n_done, hipStream_t s);

bool gemv_dma_supported(const _Float16 *X, const uint8_t *W, int64_t K, int64_t N);
hipError_t launch_gemv_dma(const _Float16 *X, const uint8_t *W, _Float16 *Y, int K, int N,
                           int *n_done, hipStream_t s);

bool gemvm_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K,
                     int64_t N);
hipError_t launch_gemvm(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                        int64_t ldy, int M, int K, int N, void *ws, int *n_done, hipStream_t s);

static bool use_decode_lds(const uint8_t *W, int64_t N, int64_t ldx) {
    if (opt_is("MCQ4_DECODE_PATH", 'd')) return false;   // "direct" forces this file's kernel
    return decode_lds_supported(W, N, ldx);
}

hipError_t launch_skinny(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                         int64_t ldy, int M, int K, int N, void *ws, hipStream_t s) {
    int n_begin = 0;
    if (use_decode_lds(W, N, ldx) && skinny_config(M, K, N).S == 1) {
        hipError_t e;
        if (M == 1 && gemv_dma_supported(X, W, K, N))
            e = launch_gemv_dma(X, W, Y, K, N, &n_begin, s);
        else if (gemvm_supported(X, ldx, W, M, K, N))
            e = launch_gemvm(X, ldx, W, Y, ldy, M, K, N, ws, &n_begin, s);
        else
            e = launch_decode_lds(X, ldx, W, Y, ldy, M, K, N, &n_begin, s);
        if (e != hipSuccess || n_begin == N) return e;
    }
    SkinnyCfg c = skinny_config(M, K, N);
    const int MT = (M + 15) / 16;
    const int64_t tiles = (N - n_begin + 16 * c.NT - 1) / (16 * c.NT);
    SkinnyArgs a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N; a.S = c.S;
    a.n_begin = n_begin;
    a.partials = nullptr; a.counters = nullptr;
    if (c.S > 1) {
        a.counters = (uint32_t *)ws;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
    }
    const bool tail = n_begin > 0 && tiles <= 2 && ws && skinny_tail_splits(K) > 1;
    if (tail) {
        c.S = a.S = skinny_tail_splits(K);
        c.WAVES = 8;
        a.counters = nullptr;
        a.partials = (float *)((char *)ws + COUNTER_BYTES);
        hipError_t e;
        switch (MT) {
            case 1: e = launch_mt<1>(a, c, (int)tiles, s); break;
            case 2: e = launch_mt<2>(a, c, (int)tiles, s); break;
            case 3: e = launch_mt<3>(a, c, (int)tiles, s); break;
            default: e = launch_mt<4>(a, c, (int)tiles, s); break;
        }
        if (e != hipSuccess) return e;
        const int64_t nout = (int64_t)M * (N - n_begin);
        hipLaunchKernelGGL(q4_skinny_reduce_kernel, dim3((unsigned)((nout + 255) / 256)), dim3(256), 0, s, a,
                           MT > 4 ? 4 : MT, c.NT);
        return hipGetLastError();
    }
    switch (MT) {
        case 1: return launch_mt<1>(a, c, (int)tiles, s);
        case 2: return launch_mt<2>(a, c, (int)tiles, s);
        case 3: return launch_mt<3>(a, c, (int)tiles, s);
        default: return launch_mt<4>(a, c, (int)tiles, s);
    }
}

}  // namespace mcq4
