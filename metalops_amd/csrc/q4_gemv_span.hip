// Single-row (M == 1) q4_0 GEMV for 4096 < N <= 12288 columns at K <= 4096:
// one workgroup per CU owning a contiguous span of 16-column groups.
//
// The M == 1 strip kernel (q4_gemv.hip) gives each workgroup tiles wg, wg + G, ...
// and copies 16-column items (288-byte pieces of each K row).  A plain read of
// that pattern is 26-36% slower than a contiguous read of the same bytes, while
// wider pieces read faster: at N = 12288, 48-column spans (864-byte pieces, one
// per workgroup on 256 CUs) read 12% faster than 16-column strips.  Here:
//
//   * Workgroup wg (XCD-renumbered, so neighbouring spans run on one XCD) owns
//     groups [wg G / grid, (wg + 1) G / grid) of the N / 16 column groups: ng = 1..3
//     groups, 16 ng columns, a row piece of 288 ng contiguous bytes per K block.
//   * Wave w owns batch w (K blocks 8w .. 8w + 7): one item of 8 row pieces,
//     copied with ceil(144 ng / 64) global_load_lds_dwordx4 (each 1 KiB of the
//     item in row-major order, so a copy reads contiguous spans of a row) into
//     the wave's LDS slot after the batch's activations.  Every wave has at most
//     one item (K <= 8 * 16 * 32 = 4096), so there is no ring; the wave waits
//     (vmcnt) only for the copies that hold the next two rows before their math,
//     so the math of the first rows overlaps the rest of the item's copies.
//   * Per 16-column group of the span: the M == 1 kernel's math -- LDS reads of
//     the 8 rows first, then four v_and_or_b32 per row into fp16 1024 + q (low
//     nibbles) and 64 + q (high nibbles in place), mfma(x', B, -S) with
//     x' = [x0, x4, x1, x5, x2, x6, x3, x7] and -S = mfma(x', -C) per K block,
//     then acc += d * that in fp32.
//   * Epilogue: the waves' partials per column summed through LDS in wave order
//     after one barrier, stored as fp16.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_common.h"

namespace mcq4 {

constexpr int GS_NW = 16;                    // waves per workgroup
constexpr int GS_B = 8;                      // K blocks per item (one batch)
constexpr int GS_NGMAX = 3;                  // 16-column groups per workgroup at most
constexpr int GS_COPIES = (144 * GS_NGMAX + 63) / 64;   // 7
constexpr int GS_SLOT = GS_COPIES * 1024;    // item bytes (6912 at ng = 3) + read overhang
constexpr int GS_NT = 2;                     // weight copies non-temporal
#ifndef GS_RP_SET
constexpr int GS_RP = 2;                     // K rows per wait
#else
constexpr int GS_RP = GS_RP_SET;
#endif

// Weight copies of an item of ng groups, and how many of them hold rows 0 .. 2h+1.
__host__ __device__ constexpr int gs_ncopy(int ng) { return (144 * ng + 63) / 64; }
__host__ __device__ constexpr int gs_need(int ng, int h) { return (288 * ng * (GS_RP * h + GS_RP) + 1023) / 1024; }

template <int N, typename F, int I = 0>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, F, I + 1>(static_cast<F &&>(f));
    }
}

struct GemvSpanArgs {
    const _Float16 *X;
    const uint8_t *W;
    _Float16 *Y;
    int nb, groups;                          // K blocks; 16-column groups of N
    uint32_t grow;                           // bytes per K row (18 N)
};

__global__ void __launch_bounds__(GS_NW * 64)
q4_gemv_span_kernel(GemvSpanArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int G = (int)gridDim.x, nb = a.nb, ngt = a.groups;
    const uint32_t grow = a.grow;
    const _Float16 *X = a.X;
    const uint8_t *W = a.W;
    _Float16 *Y = a.Y;
    asm volatile("" ::"s"(nb), "s"(ngt), "s"(grow), "s"(X), "s"(W), "s"(Y));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;

    uint8_t *xs = smem + wave * (GS_B * 64);
    uint8_t *slot = smem + GS_NW * GS_B * 64 + wave * GS_SLOT;
    float *red = (float *)(smem + GS_NW * GS_B * 64 + GS_NW * GS_SLOT);

    const int G8 = G & ~7;
    int wg = (int)blockIdx.x;
    {
        const int r = (wg & 7) * (G8 >> 3) + (wg >> 3);
        wg = wg < G8 ? r : wg;
    }
    const int g0 = (int)((int64_t)wg * ngt / G), g1 = (int)((int64_t)(wg + 1) * ngt / G);
    const int ng = g1 - g0;                                        // 1..GS_NGMAX
    const int cpr = 18 * ng;                                       // 16-byte chunks per row piece
    const int row0 = wave * GS_B;
    const int rows = max(0, min(GS_B, nb - row0));                 // 0: no item for this wave
    const uint8_t *wb = W + (int64_t)g0 * 288 + (int64_t)row0 * grow;

    if (rows > 0) {
        // Activations of the batch (lanes 0..31: row lane/4, piece lane%4; rows past
        // K clamp to the last row), then the item.
        if (lane < 4 * GS_B) {
            const int r = min(row0 + (lane >> 2), nb - 1);
            __builtin_amdgcn_global_load_lds((void *)((const uint8_t *)X + (int64_t)r * 64 + 16 * (lane & 3)),
                                             (__attribute__((address_space(3))) void *)xs, 16, 0, 0);
        }
        const int nq = GS_B * cpr;
#pragma unroll
        for (int i = 0; i < GS_COPIES; ++i) {
            const int q = lane + 64 * i;
            if (64 * i < nq) {                                     // uniform: copy i exists
                const int qq = min(q, nq - 1);
                const int r = qq / cpr, p = qq - r * cpr;
                // Rows past K re-copy row 0 (valid memory, never summed).
                const uint32_t off = (r < rows ? (uint32_t)r * grow : 0u) + 16u * (uint32_t)p;
                __builtin_amdgcn_global_load_lds((void *)(wb + off),
                                                 (__attribute__((address_space(3))) void *)(slot + 1024 * i),
                                                 16, 0, GS_NT);
            }
        }
    }

    const int qoff = c * BLOCK_BYTES + 2 + 4 * g;
    const uint32_t qal = (uint32_t)(qoff & ~3), qsh = (uint32_t)(qoff & 3) * 8;
    const uint32_t doff = (uint32_t)(c * BLOCK_BYTES);
    const uint32_t e1024 = opaque_vgpr(0x64006400u), e64 = opaque_vgpr(0x54005400u);
    const uint32_t mlo = opaque_sgpr(0x000F000Fu), mhi = opaque_sgpr(0x00F000F0u);
    const uint32_t nlo = 0xE408E408u, nhi = 0xD480D480u;          // -1032, -72 pairs
    const half8_t negc = bitcast<half8_t>(uint4_t{nlo, nhi, nlo, nhi});
    const float4_t z = {0.f, 0.f, 0.f, 0.f};

    float acc[GS_NGMAX] = {0.f, 0.f, 0.f};
    if (rows > 0) {
        // The activations (the oldest copy) first.
        switch (ng) {
            case 1: wait_vmcnt<gs_ncopy(1)>(); break;
            case 2: wait_vmcnt<gs_ncopy(2)>(); break;
            default: wait_vmcnt<gs_ncopy(3)>(); break;
        }
        half8_t xq[GS_B];
        float4_t negs[GS_B];
        const uint32_t xa = lds_addr(xs + 16 * g);
#pragma unroll
        for (int u = 0; u < GS_B; ++u) {
            const uint4_t x = bitcast<uint4_t>(*(const lds_half8 *)(lds_ptr(xa) + u * 64));
            const uint4_t v = {__builtin_amdgcn_perm(x[2], x[0], 0x05040100u),   // x0, x4
                               __builtin_amdgcn_perm(x[2], x[0], 0x07060302u),   // x1, x5
                               __builtin_amdgcn_perm(x[3], x[1], 0x05040100u),   // x2, x6
                               __builtin_amdgcn_perm(x[3], x[1], 0x07060302u)};  // x3, x7
            xq[u] = bitcast<half8_t>(v);
            negs[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[u], negc, z, 0, 0, 0);
        }
        const uint32_t base = lds_addr(slot);
        // Two K rows (all groups of the span) at a time, each pair as soon as the
        // copies holding it have landed (the copies cover the item in row-major
        // order, so rows 2h, 2h + 1 need the first ceil(288 ng (2h + 2) / 1024)).
        auto pair = [&](auto NGc, int h) {
            constexpr int NG = decltype(NGc)::value;
            constexpr uint32_t rowb = 288u * NG;
            uint32_t q0[GS_RP][NG], q1[GS_RP][NG];
            _Float16 dh[GS_RP][NG];
#pragma unroll
            for (int v = 0; v < GS_RP; ++v)
#pragma unroll
                for (int grp = 0; grp < NG; ++grp) {
                    const uint32_t ra = base + (GS_RP * h + v) * rowb + grp * 288;
                    const lds_u32 *qp = (const lds_u32 *)lds_ptr(ra + qal);
                    q0[v][grp] = qp[0];
                    q1[v][grp] = qp[1];
                    dh[v][grp] = bitcast<_Float16>(*(const lds_u16 *)lds_ptr(ra + doff));
                }
            float4_t r[GS_RP][NG];
#pragma unroll
            for (int v = 0; v < GS_RP; ++v)
#pragma unroll
                for (int grp = 0; grp < NG; ++grp) {
                    const uint32_t w = __builtin_amdgcn_alignbit(q1[v][grp], q0[v][grp], qsh);
                    const uint32_t w8 = __builtin_amdgcn_alignbit(q1[v][grp], q0[v][grp], qsh + 8);
                    const uint4_t bq = {and_or(w, mlo, e1024), and_or(w, mhi, e64), and_or(w8, mlo, e1024),
                                        and_or(w8, mhi, e64)};
                    r[v][grp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[GS_RP * h + v], bitcast<half8_t>(bq),
                                                                       negs[GS_RP * h + v], 0, 0, 0);
                }
#pragma unroll
            for (int v = 0; v < GS_RP; ++v)
                if (GS_RP * h + v < rows) {
#pragma unroll
                    for (int grp = 0; grp < NG; ++grp) acc[grp] += (float)dh[v][grp] * r[v][grp][0];
                }
        };
        auto run = [&](auto NGc) {
            constexpr int NG = decltype(NGc)::value;
            constexpr int NC = gs_ncopy(NG);
            constexpr int NH = GS_B / GS_RP;
            static_for<NH>([&](auto H) {
                constexpr int h = decltype(H)::value;
                if constexpr (h + 1 < NH) wait_vmcnt<NC - gs_need(NG, h)>();
                else wait_vmcnt<0>();
                pair(NGc, h);
            });
        };
        switch (ng) {
            case 1: run(std::integral_constant<int, 1>{}); break;
            case 2: run(std::integral_constant<int, 2>{}); break;
            default: run(std::integral_constant<int, 3>{}); break;
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int grp = 0; grp < GS_NGMAX; ++grp) red[wave * (16 * GS_NGMAX) + grp * 16 + lane] = acc[grp];
    }
    lds_barrier();
    if (tid < 16 * ng) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < GS_NW; ++w) s += red[w * (16 * GS_NGMAX) + tid];
        Y[16 * g0 + tid] = (_Float16)s;
    }
}

static size_t gemv_span_lds_bytes() {
    return (size_t)GS_NW * GS_B * 64 + (size_t)GS_NW * GS_SLOT + (size_t)GS_NW * 16 * GS_NGMAX * sizeof(float);
}

// True when the span kernel takes the whole of W: N % 16 == 0 with 256 < N/16 <=
// 768 groups (one span of 1..3 groups per workgroup on 256 workgroups), at most
// 16 batches of 8 K blocks (K <= 4096, one item per wave), aligned operands.
bool gemv_span_supported(const _Float16 *X, const uint8_t *W, int64_t K, int64_t N) {
    if (opt_is("MCQ4_GEMV_SPAN", '0')) return false;
    const int64_t groups = N / 16, nb = K / QK;
    return N % 16 == 0 && groups > 256 && groups <= 256 * GS_NGMAX && nb >= 1 && nb <= GS_NW * GS_B &&
           ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 && N * 18 * 8 < ((int64_t)1 << 31);
}

hipError_t launch_gemv_span(const _Float16 *X, const uint8_t *W, _Float16 *Y, int K, int N, hipStream_t s) {
    GemvSpanArgs a;
    a.X = X; a.W = W; a.Y = Y;
    a.nb = K / QK;
    a.groups = N / 16;
    a.grow = (uint32_t)N * BLOCK_BYTES;
    const size_t lds = gemv_span_lds_bytes();
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemv_span_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL(q4_gemv_span_kernel, dim3(256), dim3(GS_NW * 64), lds, s, a);
    return hipGetLastError();
}

}  // namespace mcq4
