// q4_0 GEMV for M == 1 and 9 <= M <= 16 rows at 4096 < N <= 16384 columns and
// K <= 4096: one workgroup per CU owning a contiguous span of 16-column groups.
//
// The strip kernels (q4_gemv.hip at M == 1, q4_gemvm.hip at M = 2..32) give each
// workgroup tiles wg, wg + G, ... and copy 16-column items (288-byte pieces of each
// K row).  A plain read of that pattern is 26-36% slower than a contiguous read of
// the same bytes, while wider pieces read faster: at N = 12288, 48-column spans
// (864-byte pieces, one per workgroup on 256 CUs) read 12% faster than 16-column
// strips.  Here:
//
//   * Workgroup wg (XCD-renumbered, so neighbouring spans run on one XCD) owns
//     groups [wg G / grid, (wg + 1) G / grid) of the N / 16 column groups: ng = 1..4
//     groups, 16 ng columns, a row piece of 288 ng contiguous bytes per K block.
//   * Wave w owns batch w (K blocks 8w .. 8w + 7): one item of 8 row pieces,
//     copied with ceil(144 ng / 64) global_load_lds_dwordx4 (each 1 KiB of the
//     item in row-major order, so a copy reads contiguous spans of a row) into
//     the wave's LDS slot.  Every wave has at most one item (K <= 8 * 16 * 32 =
//     4096), so there is no ring; the wave waits (vmcnt) only for the copies that
//     hold the next two rows before their math, so the math of the first rows
//     overlaps the rest of the item's copies.
//   * Activations, issued before the item: at M == 1 (GR = 1) the batch's row is
//     copied into LDS ahead of the item; at M >= 9 (GR = 16) lane (c, g) loads
//     activation row min(c, M - 1) straight into registers as its MFMA A row, so
//     accumulator i of the lane is output row 4g + i (four fp32 updates per K-block
//     row).  At M = 2..8 the strip kernel (q4_gemvm.hip) measured as fast or
//     faster (M = 4: 10.1 against 10.3-10.5 us at 4096 x 14336), so it keeps them.
//   * Per 16-column group of the span: LDS reads of two rows first, then four
//     v_and_or_b32 per row into fp16 1024 + q (low nibbles) and 64 + q (high
//     nibbles in place), mfma(x', B, -S) with x' = [x0, x4, x1, x5, x2, x6, x3, x7]
//     and -S = mfma(x', -C) per K block, then acc += d * that in fp32.
//   * Epilogue: each wave's partials per output row and column go to its own
//     (drained) LDS slot; after one barrier they are summed in wave order and
//     stored as fp16.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_common.h"

namespace mcq4 {

constexpr int GS_GRID = 256;                 // workgroups: one per CU
constexpr int GS_NW = 16;                    // waves per workgroup
constexpr int GS_B = 8;                      // K blocks per item (one batch)
constexpr int GS_NGMAX = 4;                  // 16-column groups per workgroup at most
constexpr int GS_COPIES = (144 * GS_NGMAX + 63) / 64;   // 9
constexpr int GS_SLOT = GS_COPIES * 1024;    // item bytes (9216 at ng = 4)
constexpr int GS_XS = GS_NW * GS_B * 64;     // M == 1 activation area
constexpr int GS_PAD = 64;                   // read overhang of the last slot
constexpr int GS_NT = 2;                     // weight copies non-temporal
#ifndef GS_RP_SET
constexpr int GS_RP = 2;                     // K rows per wait
#else
constexpr int GS_RP = GS_RP_SET;
#endif
static_assert(16 * 64 * 4 <= GS_SLOT, "a wave's partials fit its slot");

// Weight copies of an item of ng groups, and how many of them hold rows 0 .. RP(h+1)-1.
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
    int64_t ldx, ldy;                        // row strides of X and Y (elements)
    int M, nb, groups;                       // rows; K blocks; 16-column groups of N
    uint32_t grow;                           // bytes per K row (18 N)
};

template <int GR>
__global__ void __launch_bounds__(GS_NW * 64)
q4_gemv_span_kernel(GemvSpanArgs a) {
    static_assert(GR == 1 || GR == 16, "row groups");
    constexpr int NA = GR == 1 ? 1 : 4;          // accumulators per group
    constexpr bool HOIST = GR == 1;              // -S for all 8 rows up front (else per row pair)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = a.nb, ngt = a.groups, M = a.M;
    const uint32_t grow = a.grow;
    const _Float16 *X = a.X;
    const uint8_t *W = a.W;
    _Float16 *Y = a.Y;
    const int64_t ldx = a.ldx, ldy = a.ldy;
    asm volatile("" ::"s"(nb), "s"(ngt), "s"(M), "s"(grow), "s"(X), "s"(W), "s"(Y), "s"(ldx), "s"(ldy));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;

    constexpr int XS = GR == 1 ? GS_XS : 0;
    uint8_t *xs = smem + wave * (GS_B * 64);
    uint8_t *slot = smem + XS + wave * GS_SLOT;

    // XCD renumbering of the GS_GRID workgroups; span bounds by a shift (the grid
    // is fixed, groups <= 1024, so wg * groups fits 32 bits).
    const int wg = ((int)blockIdx.x & 7) * (GS_GRID / 8) + ((int)blockIdx.x >> 3);
    const int g0 = (wg * ngt) >> 8, g1 = ((wg + 1) * ngt) >> 8;
    static_assert(GS_GRID == 256, "span bounds by a shift of 8");
    const int ng = g1 - g0;                                        // 1..GS_NGMAX
    const int row0 = wave * GS_B;
    const int rows = max(0, min(GS_B, nb - row0));                 // 0: no item for this wave
    const uint8_t *wb = W + (int64_t)g0 * 288 + (int64_t)row0 * grow;

    const int qoff = c * BLOCK_BYTES + 2 + 4 * g;
    const uint32_t qal = (uint32_t)(qoff & ~3), qsh = (uint32_t)(qoff & 3) * 8;
    const uint32_t doff = (uint32_t)(c * BLOCK_BYTES);
    const uint32_t e1024 = opaque_vgpr(0x64006400u), e64 = opaque_vgpr(0x54005400u);
    const uint32_t mlo = opaque_sgpr(0x000F000Fu), mhi = opaque_sgpr(0x00F000F0u);
    const uint32_t nlo = 0xE408E408u, nhi = 0xD480D480u;          // -1032, -72 pairs
    const half8_t negc = bitcast<half8_t>(uint4_t{nlo, nhi, nlo, nhi});
    const float4_t z = {0.f, 0.f, 0.f, 0.f};

    float acc[GS_NGMAX][NA];
#pragma unroll
    for (int grp = 0; grp < GS_NGMAX; ++grp)
#pragma unroll
        for (int i = 0; i < NA; ++i) acc[grp][i] = 0.f;
    // One templated body per span width ng (the copy addresses divide by the
    // constant 18 ng, and the waits count its copies).
    auto item = [&](auto NGc) {
        constexpr int NG = decltype(NGc)::value;
        constexpr int NC = gs_ncopy(NG);
        constexpr int CPR = 18 * NG;                               // 16-byte chunks per row piece
        uint4_t xr[GR == 1 ? 1 : GS_B];
        if constexpr (GR == 1) {
            // The batch's activations (lanes 0..31: K block lane/4, piece lane%4;
            // blocks past K clamp to the last one), then the item.
            if (lane < 4 * GS_B) {
                const int r = min(row0 + (lane >> 2), nb - 1);
                __builtin_amdgcn_global_load_lds((void *)((const uint8_t *)X + (int64_t)r * 64 + 16 * (lane & 3)),
                                                 (__attribute__((address_space(3))) void *)xs, 16, 0, 0);
            }
        } else {
            // Lane (c, g): activation row min(c, M - 1), elements 8g..8g+7 of each K
            // block of the batch (blocks past K clamp to the last one).
            const uint8_t *xrow = (const uint8_t *)X + (int64_t)min(c, M - 1) * ldx * 2 + 16 * g;
#pragma unroll
            for (int u = 0; u < GS_B; ++u) xr[u] = *(const uint4_t *)(xrow + (int64_t)min(row0 + u, nb - 1) * 64);
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int qq = min(lane + 64 * i, GS_B * CPR - 1);
            const int r = qq / CPR, p = qq - r * CPR;
            // Rows past K re-copy row 0 (valid memory, never summed).
            const uint32_t off = (r < rows ? __umul24((uint32_t)r, grow) : 0u) + 16u * (uint32_t)p;
            __builtin_amdgcn_global_load_lds((void *)(wb + off),
                                             (__attribute__((address_space(3))) void *)(slot + 1024 * i), 16, 0,
                                             GS_NT);
        }
        // The activations (the oldest loads) first.
        wait_vmcnt<NC>();
        half8_t xq[GS_B];
        float4_t negs[HOIST ? GS_B : 1];
        const uint32_t xa = lds_addr(xs + 16 * g);
#pragma unroll
        for (int u = 0; u < GS_B; ++u) {
            uint4_t x;
            if constexpr (GR == 1) x = bitcast<uint4_t>(*(const lds_half8 *)(lds_ptr(xa) + u * 64));
            else x = xr[u];
            const uint4_t v = {__builtin_amdgcn_perm(x[2], x[0], 0x05040100u),   // x0, x4
                               __builtin_amdgcn_perm(x[2], x[0], 0x07060302u),   // x1, x5
                               __builtin_amdgcn_perm(x[3], x[1], 0x05040100u),   // x2, x6
                               __builtin_amdgcn_perm(x[3], x[1], 0x07060302u)};  // x3, x7
            xq[u] = bitcast<half8_t>(v);
            if constexpr (HOIST) negs[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[u], negc, z, 0, 0, 0);
        }
        const uint32_t base = lds_addr(slot);
        // GS_RP K rows (all groups of the span) at a time, each set as soon as the
        // copies holding it have landed (the copies cover the item in row-major
        // order, so rows up to RP (h + 1) - 1 need the first gs_need(ng, h)).
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
            float4_t ns[GS_RP];
#pragma unroll
            for (int v = 0; v < GS_RP; ++v) {
                if constexpr (HOIST) ns[v] = negs[GS_RP * h + v];
                else ns[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[GS_RP * h + v], negc, z, 0, 0, 0);
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
                                                                       ns[v], 0, 0, 0);
                }
#pragma unroll
            for (int v = 0; v < GS_RP; ++v)
                if (GS_RP * h + v < rows) {
#pragma unroll
                    for (int grp = 0; grp < NG; ++grp)
#pragma unroll
                        for (int i = 0; i < NA; ++i)
                            acc[grp][i] += (float)dh[v][grp] * r[v][grp][i];
                }
        };
        constexpr int NH = GS_B / GS_RP;
        static_for<NH>([&](auto H) {
            constexpr int h = decltype(H)::value;
            if constexpr (h + 1 < NH) wait_vmcnt<NC - gs_need(NG, h)>();
            else wait_vmcnt<0>();
            pair(NGc, h);
        });
    };
    if (rows > 0) {
        switch (ng) {
            case 1: item(std::integral_constant<int, 1>{}); break;
            case 2: item(std::integral_constant<int, 2>{}); break;
            case 3: item(std::integral_constant<int, 3>{}); break;
            default: item(std::integral_constant<int, GS_NGMAX>{}); break;
        }
        // Every LDS read of the slot has returned before it holds the partials.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // Partials into this wave's slot: [output row][64 columns] floats.  Accumulator
    // i of lane (c, g) is output row 4g + i (row 0 for every lane at M == 1).
    float *mine = (float *)slot;
    if (GR > 1 || lane < 16) {
#pragma unroll
        for (int i = 0; i < NA; ++i)
#pragma unroll
            for (int grp = 0; grp < GS_NGMAX; ++grp)
                mine[(GR == 1 ? 0 : 4 * g + i) * 64 + grp * 16 + c] = acc[grp][i];
    }
    lds_barrier();
    // Thread (row, col) = (tid / 64, tid % 64): 16 rows x 64 columns = the workgroup.
    const int row = tid >> 6, col = tid & 63;
    if (col < 16 * ng && row < (GR == 1 ? 1 : M)) {
        const float *p = (const float *)(smem + XS) + row * 64 + col;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < GS_NW; ++w) s += p[w * (GS_SLOT / 4)];
        Y[(int64_t)row * ldy + 16 * g0 + col] = (_Float16)s;
    }
}

// True when the span kernel takes the whole of W for M rows: M == 1 or 9 <= M <= 16,
// N % 16 == 0 with 256 < N/16 <= 1024 groups (one span of 1..4 groups per
// workgroup on 256 workgroups), at most 16 batches of 8 K blocks (K <= 4096, one
// item per wave), 16-byte aligned weights and activation rows.
bool gemv_span_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N) {
    if (opt_is("MCQ4_GEMV_SPAN", '0')) return false;
    const int64_t groups = N / 16, nb = K / QK;
    return (M == 1 || (M >= 9 && M <= 16)) && N % 16 == 0 && groups > GS_GRID && groups <= GS_GRID * GS_NGMAX && nb >= 1 &&
           nb <= GS_NW * GS_B && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 &&
           (M == 1 || ldx % 8 == 0) && N * 18 * 8 < ((int64_t)1 << 31);
}

template <int GR>
static hipError_t launch_span_gr(const GemvSpanArgs &a, hipStream_t s) {
    const size_t lds = (GR == 1 ? GS_XS : 0) + (size_t)GS_NW * GS_SLOT + GS_PAD;
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemv_span_kernel<GR>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL(q4_gemv_span_kernel<GR>, dim3(GS_GRID), dim3(GS_NW * 64), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_gemv_span(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y, int64_t ldy, int M,
                            int K, int N, hipStream_t s) {
    GemvSpanArgs a;
    a.X = X; a.W = W; a.Y = Y;
    a.ldx = ldx; a.ldy = ldy;
    a.M = M;
    a.nb = K / QK;
    a.groups = N / 16;
    a.grow = (uint32_t)N * BLOCK_BYTES;
    return M == 1 ? launch_span_gr<1>(a, s) : launch_span_gr<16>(a, s);
}

}  // namespace mcq4
