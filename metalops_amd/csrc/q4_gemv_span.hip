// q4_0 GEMV for 1 <= M <= 16 rows at 4096 < N <= 16384 columns and K <= 4096:
// one workgroup per CU owning a contiguous span of 16-column groups;
// and, split along K, for 2 <= M <= 16 at N <= 4096 with long K.
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
//     copied into LDS ahead of the item; at M >= 2 each lane loads its MFMA A row
//     straight into registers.  With GR distinct rows per 16-row A operand (GR = 4
//     for M <= 4, 8 for M <= 8, else 16), A row r holds activation row
//     min(r / (16 / GR), M - 1), so accumulator i of lane (c, g) is output row
//     (4g + i (16 / GR)) GR / 16: one fp32 update per K-block row at M <= 4, two
//     at M <= 8, four above.
//   * Per 16-column group of the span: LDS reads of two rows first, then four
//     v_and_or_b32 per row into fp16 1024 + q (low nibbles) and 64 + q (high
//     nibbles in place), mfma(x', B, -S) with x' = [x0, x4, x1, x5, x2, x6, x3, x7]
//     and -S = mfma(x', -C) per K block, then acc += d * that in fp32.
//   * Epilogue: each wave's partials per output row and column go to its own
//     (drained) LDS slot; after one barrier they are summed in wave order and
//     stored as fp16.
//
// Split form (SPLIT, 2 <= M <= 16 at N <= 4096, where the groups would give one
// 288-byte strip per workgroup): workgroup (tile, split) owns 64 neighbouring
// columns (1152-byte row pieces, the pattern a plain read serves ~20% faster than
// strips) and one K range of up to 128 K blocks, the same one item per wave.  The
// K splits of a tile share blockIdx.x and run on one XCD; their fp32 partials meet
// in that XCD's L2 and split 0 sums them in split order once each other split's
// flag shows its partial stored (a split whose flag comes from another XCD, or
// not in time, is recomputed from the inputs).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "q4_common.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(q4_gemv_span_split_fallbacks)

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

// Weight copies of an item of ng groups, and how many of them hold rows 0 .. n-1.
__host__ __device__ constexpr int gs_ncopy(int ng) { return (144 * ng + 63) / 64; }
__host__ __device__ constexpr int gs_need_rows(int ng, int n) { return (288 * ng * n + 1023) / 1024; }
// Row segments of an item, each processed once its copies have landed: GS_RP rows
// at a time.  (Taking the last two rows one at a time, so that less math waits
// for the last copy, measured the same.)
constexpr int GS_NSEG = GS_B / GS_RP;
__host__ __device__ constexpr int gs_seg_r0(int sg) { return GS_RP * sg; }
__host__ __device__ constexpr int gs_seg_nr(int) { return GS_RP; }

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
    // Split form: 64-column tiles (blockIdx.x, XCD-renumbered, grid.x a multiple of
    // 8) and K splits (blockIdx.y) of bps K blocks each.
    int S = 1, bps = 0;
    float *part = nullptr;                   // [S][M][N] fp32 partials
    uint32_t *flags = nullptr;               // split flags [tiles][S], behind the partials
    uint32_t spin = 0;                       // polls of a flag before its split is recomputed
    uint32_t foreign = 0;                    // splits treated as run on another XCD (test switch)
};

template <int GR, bool SPLIT>
__global__ void __launch_bounds__(GS_NW * 64)
q4_gemv_span_kernel(GemvSpanArgs a) {
    static_assert(GR == 1 || GR == 4 || GR == 8 || GR == 16, "row groups");
    constexpr int NA = GR <= 4 ? 1 : GR / 4;     // accumulators per group
    constexpr int IS = GR == 1 ? 0 : 16 / GR;    // accumulator i is MFMA result element i * IS
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
    // MFMA lane rows g = 0..3 take K quarters kq = 0, 2, 1, 3 of each block (the
    // activations to match): a 32-lane half then reads quarters {0, 2} or {1, 3}
    // of the 16 columns' nibbles, whose words fall on the 32 LDS banks with fewer
    // conflicts than {0, 1} / {2, 3} (M = 1: 9 against 11 cycles per four
    // half-wave reads, M >= 2: 8 against 12).
    const int kq = ((g & 1) << 1) | (g >> 1);

    constexpr int XS = GR == 1 ? GS_XS : 0;
    uint8_t *xs = smem + wave * (GS_B * 64);
    uint8_t *slot = smem + XS + wave * GS_SLOT;

    int g0, ng, kb0 = 0, kbe = nb;
    uint32_t fb = 0;                         // SPLIT: the tile's split flags as the launch starts
    if constexpr (SPLIT) {
        // Tile t (64 columns) of the XCD-renumbered grid.x; split blockIdx.y owns
        // K blocks [sp bps, (sp + 1) bps).  Every split of a tile has the same
        // blockIdx.x, so the same linear id mod 8 (grid.x a multiple of 8): one XCD.
        const int gx = (int)gridDim.x;
        const int t = ((int)blockIdx.x & 7) * (gx >> 3) + ((int)blockIdx.x >> 3);
        if (t >= (ngt >> 2)) return;                               // grid padding
        if (wave == 0 && lane < a.S)
            fb = __hip_atomic_load(a.flags + t * a.S + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        g0 = 4 * t;
        ng = 4;
        kb0 = (int)blockIdx.y * a.bps;
        kbe = min(kb0 + a.bps, nb);
    } else {
        // XCD renumbering of the GS_GRID workgroups; span bounds by a shift (the
        // grid is fixed, groups <= 1024, so wg * groups fits 32 bits).
        const int wg = ((int)blockIdx.x & 7) * (GS_GRID / 8) + ((int)blockIdx.x >> 3);
        g0 = (wg * ngt) >> 8;
        ng = (((wg + 1) * ngt) >> 8) - g0;                         // 1..GS_NGMAX
        static_assert(GS_GRID == 256, "span bounds by a shift of 8");
    }
    const int row0 = kb0 + wave * GS_B;
    const int rows = max(0, min(GS_B, kbe - row0));                // 0: no item for this wave
    const uint8_t *wb = W + (int64_t)g0 * 288 + (int64_t)row0 * grow;

    const int qoff = c * BLOCK_BYTES + 2 + 4 * kq;
    const uint32_t qal = (uint32_t)(qoff & ~3), qsh = (uint32_t)(qoff & 3) * 8;
    const uint32_t doff = (uint32_t)(c * BLOCK_BYTES);
    // M == 1: only lanes g == 0 keep their sums (every A row is the one activation
    // row), so their second word is taken where it holds the block's scale -- after
    // the first for an even column (whose first word starts at the block), before it
    // for an odd one (whose first word is the nibble bytes exactly) -- and the scale
    // comes from the two words instead of a read of its own.  The B operand is
    // unchanged: the second word only feeds byte 3 of w8, which the masks drop.
    const uint32_t q1off = GR == 1 && g == 0 && (c & 1) ? doff - 2 : qal + 4;
    const uint32_t dsel = (c & 1) ? 0x0C0C0706u : 0x0C0C0100u;     // scale bytes of (q1, q0)
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
            // Lane (c, g): activation row min(c / (16 / GR), M - 1), elements 8g..8g+7
            // of each K block of the batch (blocks past K clamp to the last one).
            const uint8_t *xrow = (const uint8_t *)X + (int64_t)min(c / (16 / GR), M - 1) * ldx * 2 + 16 * kq;
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
        const uint32_t xa = lds_addr(xs + 16 * kq);
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
        const uint32_t vq0 = opaque_vgpr(base + qal), vq1 = opaque_vgpr(base + q1off),
                       vd = opaque_vgpr(base + doff);
        // GS_RP K rows (all groups of the span) at a time, each set as soon as the
        // copies holding it have landed (the copies cover the item in row-major
        // order, so rows up to RP (h + 1) - 1 need the first gs_need(ng, h)).
        // Rows R0 .. R0 + NR - 1 (all groups of the span): their LDS reads first,
        // then the unpacks and MFMAs, then the scaled sums.
        auto proc = [&](auto NGc, auto R0c, auto NRc) {
            constexpr int NG = decltype(NGc)::value;
            constexpr int R0 = decltype(R0c)::value, NR = decltype(NRc)::value;
            constexpr uint32_t rowb = 288u * NG;
            uint32_t q0[NR][NG], q1[NR][NG];
            _Float16 dh[NR][NG];
#pragma unroll
            for (int v = 0; v < NR; ++v)
#pragma unroll
                for (int grp = 0; grp < NG; ++grp) {
                    // Immediate offsets from per-lane bases (one VGPR each for the two
                    // words and the scale), so no address arithmetic per row.
                    const uint32_t ro = (R0 + v) * rowb + grp * 288;
                    q0[v][grp] = *(const lds_u32 *)(lds_ptr(vq0) + ro);
                    q1[v][grp] = *(const lds_u32 *)(lds_ptr(vq1) + ro);
                    if constexpr (GR == 1)
                        dh[v][grp] = bitcast<_Float16>((uint16_t)__builtin_amdgcn_perm(q1[v][grp], q0[v][grp], dsel));
                    else
                        dh[v][grp] = bitcast<_Float16>(*(const lds_u16 *)(lds_ptr(vd) + ro));
                }
            float4_t ns[NR];
#pragma unroll
            for (int v = 0; v < NR; ++v) {
                if constexpr (HOIST) ns[v] = negs[R0 + v];
                else ns[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[R0 + v], negc, z, 0, 0, 0);
            }
            float4_t r[NR][NG];
#pragma unroll
            for (int v = 0; v < NR; ++v)
#pragma unroll
                for (int grp = 0; grp < NG; ++grp) {
                    const uint32_t w = __builtin_amdgcn_alignbit(q1[v][grp], q0[v][grp], qsh);
                    const uint32_t w8 = __builtin_amdgcn_alignbit(q1[v][grp], q0[v][grp], qsh + 8);
                    const uint4_t bq = {and_or(w, mlo, e1024), and_or(w, mhi, e64), and_or(w8, mlo, e1024),
                                        and_or(w8, mhi, e64)};
                    r[v][grp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[R0 + v], bitcast<half8_t>(bq), ns[v], 0,
                                                                       0, 0);
                }
#pragma unroll
            for (int v = 0; v < NR; ++v)
                if (R0 + v < rows) {
#pragma unroll
                    for (int grp = 0; grp < NG; ++grp)
#pragma unroll
                        for (int i = 0; i < NA; ++i)
                            acc[grp][i] += (float)dh[v][grp] * r[v][grp][i * IS];
                }
        };
        // Segments of rows, each run as soon as the copies holding it have landed
        // (the copies cover the item in row-major order).
        static_for<GS_NSEG>([&](auto Sg) {
            constexpr int sg = decltype(Sg)::value;
            constexpr int r0 = gs_seg_r0(sg), nr = gs_seg_nr(sg);
            if constexpr (sg + 1 < GS_NSEG) wait_vmcnt<NC - gs_need_rows(NG, r0 + nr)>();
            else wait_vmcnt<0>();
            proc(NGc, std::integral_constant<int, r0>{}, std::integral_constant<int, nr>{});
        });
    };
    if (rows > 0) {
        if constexpr (SPLIT) {
            item(std::integral_constant<int, 4>{});
        } else {
            switch (ng) {
                case 1: item(std::integral_constant<int, 1>{}); break;
                case 2: item(std::integral_constant<int, 2>{}); break;
                case 3: item(std::integral_constant<int, 3>{}); break;
                default: item(std::integral_constant<int, GS_NGMAX>{}); break;
            }
        }
        // Every LDS read of the slot has returned before it holds the partials.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // Partials into this wave's slot: [output row][64 columns] floats.  Accumulator
    // i of lane (c, g) is output row g GR/4 + i (row 0 for every lane at M == 1).
    float *mine = (float *)slot;
    if (GR > 1 || lane < 16) {
#pragma unroll
        for (int i = 0; i < NA; ++i)
#pragma unroll
            for (int grp = 0; grp < GS_NGMAX; ++grp)
                mine[(GR == 1 ? 0 : g * (GR / 4) + i) * 64 + grp * 16 + c] = acc[grp][i];
    }
    lds_barrier();
    // Thread (row, col) = (tid / 64, tid % 64): 16 rows x 64 columns = the workgroup.
    const int row = tid >> 6, col = tid & 63;
    const bool live = col < 16 * ng && row < (GR == 1 ? 1 : M);
    const int n = 16 * g0 + col;
    float s = 0.f;
    if (live) {
        const float *p = (const float *)(smem + XS) + row * 64 + col;
#pragma unroll
        for (int w = 0; w < GS_NW; ++w) s += p[w * (GS_SLOT / 4)];
        if constexpr (!SPLIT) Y[(int64_t)row * ldy + n] = (_Float16)s;
    }
    if constexpr (SPLIT) {
        // Split 0 sums the S partials in split order: its own from registers, the
        // others through the XCD's L2 (plain stores), each once that split's flag
        // shows it stored.  A flag is one word per (tile, split) written only by
        // that split, which adds 8 to the value it held when the launch started
        // and puts its XCD id in the low 3 bits; split 0 read the same starting
        // values and polls (at most a.spin times) for start + 8.  A split whose
        // flag comes from another XCD, or not in time, is recomputed from the
        // inputs.  Nothing else writes a flag during a launch, so whatever other
        // kernels left in the words between launches, a flag holds its starting
        // value or this launch's.
        const int N = ngt * 16, sp = (int)blockIdx.y, S = a.S;
        const int t = (int)(g0 >> 2);
        uint32_t *last_flag = (uint32_t *)smem;                    // the slots are idle from here
        const uint32_t xcc = xcc_id();
        if (sp != 0) {
            if (live) a.part[((int64_t)sp * M + row) * N + n] = s;
            wait_vmcnt<0>();
            __syncthreads();
            if (wave == 0 && lane == sp)
                __hip_atomic_store(a.flags + t * S + sp, (fb & ~7u) + 8u + xcc, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            return;
        }
        __syncthreads();
        if (wave == 0) {
            const bool mine = lane >= 1 && lane < S;
            const uint32_t want = (fb & ~7u) + 8u;
            uint32_t v = 0;
            bool seen = !mine;
            for (uint32_t it = 0; it < a.spin; ++it) {
                if (!seen) {
                    v = __hip_atomic_load(a.flags + t * S + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    seen = (v & ~7u) == want;
                }
                if (__all(seen)) break;
                __builtin_amdgcn_s_sleep(1);
            }
            const uint64_t good = __ballot(mine && seen && (v & 7u) == xcc);
            if (lane == 0) {
                const uint32_t local = ((uint32_t)good | 1u) & ~a.foreign;
                *last_flag = local;
                if (local != (1u << S) - 1) note_split_fallback();
            }
        }
        __syncthreads();
        if (!live) return;
        const uint32_t local = *last_flag;
        float tot = 0.f;
        for (int q = 0; q < S; ++q) {
            float pv;
            if (q == sp && ((local >> q) & 1)) pv = s;
            else if ((local >> q) & 1) pv = load_l2_f32(a.part, (int)((((int64_t)q * M + row) * N + n) * 4));
            else pv = q4_dot_range(X + (int64_t)row * ldx, W, N, n, min(q * a.bps, nb), min((q + 1) * a.bps, nb));
            tot += pv;
        }
        Y[(int64_t)row * ldy + n] = (_Float16)tot;
    }
}

// True when the span kernel takes the whole of W for M rows: 1 <= M <= 16,
// N % 16 == 0 with 256 < N/16 <= 1024 groups (one span of 1..4 groups per
// workgroup on 256 workgroups), at most 16 batches of 8 K blocks (K <= 4096, one
// item per wave), 16-byte aligned weights and activation rows.
bool gemv_span_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N) {
    if (opt_is("MCQ4_GEMV_SPAN", '0')) return false;
    const int64_t groups = N / 16, nb = K / QK;
    return M >= 1 && M <= 16 && N % 16 == 0 && groups > GS_GRID && groups <= GS_GRID * GS_NGMAX && nb >= 1 &&
           nb <= GS_NW * GS_B && ((uintptr_t)W % 16) == 0 && ((uintptr_t)X % 16) == 0 &&
           (M == 1 || ldx % 8 == 0) && N * 18 * 8 < ((int64_t)1 << 31);
}

template <int GR, bool SPLIT>
static hipError_t launch_span_gr(const GemvSpanArgs &a, dim3 grid, hipStream_t s) {
    const size_t lds = (GR == 1 ? GS_XS : 0) + (size_t)GS_NW * GS_SLOT + GS_PAD;
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemv_span_kernel<GR, SPLIT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((q4_gemv_span_kernel<GR, SPLIT>), grid, dim3(GS_NW * 64), lds, s, a);
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
    const dim3 grid(GS_GRID);
    if (M == 1) return launch_span_gr<1, false>(a, grid, s);
    if (M <= 4) return launch_span_gr<4, false>(a, grid, s);
    if (M <= 8) return launch_span_gr<8, false>(a, grid, s);
    return launch_span_gr<16, false>(a, grid, s);
}

// Split form, 2 <= M <= 16 at N <= 4096: 64-column tiles (N % 64 == 0) and S K
// splits, S the largest power of two (<= 8) with tiles x S <= 256, then bps = K
// blocks per split rounded up to whole batches of 8 (<= 128: one item per wave)
// and S recounted from it.
struct SpanSplitPlan {
    int S, bps, gx;
};
static SpanSplitPlan span_split_plan(int64_t K, int64_t N) {
    const int64_t ntiles = N / 64, nb = K / QK;
    int S = 1;
    while (S < 8 && ntiles * S * 2 <= 256) S *= 2;
    int bps = (int)((nb + S - 1) / S);
    bps = (bps + GS_B - 1) / GS_B * GS_B;
    S = (int)((nb + bps - 1) / bps);
    return {S, bps, (int)((ntiles + 7) / 8 * 8)};
}

// True when the split form takes the whole of W: 2 <= M <= 16, N % 64 == 0 with
// N <= 4096, at least two K splits of at most 128 K blocks each, 16-byte aligned
// weights and activation rows -- and, unless MCQ4_GEMV_SPAN=1 forces it, at least
// 64 K blocks (8 busy waves) per split.  Shorter splits leave most of a workgroup
// idle and pay an exchange the strip kernel does not need there (M = 4 at
// 4096 x 4096: 6.8 against 5.0 us); at K = 14336, N = 4096 the split form is 5-8%
// faster at M = 2..16.  It sums the splits through the XCD's L2 only, so
// MCQ4_XCD_LOCAL=0 (and a forced MCQ4_GEMVM_SPLIT) leave these shapes to the strip
// kernel.
bool gemv_span_split_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N) {
    if (opt_is("MCQ4_GEMV_SPAN", '0') || opt_is("MCQ4_XCD_LOCAL", '0') || opt("MCQ4_GEMVM_SPLIT")) return false;
    if (M < 2 || M > 16 || N % 64 || N < 64 || N > 4096 || K < QK || ldx % 8 || ((uintptr_t)W % 16) ||
        ((uintptr_t)X % 16))
        return false;
    const SpanSplitPlan p = span_split_plan(K, N);
    if (p.S < 2 || p.bps > GS_NW * GS_B) return false;
    return opt_is("MCQ4_GEMV_SPAN", '1') || K / QK >= (int64_t)64 * p.S;
}

size_t gemv_span_split_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M < 2 || M > 16 || N % 64 || N < 64 || N > 4096 || K < QK) return 0;
    const SpanSplitPlan p = span_split_plan(K, N);
    return COUNTER_BYTES + (size_t)p.S * M * N * sizeof(float) + (size_t)(N / 64) * p.S * sizeof(uint32_t);
}

hipError_t launch_gemv_span_split(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y, int64_t ldy,
                                  int M, int K, int N, void *ws, hipStream_t s) {
    if (!ws) return hipErrorInvalidValue;
    const SpanSplitPlan p = span_split_plan(K, N);
    GemvSpanArgs a;
    a.X = X; a.W = W; a.Y = Y;
    a.ldx = ldx; a.ldy = ldy;
    a.M = M;
    a.nb = K / QK;
    a.groups = N / 16;
    a.grow = (uint32_t)N * BLOCK_BYTES;
    a.S = p.S;
    a.bps = p.bps;
    a.part = (float *)((char *)ws + COUNTER_BYTES);
    a.flags = (uint32_t *)(a.part + (int64_t)p.S * M * N);
    a.spin = split_spin();
    a.foreign = split_foreign_mask();
    const dim3 grid(p.gx, p.S);
    // M <= 8: the 8-row instance (at M = 3, 4 on 14336 x 4096 the 4-row one ran
    // 11.3-11.8 against 10.8-11.0 us, same box; equal at M = 2).
    if (M <= 8) return launch_span_gr<8, true>(a, grid, s);
    return launch_span_gr<16, true>(a, grid, s);
}

}  // namespace mcq4
