// Decode-shaped q4_0 matmul (M <= 64), LDS-staged strip variant (the default
// decode path when N % 8 == 0 and W is 16-byte aligned).
//
// Why: in the [K/32][N][18] layout a 16-column tile is a strip of 288-byte row
// segments 18*N bytes apart.  Fetching it with per-lane 2/4-byte loads (one
// wave instruction = 144 useful bytes) starves the memory pipeline; the same
// bytes fetched as 16-byte coalesced loads (1 KiB per wave instruction) stream
// at close to the plain-copy rate.
//
// Structure.  A workgroup has WAVES waves in TPW = WAVES/KS tile slots of KS
// waves each.  A slot's KS waves split the K-block rows of one column tile of
// 16*NT columns; the workgroup walks tile groups (blockIdx.x, +gridDim.x, ...)
// so that a small grid stays resident and streams continuously.
//   * Rows are streamed in batches of B.  A batch's strip bytes (B rows of
//     288*NT contiguous bytes) and its activations (M rows x B*64 bytes) are
//     fetched with 16-byte coalesced loads into registers.  The next batch --
//     possibly of the next tile -- is issued before the current one is
//     computed, so memory latency overlaps the math and the tile epilogue.
//   * Each wave bounces its batch through a private LDS slice (no workgroup
//     barrier: a wave's LDS accesses are ordered) to regroup bytes into the
//     MFMA layout: lane (column c = l%16, k-group g = l/16) reads the fp16 scale
//     and qs bytes 4g..4g+3 of its block, dequant8_perm turns them into fp16
//     (q-8)*d, and one v_mfma_f32_16x16x32_f16 per 16-row M tile accumulates in
//     fp32.  The kernel covers whole column tiles only; the launcher sends the
//     remaining N % (16*NT) columns to the generic decode kernel.
//   * KS > 1: the slot's partial tiles are summed through LDS in a fixed order
//     (one barrier pair per 16x16 fragment); KS == 1: each wave stores its own
//     tile.  Results are written as fp16.
#include <algorithm>
#include <atomic>

#include "q4_common.h"

namespace mcq4 {

struct DecodeArgs {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *W;
    _Float16 *Y;
    int64_t ldy;
    int M, nb, N;
    int ntiles;
};

template <int MR, int NT>
struct DecodeShape {
    static constexpr int MT = (MR + 15) / 16;           // 16-row M tiles
    static constexpr int B = (MR <= 4) ? 8 : 4;         // rows (K blocks) per batch
    static constexpr int ROW_BYTES = 288 * NT;          // strip bytes per row
    static constexpr int CPR = 18 * NT;                 // 16-byte strip chunks per row
    static constexpr int CH = B * CPR;                  // strip chunks per batch
    static constexpr int LPL = (CH + 63) / 64;          // strip loads per lane per batch
    static constexpr int XROW = B * 64 + 16;            // LDS bytes per activation row (+pad)
    static constexpr int XCPR = B * 4;                  // 16-byte activation chunks per row
    static constexpr int XL = (MR * XCPR + 63) / 64;    // activation loads per lane
    static constexpr int W_LDS = B * ROW_BYTES + 16;    // +16: the last row's qs read2 overhang
    static constexpr int ZERO_LDS = B * 64;             // zero activations for rows m >= M
    // Per-wave LDS slice for `mrows` activation rows (the launch sizes it for M).
    static constexpr int wave_lds(int mrows) { return W_LDS + mrows * XROW; }
    // Batch row r is complete once strip load (r*CPR + CPR - 1) / 64 has landed.
    static constexpr int last_load_of_row(int r) { return (r * CPR + CPR - 1) / 64; }
};

template <int MR, int NT, int WAVES, int KS>
__global__ void __launch_bounds__(WAVES * 64)
q4_decode_lds_kernel(DecodeArgs a) {
    using S = DecodeShape<MR, NT>;
    constexpr int MT = S::MT;
    constexpr int B = S::B, CPR = S::CPR, LPL = S::LPL, ROW_BYTES = S::ROW_BYTES;
    constexpr int XROW = S::XROW, XCPR = S::XCPR, XL = S::XL;
    constexpr int NFRAG = MT * NT;
    constexpr int TPW = WAVES / KS;
    static_assert(WAVES % KS == 0, "KS must divide WAVES");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int slot = wave / KS, kp = wave % KS;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int mrows = min(a.M, MR);
    const uint32_t grow = (uint32_t)a.N * BLOCK_BYTES;
    // LDS: [zero activations][WAVES x per-wave slice][reduction scratch when KS > 1]
    uint8_t *zero = smem;
    uint8_t *wlds = smem + S::ZERO_LDS + wave * S::wave_lds(mrows);
    uint8_t *xlds = wlds + S::W_LDS;
    float *red = (float *)(smem + S::ZERO_LDS + WAVES * S::wave_lds(mrows));

    // Strip chunk geometry of one batch (global offset from the batch's first row,
    // LDS offset, batch row).  Chunk q = lane + 64*i.
    uint32_t soff[LPL], slds[LPL];
    int srow[LPL];
#pragma unroll
    for (int i = 0; i < LPL; ++i) {
        const int q = lane + 64 * i;
        const int r = q / CPR, k = q - r * CPR;
        srow[i] = q < S::CH ? r : B;            // B = never valid
        soff[i] = (uint32_t)r * grow + 16u * k;
        slds[i] = (uint32_t)(r * ROW_BYTES + 16 * k);
    }
    // Activation chunk geometry: row m, 16-byte chunk k of the batch's B*32 halves.
    uint32_t xoff[XL], xlo[XL];
    int xrw[XL];
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int q = lane + 64 * i;
        const int m = q / XCPR, k = q - m * XCPR;
        xrw[i] = m < mrows ? (k >> 2) : B;      // batch row of this chunk (B = none)
        xoff[i] = (uint32_t)(m * a.ldx * 2 + 16 * k);
        xlo[i] = (uint32_t)(m * XROW + 16 * k);
    }
    // A-operand read base per M tile (row u adds u*64): lanes past M read zeros.
    const uint8_t *abase[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        abase[mt] = (mt * 16 + c < mrows) ? xlds + (mt * 16 + c) * XROW + 16 * g : zero + 16 * g;
    // B-operand reads: d at c*18, qs bytes 4g..4g+3 at c*18 + 2 + 4g, fetched as the
    // aligned dword pair around them and funnel-shifted.
    const int qoff = c * BLOCK_BYTES + 2 + 4 * g;
    const uint32_t qal = (uint32_t)(qoff & ~3), qsh = (uint32_t)(qoff & 3) * 8;
    const uint32_t doff = (uint32_t)(c * BLOCK_BYTES);

    // Zero activations for lanes past M (written once, read-only afterwards).
    for (int i = tid; i < S::ZERO_LDS / 16; i += WAVES * 64)
        *(uint4_t *)(zero + 16 * i) = uint4_t{0u, 0u, 0u, 0u};
    __syncthreads();

    // This wave's K rows (identical for every tile) and its batch count.
    const int rpp = (a.nb + KS - 1) / KS;
    const int rbeg = min(a.nb, kp * rpp);
    const int rend = min(a.nb, rbeg + rpp);
    const int nbatch = (rend - rbeg + B - 1) / B;
    // XCD-aware numbering: workgroups are dispatched round-robin over the 8 XCDs,
    // so workgroup b runs on XCD b % 8.  Neighbouring tile groups share 128-byte
    // lines (a 16-column strip row is 288 bytes), so consecutive groups go to
    // workgroups of one XCD, whose L2 then fetches each shared line once.
    const int G = (int)gridDim.x, G8 = G & ~7;
    int wg = (int)blockIdx.x;
    if (wg < G8) wg = (wg & 7) * (G8 >> 3) + (wg >> 3);
    const int ngroups_total = (a.ntiles + TPW - 1) / TPW;
    const int ngroups = (ngroups_total - wg + G - 1) / G;
    const uint8_t *xbase = (const uint8_t *)a.X;
    auto tile_of = [&](int j) { return (wg + j * G) * TPW + slot; };

    uint4_t wv[LPL], xr[XL];
    auto issue_w = [&](int i, int tile, int row0) {
        const int rows = min(B, rend - row0);
        const uint8_t *gb = a.W + (int64_t)tile * (16 * NT * BLOCK_BYTES) + (int64_t)row0 * grow;
        if (srow[i] < rows) wv[i] = __builtin_nontemporal_load((const uint4_t *)(gb + soff[i]));
    };
    auto issue_x = [&](int row0) {
        const int rows = min(B, rend - row0);
        const uint8_t *xb = xbase + (int64_t)row0 * (QK * 2);
#pragma unroll
        for (int i = 0; i < XL; ++i)
            if (xrw[i] < rows) xr[i] = *(const uint4_t *)(xb + xoff[i]);
    };
    auto issue_all = [&](int tile, int row0) {
        issue_x(row0);
#pragma unroll
        for (int i = 0; i < LPL; ++i) issue_w(i, tile, row0);
    };

    // Per-lane LDS read bases, materialized once so that rows and column tiles
    // become immediate offsets of the ds_read instructions.
    uint32_t qo = lds_addr(wlds + qal);
    uint32_t dof = lds_addr(wlds + doff);
    uint32_t ao[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) ao[mt] = lds_addr(abase[mt]);
    asm volatile("" : "+v"(qo), "+v"(dof));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) asm volatile("" : "+v"(ao[mt]));

    float4_t acc[MT][NT];
    // Operands of one batch row read from LDS: activations (per M tile), the qs
    // dword pair and the scale of each column tile.
    struct RowOps {
        half8_t av[MT];
        uint32_t q0[NT], q1[NT], d[NT];
    };
    auto row_read = [&](int u) {
        RowOps o;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o.av[mt] = *(const lds_half8 *)(lds_ptr(ao[mt]) + u * 64);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const lds_u32 *qp = (const lds_u32 *)(lds_ptr(qo) + u * ROW_BYTES + t * 288);
            o.q0[t] = qp[0];
            o.q1[t] = qp[1];
            o.d[t] = *(const lds_u16 *)(lds_ptr(dof) + u * ROW_BYTES + t * 288);
        }
        return o;
    };
    auto row_math = [&](const RowOps &o) {
        if constexpr (MR == 1) {
            // Single activation row: B holds the exact halves 1024 + q, a second
            // MFMA against ones gives sum(x) of the block, and the -8 offset and
            // scale are applied in fp32 on the one output lane that matters
            // (D[0][c], i = 0 of lanes 0..15):
            //   y += d * (sum x*(1024+q) - 1032 * sum x) = d * sum x*(q-8).
            const half8_t ones = {(_Float16)1, (_Float16)1, (_Float16)1, (_Float16)1,
                                  (_Float16)1, (_Float16)1, (_Float16)1, (_Float16)1};
            const float4_t z = {0.f, 0.f, 0.f, 0.f};
            const float4_t sx = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.av[0], ones, z, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint32_t w = __builtin_amdgcn_alignbit(o.q1[t], o.q0[t], qsh);
                const float d = (float)bitcast<_Float16>((uint16_t)o.d[t]);
                const float4_t blk =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(o.av[0], unpack8_1024(w), z, 0, 0, 0);
                acc[0][t][0] = __builtin_fmaf(d, __builtin_fmaf(-1032.f, sx[0], blk[0]), acc[0][t][0]);
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint32_t w = __builtin_amdgcn_alignbit(o.q1[t], o.q0[t], qsh);
                const half8_t bv = dequant8_perm(w, o.d[t]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.av[mt], bv, acc[mt][t], 0, 0, 0);
            }
        }
    };

    if (nbatch > 0 && ngroups > 0 && tile_of(0) < a.ntiles) issue_all(tile_of(0), rbeg);
    for (int j = 0; j < ngroups; ++j) {
        const int tile = tile_of(j);
        const bool tile_ok = tile < a.ntiles;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};

        for (int b = 0; b < nbatch; ++b) {
            const int row0 = rbeg + b * B;
            const int rows = min(B, rend - row0);
            // Next batch: this tile's, or the next group's tile's first.
            int ntile = tile, nrow0 = row0 + B;
            bool more = b + 1 < nbatch && tile_ok;
            if (b + 1 >= nbatch && j + 1 < ngroups && tile_of(j + 1) < a.ntiles) {
                ntile = tile_of(j + 1);
                nrow0 = rbeg;
                more = true;
            }
            // Activations: stage (permuted to the dequant slot order), then prefetch.
            if (tile_ok) {
#pragma unroll
                for (int i = 0; i < XL; ++i)
                    if (xrw[i] < rows)
                        *(half8_t *)(xlds + xlo[i]) = perm_act8(xr[i]);
            }
            if (more) issue_x(nrow0);
            // Strip: stage load i, prefetch its successor, then run the rows it completed.
#pragma unroll
            for (int i = 0; i < LPL; ++i) {
                if (tile_ok && srow[i] < rows) *(uint4_t *)(wlds + slds[i]) = wv[i];
                if (more) issue_w(i, ntile, nrow0);
                if (tile_ok) {
#pragma unroll
                    for (int u = 0; u < B; ++u)
                        if (S::last_load_of_row(u) == i && u < rows) row_math(row_read(u));
                }
            }
        }

        // ---- tile epilogue ---------------------------------------------------
        const int n0 = tile * 16 * NT;
        if constexpr (KS == 1) {
            if (tile_ok) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int m = mt * 16 + 4 * g + i;
                            if (m < a.M)
                                a.Y[(int64_t)m * a.ldy + n0 + t * 16 + c] = (_Float16)acc[mt][t][i];
                        }
            }
        } else {
#pragma unroll
            for (int f = 0; f < NFRAG; ++f) {
                const int mt = f / NT, t = f % NT;
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave * 256 + lane * 4 + i] = acc[mt][t][i];
                __syncthreads();
                // The slot's KS*64 threads finish its 256 values, summing waves in order.
                for (int vi = tid - slot * KS * 64; vi < 256; vi += KS * 64) {
                    float s = 0.f;
#pragma unroll
                    for (int w = 0; w < KS; ++w) s += red[(slot * KS + w) * 256 + vi];
                    const int l = vi >> 2, i = vi & 3;
                    const int m = mt * 16 + 4 * (l >> 4) + i;
                    if (tile_ok && m < a.M)
                        a.Y[(int64_t)m * a.ldy + n0 + t * 16 + (l & 15)] = (_Float16)s;
                }
                __syncthreads();
            }
        }
    }
}

// ---- launch -----------------------------------------------------------------

struct DecodeCfg {
    int NT, WAVES, KS, grid_cap;
};

// Small N (few column tiles): all waves of a 16-wave workgroup split K of one
// tile.  Large N: 4-wave workgroups whose waves each own a whole tile (no
// reduction); the grid is capped so workgroups stay resident and pipeline
// across the tiles they walk.
static DecodeCfg decode_config(int64_t M, int64_t K, int64_t N) {
    (void)K;
    DecodeCfg c{1, 16, 16, 256};                  // one resident 16-wave workgroup per CU
    if (M > 4 && N >= 8192) c = DecodeCfg{2, 16, 16, 0};
    if (M <= 16 && N / 16 >= 4096) c = DecodeCfg{2, 8, 1, 0};     // lm_head-sized N
    return c;
}

template <int MR, int NT, int WAVES, int KS>
static hipError_t launch_dec_t(const DecodeArgs &a, int grid_cap, hipStream_t s) {
    using S = DecodeShape<MR, NT>;
    const int mrows = std::min(a.M, MR);
    size_t lds = S::ZERO_LDS + (size_t)WAVES * S::wave_lds(mrows);
    if (KS > 1) lds += (size_t)WAVES * 256 * sizeof(float);
    if (lds > 160 * 1024) return hipErrorInvalidConfiguration;
    // Raise the dynamic-LDS limit once per device (bit d of `done`).
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_decode_lds_kernel<MR, NT, WAVES, KS>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    constexpr int TPW = WAVES / KS;
    int grid = (a.ntiles + TPW - 1) / TPW;
    if (grid_cap > 0) grid = std::min(grid, grid_cap);
    hipLaunchKernelGGL((q4_decode_lds_kernel<MR, NT, WAVES, KS>), dim3(grid), dim3(WAVES * 64),
                       lds, s, a);
    return hipGetLastError();
}

template <int MR, int NT>
static hipError_t launch_dec_nt(const DecodeArgs &a, const DecodeCfg &c, hipStream_t s) {
    if (c.KS == 1) {
        if (c.WAVES == 4) return launch_dec_t<MR, NT, 4, 1>(a, c.grid_cap, s);
        return launch_dec_t<MR, NT, 8, 1>(a, c.grid_cap, s);
    }
    if (c.KS == 4) return launch_dec_t<MR, NT, 8, 4>(a, c.grid_cap, s);
    // K split by all waves; fall back to fewer waves when the LDS slices do not fit.
    if (c.WAVES == 16 && MR <= 32) {
        hipError_t e = launch_dec_t<MR, NT, 16, 16>(a, c.grid_cap, s);
        if (e != hipErrorInvalidConfiguration) return e;
    }
    if (c.WAVES >= 8) {
        hipError_t e = launch_dec_t<MR, NT, 8, 8>(a, c.grid_cap, s);
        if (e != hipErrorInvalidConfiguration) return e;
    }
    return launch_dec_t<MR, NT, 4, 4>(a, c.grid_cap, s);
}

template <int MR>
static hipError_t launch_dec_mr(const DecodeArgs &a, const DecodeCfg &c, hipStream_t s) {
    if (c.NT == 1) return launch_dec_nt<MR, 1>(a, c, s);
    return launch_dec_nt<MR, 2>(a, c, s);
}

// True when the LDS-staged decode kernel applies: 16-byte loads of strip rows
// need 18*N to be a multiple of 16 (N % 8 == 0; 18*8 = 144 = 9*16), a 16-byte
// aligned weight base, activation rows 16-byte aligned, and the strip row
// offsets of one batch within 32 bits.
bool decode_lds_supported(const uint8_t *W, int64_t N, int64_t ldx) {
    return N % 8 == 0 && ((uintptr_t)W % 16) == 0 && N * 18 * 8 < ((int64_t)1 << 31) &&
           ldx * 2 * 64 < ((int64_t)1 << 31);
}

// Launches the LDS-staged kernel over the whole column tiles of 16*NT columns;
// returns through *n_done how many leading columns it covers (a multiple of 16*NT).
hipError_t launch_decode_lds(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y,
                             int64_t ldy, int M, int K, int N, int *n_done, hipStream_t s) {
    const DecodeCfg c = decode_config(M, K, N);
    DecodeArgs a;
    a.X = X; a.ldx = ldx; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.nb = K / QK; a.N = N;
    a.ntiles = N / (16 * c.NT);
    *n_done = a.ntiles * 16 * c.NT;
    if (a.ntiles == 0) return hipSuccess;
    if (M == 1) return launch_dec_mr<1>(a, c, s);
    if (M <= 4) return launch_dec_mr<4>(a, c, s);
    if (M <= 16) return launch_dec_mr<16>(a, c, s);
    if (M <= 32) return launch_dec_mr<32>(a, c, s);
    if (M <= 48) return launch_dec_mr<48>(a, c, s);
    return launch_dec_mr<64>(a, c, s);
}

}  // namespace mcq4
