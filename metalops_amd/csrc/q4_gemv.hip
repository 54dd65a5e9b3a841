// Single-row (M == 1) q4_0 GEMV on gfx950.
//
// A decode projection reads 9-30 MB of q4_0 weights once; at that size the
// launch latency and every serial step of a workgroup matter as much as the
// bandwidth.  The kernel keeps the weight stream in asynchronous
// global->LDS copies (no VGPR staging, exact vmcnt accounting) and keeps the
// per-row math to one MFMA, two LDS reads and seven VALU instructions.
//
// Work decomposition
//   * Column tile = TW columns (a TW*18-byte strip row per K block).  Item = one
//     tile's batch of B = 2304 / (18 TW) consecutive K blocks (2304 bytes):
//     TW = 16, B = 8 for the layer shapes; TW = 64, B = 2 for N >= 65536
//     (lm_head), whose 1152-byte row pieces are nine whole 128-byte lines.
//     A 16-column tile's 288-byte pieces straddle lines shared with the
//     neighbouring tiles; a plain read of that pattern is 13-17% slower than one
//     of 1152-byte pieces, but a 64-column tile leaves too few workgroups
//     (N/64/TPW) to spread the per-row math over all CUs below N ~ 64K.
//   * Workgroup = NW waves (16; 8 for N > 16384) owning TPW tiles: wg, wg+G, ...
//     (wg renumbered so consecutive tiles, which share 128-byte lines, run on one
//     XCD).  Wave w owns batches b = w, w+NW, ... of every one of those tiles and walks them
//     batch-major: for each of its batches, the TPW tiles in turn.  The
//     batch's activations therefore stay in registers across the tiles.
//   * Copies: per item exactly three global_load_lds_dwordx4 (1 KiB each; 144
//     chunks, lanes 16..63 of the last masked) into a per-wave ring of R LDS
//     slots; item k+R-1 is issued (into the slot item k-1 freed) before the wave
//     waits for item k.  Rows past K re-copy row 0, so every item issues the same number of
//     copies and the vmcnt waits are exact.
//   * Activations: lane (c = l%16, g = l/16) reads elements 8g..8g+7 of each of
//     the batch's B K blocks from the wave's LDS copy (all 16 lanes of a group
//     read the same 16 bytes) and rearranges them to
//     x' = [x0, x4, x1, x5, x2, x6, x3, x7] (4 v_perm).
//   * Weights: for each 16-column group of the tile, lane (c, g) reads the qs
//     dword w of elements 8g..8g+7 of column c of the group.  Four v_and_or_b32
//     build the fp16 operand [1024+q0, 1024+q4, 64+q1, 64+q5, 1024+q2, 1024+q6,
//     64+q3, 64+q7]: a low nibble under the exponent of 1024 is 1024 + q, a high
//     nibble left in place (bits 4..7 of the half) under the exponent of 64 is
//     64 * (1 + 16q/1024) = 64 + q.  Against the constant operand
//     C = [1032, 1032, 72, 72, 1032, 1032, 72, 72] the same x' gives the block
//     sum S, so one MFMA per K block and batch, mfma(x', -C), yields -S; it is
//     the accumulator input of the per-row MFMA:
//     mfma(x', B, -S)[0] = sum x*(q - 8), exact products, fp32 sums.
//   * Per item, the LDS reads of all eight rows (K block x 16-column group) are
//     issued first, then the unpacks and MFMAs, then acc += d * that in fp32, so
//     the wave that finishes last is not serialised on LDS and MFMA latency.
//   * Epilogue: partials of the waves per column summed through LDS in wave
//     order (deterministic), stored as fp16.
#include <algorithm>
#include <atomic>

#include "q4_common.h"



namespace mcq4 {

constexpr int GV_ITEM = 2304;                // strip bytes per item
constexpr int GV_WCH = GV_ITEM / 16;         // 144 strip chunks of 16 bytes per item
constexpr int GV_LOADS = 3;                  // copies per item (chunks 0..143 of 192)
constexpr int GV_SLOT = GV_ITEM + 64;        // + read overhang
constexpr int GV_WIDE = 64;                  // tile width of the large-N plan
constexpr int GV_WIDE_MIN_TILES = 1024;      // 64-column tiles from N = 65536 on
constexpr int GV_TPW_MAX = 4;                // tiles per workgroup
constexpr int GV_K_MAX = 16384;
#ifndef GV_RING_SET
constexpr int GV_RING = 2;                   // items in flight per wave (1 and 3 measured slower)
#else
constexpr int GV_RING = GV_RING_SET;
#endif
constexpr int GV_NT = 2;                     // cache policy of the weight copies: non-temporal

constexpr int GV_GROUP_MAX = 4;              // weights sharing X in one launch

struct GemvArgs {
    const _Float16 *X;
    // Up to GV_GROUP_MAX weights of the same [K/32][N][18] shape, and their
    // outputs: tile t is tile t % tiles_per_w of weight t / tiles_per_w.
    const uint8_t *W[GV_GROUP_MAX];
    _Float16 *Y[GV_GROUP_MAX];
    int tiles_per_w;
    int nb, N, ntiles, nbt;                  // N per weight; ntiles over all; nbt = batches per tile
    int xw;                                  // activation bytes per wave in LDS
    // Columns of the last tile (one weight, TW = 16): 16, or 8 when N % 16 == 8;
    // that tile's copies of the other chunks re-read its first chunk of the row,
    // and only its first tail_cols outputs are stored.
    int tail_cols = 16;
};

template <int R>
__device__ __forceinline__ void gv_wait(int pending) {
    // Wait until at most `pending` items (LOADS copies each) are still in flight.
    if (R > 4 && pending >= 4) { wait_vmcnt<4 * GV_LOADS>(); return; }
    if (R > 3 && pending >= 3) { wait_vmcnt<3 * GV_LOADS>(); return; }
    if (R > 2 && pending >= 2) { wait_vmcnt<2 * GV_LOADS>(); return; }
    if (R > 1 && pending >= 1) { wait_vmcnt<1 * GV_LOADS>(); return; }
    wait_vmcnt<0>();
}

template <int R, int TPW, int NW, int TW, bool GROUP>
__global__ void __launch_bounds__(NW * 64)
q4_gemv_dma_kernel(GemvArgs a) {
    static_assert(R >= 1 && R <= 3 && TPW >= 1 && TPW <= GV_TPW_MAX, "config");
    constexpr int ROWB = TW * BLOCK_BYTES;   // strip bytes per K block
    constexpr int B = GV_ITEM / ROWB;        // K blocks per item
    constexpr int CPR = ROWB / 16;           // 16-byte chunks per strip row
    constexpr int NG = TW / 16;              // 16-column MFMA groups per tile
    // 16-column tiles keep the wave partials in an LDS area of their own (one
    // barrier in the epilogue); 64-column tiles put them in the ring slots once
    // every wave is done (a second barrier) to stay at three workgroups per CU.
    constexpr bool SEPRED = TW == 16;
    static_assert(B * ROWB == GV_ITEM && NG * 16 == TW && B * NG == 8, "tile width");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // Every kernel argument the prologue needs, loaded in one scalar round trip
    // (the uses below sit behind branches, which would otherwise split the loads).
    const int G = (int)gridDim.x, ntiles = a.ntiles, tpwt = a.tiles_per_w, nb = a.nb, nbt = a.nbt, xw = a.xw;
    const uint32_t grow = (uint32_t)a.N * BLOCK_BYTES;
    const _Float16 *X = a.X;
    const uint8_t *W0 = a.W[0];
    _Float16 *Y0 = a.Y[0];
    asm volatile("" ::"s"(ntiles), "s"(tpwt), "s"(nb), "s"(nbt), "s"(xw), "s"(grow), "s"(X), "s"(W0), "s"(Y0));
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    // MFMA lane rows g = 0..3 take K quarters kq = 0, 2, 1, 3 of each block (the
    // activations to match): a 32-lane half then reads quarters {0, 2} or {1, 3}
    // of the 16 columns' nibbles, whose words fall on the 32 LDS banks with fewer
    // conflicts than {0, 1} / {2, 3} (M = 1: 9 against 11 cycles per four
    // half-wave reads, M >= 2: 8 against 12).
    const int kq = ((g & 1) << 1) | (g >> 1);

    // LDS: [NW waves x activations][NW waves x R slots][partials when SEPRED]
    uint8_t *xs = smem + wave * xw;
    uint8_t *ring = smem + NW * xw + wave * (R * GV_SLOT);
    float *red = (float *)(smem + NW * xw + (SEPRED ? NW * R * GV_SLOT : 0));

    const int G8 = G & ~7;
    int wg = (int)blockIdx.x;
    {
        const int r = (wg & 7) * (G8 >> 3) + (wg >> 3);
        wg = wg < G8 ? r : wg;
    }
    // Tile j of this workgroup: wg + j*G.  Everything up to the first copy is
    // on every launch's critical path, so no integer divisions here: the tile
    // count by compares, the weight of a tile by subtracting tiles_per_w.
    int ntl = 0;                                                  // >= 1 (grid <= ntiles)
#pragma unroll
    for (int j = 0; j < TPW; ++j) ntl += wg + j * G < ntiles ? 1 : 0;
    const uint8_t *wt[TPW];
    _Float16 *yt[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        int lt = j < ntl ? wg + j * G : 0, gi = 0;
        if (GROUP) {
#pragma unroll
            for (int r = 1; r < GV_GROUP_MAX; ++r)
                if (lt >= tpwt) { lt -= tpwt; gi = r; }
        }
        const uint8_t *w = !GROUP || gi == 0 ? W0 : gi == 1 ? a.W[1] : gi == 2 ? a.W[2] : a.W[3];
        _Float16 *y = !GROUP || gi == 0 ? Y0 : gi == 1 ? a.Y[1] : gi == 2 ? a.Y[2] : a.Y[3];
        wt[j] = w + (int64_t)lt * ROWB;
        yt[j] = y + lt * TW;
    }
    // Chunks per row of the tile (CPR, or fewer for a partial last tile).
    int tcpr[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
        tcpr[j] = !GROUP && TW == 16 && j < ntl && wg + j * G == ntiles - 1 ? a.tail_cols * BLOCK_BYTES / 16 : CPR;
    const int nbm = nbt > wave ? (nbt - wave + NW - 1) / NW : 0;  // my batches
    const int nmine = nbm * ntl;

    // Copy geometry per lane and copy i: strip chunk q = lane + 64 i of an item
    // (row q/CPR, 16-byte piece q%CPR); q >= 144 is masked off.
    int crow[GV_LOADS], cpc[GV_LOADS];
    uint32_t coff[GV_LOADS];
#pragma unroll
    for (int i = 0; i < GV_LOADS; ++i) {
        const int q = lane + 64 * i;
        crow[i] = q < GV_WCH ? q / CPR : 0;
        cpc[i] = q < GV_WCH ? q % CPR : 0;
        coff[i] = q < GV_WCH ? (uint32_t)(q / CPR) * grow + 16u * (uint32_t)(q % CPR) : 0u;
    }
    // Item (batch index m of this wave, tile j) into ring slot `slot`.
    auto issue = [&](int m, int j, int slot) {
        const int row0 = (wave + NW * m) * B;
        const int rows = min(B, nb - row0);
        const uint8_t *wb = wt[j] + (int64_t)row0 * grow;
#pragma unroll
        for (int i = 0; i < GV_LOADS; ++i) {
            // Rows past K re-copy row 0, and chunks past a partial tile's columns
            // the row's first chunk (valid memory, never stored).
            uint32_t off = crow[i] < rows ? coff[i] : coff[i] - (uint32_t)crow[i] * grow;
            if (cpc[i] >= tcpr[j]) off -= 16u * (uint32_t)cpc[i];
            if (i < GV_LOADS - 1 || lane < GV_WCH - 64 * (GV_LOADS - 1))
                __builtin_amdgcn_global_load_lds(
                    (void *)(wb + off),
                    (__attribute__((address_space(3))) void *)(ring + slot * GV_SLOT + 1024 * i),
                    16, 0, GV_NT);
        }
    };

    // Prologue: the first R items in flight (issue cursor im, ij, islot).
    int im = 0, ij = 0, islot = 0;
    auto issue_next = [&]() {
        issue(im, ij, islot);
        islot = islot + 1 == R ? 0 : islot + 1;
        if (++ij == ntl) { ij = 0; ++im; }
    };
    // Activations of all my batches first (64 B bytes each: lanes 0..4B-1 copy
    // row lane/4, piece lane%4; rows past K clamp to the last row), so they are
    // older than every weight copy and land before the first item does.
    for (int m = 0; m < nbm; ++m) {
        const int r = min((wave + NW * m) * B + (lane >> 2), nb - 1);
        if (lane < 4 * B)
            __builtin_amdgcn_global_load_lds(
                (void *)((const uint8_t *)X + (int64_t)r * (QK * 2) + 16 * (lane & 3)),
                (__attribute__((address_space(3))) void *)(xs + m * (B * 64)), 16, 0, 0);
    }
    // R-1 items ahead; each iteration issues one more before it waits, into the
    // slot the previous item freed.
    const int npro = min(R - 1, nmine);
    for (int k = 0; k < npro; ++k) issue_next();

    const int qoff = c * BLOCK_BYTES + 2 + 4 * kq;
    const uint32_t qal = (uint32_t)(qoff & ~3), qsh = (uint32_t)(qoff & 3) * 8;
    // Only lanes g == 0 keep their sums (M == 1: every A row is the activation
    // row), so their second word is taken where it holds the block's scale -- after
    // the first for an even column (whose first word starts at the block), before it
    // for an odd one (whose first word is the nibble bytes exactly) -- and the scale
    // comes from the two words instead of a read of its own.  The B operand is
    // unchanged: the second word only feeds byte 3 of w8, which the masks drop.
    const uint32_t q1off = g == 0 && (c & 1) ? (uint32_t)(c * BLOCK_BYTES - 2) : qal + 4;
    const uint32_t dsel = (c & 1) ? 0x0C0C0706u : 0x0C0C0100u;     // scale bytes of (q1, q0)
    // fp16 exponent words: 1024 + q for a low nibble (bits 0..3 of a half),
    // 64 + q for a high nibble left in place (bits 4..7: 64 * (1 + 16q/1024)).
    const uint32_t e1024 = opaque_vgpr(0x64006400u), e64 = opaque_vgpr(0x54005400u);
    const uint32_t mlo = opaque_sgpr(0x000F000Fu), mhi = opaque_sgpr(0x00F000F0u);
    // -C as the fp16 operand: (-1032, -1032) and (-72, -72) pairs.
    const uint32_t nlo = 0xE408E408u, nhi = 0xD480D480u;
    const half8_t negc = bitcast<half8_t>(uint4_t{nlo, nhi, nlo, nhi});
    const float4_t z = {0.f, 0.f, 0.f, 0.f};

    float acc[TPW][NG];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int q = 0; q < NG; ++q) acc[j][q] = 0.f;

    int k = 0, slot = 0;
    for (int m = 0; m < nbm; ++m) {
        const int rows = min(B, nb - (wave + NW * m) * B);
        half8_t xq[B];
        float4_t negs[B];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            if (j < ntl) {
                if (k + R - 1 < nmine) issue_next();
                if (j == 0) {
                    // The batch's activations, built while item k is still in flight:
                    // they were copied before any weights, so at most the items in
                    // flight (this one included) are newer.
                    gv_wait<R + 1>(min(R, nmine - k));
                    const uint32_t xa = lds_addr(xs + m * (B * 64) + 16 * kq);
#pragma unroll
                    for (int u = 0; u < B; ++u) {
                        const uint4_t x = bitcast<uint4_t>(*(const lds_half8 *)(lds_ptr(xa) + u * 64));
                        const uint4_t v = {__builtin_amdgcn_perm(x[2], x[0], 0x05040100u),   // x0, x4
                                           __builtin_amdgcn_perm(x[2], x[0], 0x07060302u),   // x1, x5
                                           __builtin_amdgcn_perm(x[3], x[1], 0x05040100u),   // x2, x6
                                           __builtin_amdgcn_perm(x[3], x[1], 0x07060302u)};  // x3, x7
                        xq[u] = bitcast<half8_t>(v);
                        negs[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[u], negc, z, 0, 0, 0);
                    }
                }
                gv_wait<R>(min(R - 1, nmine - 1 - k));
                // All eight (K block, column group) rows of the item: LDS reads
                // first, then the unpack and MFMAs, then the scaled sums, so a wave
                // that runs alone at the end of the launch is not serialised on
                // LDS and MFMA latencies row by row.
                const uint32_t base = lds_addr(ring + slot * GV_SLOT);
                uint32_t q0[B][NG], q1[B][NG];
                _Float16 dh[B][NG];
#pragma unroll
                for (int u = 0; u < B; ++u)
#pragma unroll
                    for (int grp = 0; grp < NG; ++grp) {
                        q0[u][grp] = *(const lds_u32 *)(lds_ptr(base + qal) + u * ROWB + grp * 288);
                        q1[u][grp] = *(const lds_u32 *)(lds_ptr(base + q1off) + u * ROWB + grp * 288);
                        dh[u][grp] = bitcast<_Float16>((uint16_t)__builtin_amdgcn_perm(q1[u][grp], q0[u][grp], dsel));
                    }
                float4_t r[B][NG];
#pragma unroll
                for (int u = 0; u < B; ++u)
#pragma unroll
                    for (int grp = 0; grp < NG; ++grp) {
                        const uint32_t w = __builtin_amdgcn_alignbit(q1[u][grp], q0[u][grp], qsh);
                        const uint32_t w8 = __builtin_amdgcn_alignbit(q1[u][grp], q0[u][grp], qsh + 8);
                        const uint4_t bq = {and_or(w, mlo, e1024), and_or(w, mhi, e64), and_or(w8, mlo, e1024),
                                            and_or(w8, mhi, e64)};
                        r[u][grp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xq[u], bitcast<half8_t>(bq), negs[u],
                                                                           0, 0, 0);
                    }
                if (rows == B) {
#pragma unroll
                    for (int u = 0; u < B; ++u)
#pragma unroll
                        for (int grp = 0; grp < NG; ++grp) acc[j][grp] += (float)dh[u][grp] * r[u][grp][0];
                } else {
#pragma unroll
                    for (int u = 0; u < B; ++u)
#pragma unroll
                        for (int grp = 0; grp < NG; ++grp)
                            if (u < rows) acc[j][grp] += (float)dh[u][grp] * r[u][grp][0];
                }
                // All reads of this slot are done before the next iteration refills it.
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                slot = slot + 1 == R ? 0 : slot + 1;
                ++k;
            }
        }
    }

    // Partials (lanes 0..15 hold column 16 grp + lane), then the ordered wave sum.
    if (!SEPRED) __syncthreads();                 // every wave's last slot is read
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (j < ntl)
#pragma unroll
                for (int grp = 0; grp < NG; ++grp)
                    red[(j * NW + wave) * TW + grp * 16 + lane] = nbm > 0 ? acc[j][grp] : 0.f;
    }
    lds_barrier();
    for (int v = tid; v < ntl * TW; v += NW * 64) {
        const int j = v / TW, col = v % TW;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += red[(j * NW + w) * TW + col];
        if (GROUP || TW != 16 || wg + j * G != ntiles - 1 || col < a.tail_cols) yt[j][col] = (_Float16)s;
    }
}

static size_t gemv_lds_bytes(int R, int tpw, int xw, int nw, int tw) {
    const size_t ring = (size_t)nw * R * GV_SLOT, red = (size_t)tpw * nw * tw * sizeof(float);
    return (size_t)nw * xw + (tw == 16 ? ring + red : std::max(ring, red));
}

template <int R, int TPW, int NW, int TW, bool GROUP>
static hipError_t launch_gemv_g(const GemvArgs &a, int grid, hipStream_t s) {
    const size_t lds = gemv_lds_bytes(R, TPW, a.xw, NW, TW);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)q4_gemv_dma_kernel<R, TPW, NW, TW, GROUP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((q4_gemv_dma_kernel<R, TPW, NW, TW, GROUP>), dim3(grid), dim3(NW * 64), lds, s, a);
    return hipGetLastError();
}

// One weight (the drop-in call) or up to GV_GROUP_MAX weights sharing X.
template <int R, int TPW, int NW, int TW>
static hipError_t launch_gemv_t(const GemvArgs &a, int grid, hipStream_t s) {
    return a.ntiles > a.tiles_per_w ? launch_gemv_g<R, TPW, NW, TW, true>(a, grid, s)
                                    : launch_gemv_g<R, TPW, NW, TW, false>(a, grid, s);
}

template <int R, int NW>
static hipError_t launch_gemv_r(const GemvArgs &a, int grid, int tpw, hipStream_t s) {
    switch (tpw) {
        case 1: return launch_gemv_t<R, 1, NW, 16>(a, grid, s);
        case 2: return launch_gemv_t<R, 2, NW, 16>(a, grid, s);
        case 3: return launch_gemv_t<R, 3, NW, 16>(a, grid, s);
        default: return launch_gemv_t<R, 4, NW, 16>(a, grid, s);
    }
}

// True when the M == 1 kernel applies: 16-byte aligned weights and
// activations, 18*N a multiple of 16 (N % 8 == 0), at least one whole 16-column
// tile and K <= 16384.
bool gemv_dma_supported(const _Float16 *X, const uint8_t *W, int64_t K, int64_t N) {
    if (opt_is("MCQ4_GEMV_PATH", 'o')) return false;   // "off": use the batched decode kernel
    return N % 8 == 0 && N >= 16 && ((uintptr_t)W % 16) == 0 &&
           ((uintptr_t)X % 16) == 0 && K >= QK && K <= GV_K_MAX &&
           N * 18 * 8 < ((int64_t)1 << 31);
}

// Launches the M == 1 kernel for `count` weights of the same shape that share
// X (count <= GV_GROUP_MAX; with count > 1, N % 16 == 0) over their whole
// 16-column tiles (64-column tiles when N % 64 == 0 and the weights hold 1024 or
// more of them); *n_done returns the number of leading columns of each weight
// covered.
bool gemv_span_supported(const _Float16 *X, int64_t ldx, const uint8_t *W, int64_t M, int64_t K, int64_t N);
hipError_t launch_gemv_span(const _Float16 *X, int64_t ldx, const uint8_t *W, _Float16 *Y, int64_t ldy, int M,
                            int K, int N, hipStream_t s);

hipError_t launch_gemv_dma_group(const _Float16 *X, const uint8_t *const *W, _Float16 *const *Y, int count,
                                 int K, int N, int *n_done, hipStream_t s) {
    if (count < 1 || count > GV_GROUP_MAX || (count > 1 && N % 16)) return hipErrorInvalidValue;
    // One weight with 4096 < N <= 16384 at K <= 4096: contiguous spans of 1..4
    // 16-column groups per workgroup (q4_gemv_span.hip).
    if (count == 1 && gemv_span_supported(X, K, W[0], 1, K, N)) {
        *n_done = N;
        return launch_gemv_span(X, K, W[0], Y[0], N, 1, K, N, s);
    }
    GemvArgs a;
    a.X = X;
    for (int g = 0; g < GV_GROUP_MAX; ++g) {
        a.W[g] = W[g < count ? g : 0];
        a.Y[g] = Y[g < count ? g : 0];
    }
    a.nb = K / QK; a.N = N;
    if (N % GV_WIDE == 0 && count * (N / GV_WIDE) >= GV_WIDE_MIN_TILES) {
        // Eight-wave workgroups of four 64-column tiles, two per CU (N = 128256:
        // 50.0-50.3 us against 54.6-54.8 us with 16-column tiles, same box).
        constexpr int B = GV_ITEM / (GV_WIDE * BLOCK_BYTES);
        a.tiles_per_w = N / GV_WIDE;
        a.ntiles = count * a.tiles_per_w;
        a.nbt = (a.nb + B - 1) / B;
        *n_done = N;
        const int grid = (a.ntiles + GV_TPW_MAX - 1) / GV_TPW_MAX;
        a.xw = ((a.nbt + 7) / 8) * B * 64;
        return launch_gemv_t<GV_RING, GV_TPW_MAX, 8, GV_WIDE>(a, grid, s);
    }
    constexpr int B = GV_ITEM / (16 * BLOCK_BYTES);
    // One weight with N % 16 == 8: a last tile of 8 columns (the copies stay
    // inside each row, N % 8 == 0 keeps its 144 bytes whole chunks).
    a.tiles_per_w = count == 1 ? (N + 15) / 16 : N / 16;
    a.tail_cols = count == 1 && N % 16 ? N % 16 : 16;
    a.ntiles = count * a.tiles_per_w;
    a.nbt = (a.nb + B - 1) / B;
    *n_done = count == 1 ? N : a.tiles_per_w * 16;
    // One 16-wave workgroup per CU and up to GV_TPW_MAX tiles each.  Larger N
    // (more than 1024 tiles) runs 8-wave workgroups of GV_TPW_MAX tiles, two per
    // CU, backfilled as they finish (16-column tiles at N = 128256: 56 vs 66 us
    // with 16 waves; 16 waves stay faster on the layer shapes).
#ifndef GV_NW_SET
    const int nw = a.ntiles > 256 * GV_TPW_MAX ? 8 : 16;
#else
    const int nw = GV_NW_SET;
#endif
    const int per_round = nw == 16 ? 256 : 512;
    int grid = std::min(a.ntiles, per_round);
    if (a.ntiles > per_round * GV_TPW_MAX) grid = (a.ntiles + GV_TPW_MAX - 1) / GV_TPW_MAX;
    const int tpw = (a.ntiles + grid - 1) / grid;
    a.xw = ((a.nbt + nw - 1) / nw) * B * 64;                      // my batches' activations
    if (nw == 8) return launch_gemv_r<GV_RING, 8>(a, grid, tpw, s);
    return launch_gemv_r<GV_RING, 16>(a, grid, tpw, s);
}

// The single-weight form: the whole 16-column tiles of W (64-column tiles for
// N >= 65536, N % 64 == 0); *n_done returns the number of leading columns covered.
hipError_t launch_gemv_dma(const _Float16 *X, const uint8_t *W, _Float16 *Y, int K, int N,
                           int *n_done, hipStream_t s) {
    return launch_gemv_dma_group(X, &W, &Y, 1, K, N, n_done, s);
}

}  // namespace mcq4
