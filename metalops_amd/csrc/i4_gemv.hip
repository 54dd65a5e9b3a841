// Decode-shaped (M <= 16) per-group INT4 matmul on gfx950: MFMA GEMV.
//
// Y[M][N] = X[M][K] @ W with W[k][n] = (q - z) * s per (group, column),
// packed[K/2][N] (byte row k/2, even k low nibble), fp16 activations, fp32
// accumulation.  The kernel streams the 0.5 byte/weight nibble array once from
// HBM, so its roofline is HBM bandwidth.
//
// Work decomposition
//   * Tile = 16*NC columns (128 by default); step = 32 K rows (16 byte rows of
//     the tile).  Workgroup (tile t, split sp) = IW waves; wave w owns the
//     steps [(sp*IW + w)*spw, +spw).  Waves of a workgroup are summed through
//     LDS in wave order; when K is split, splits are summed through the
//     workspace by the last-arriving workgroup of the tile in split order
//     (deterministic).
//   * Lane (c = l%16, g = l/16): columns NC*c..NC*c+NC-1 of the tile, byte rows
//     4g..4g+3 of the step (K elements 8g..8g+7), activation row min(c, M-1).
//     Per step it loads four NC-byte weight rows and 16 bytes of activations
//     into a register ring D steps ahead (loads past the range are clamped
//     to the last step so every step issues the same five loads).
//   * B operand of virtual MFMA column c (actual column NC*c + j for the j-th
//     of the NC 16x16x32 MFMAs): per byte row r, one v_perm_b32 moves the byte
//     of column NC*c+j and the same byte shifted right by 4 into bytes 0 and 2,
//     one v_and_or_b32 keeps the two nibbles and adds the 0x64 exponent bytes:
//     the fp16 pair {1024 + q(2r), 1024 + q(2r+1)}.  The activations are the
//     natural MFMA A operand (row m = l%16, K elements 8g..8g+7).
//   * Per group: P_j = sum x*(1024 + q) (MFMA chain), S = sum x (MFMA against
//     ones); at the group's last step (or the range end)
//       acc_j += s_j * (P_j - (1024 + z_j) * S)
//     in fp32 -- i.e. sum x*(q - z)*s.  The group's scales and zeros (one row
//     of the tile per group) are copied to LDS by global_load_lds before the
//     first weight load, so they have landed once the first step's weights
//     have; the flush reads them with ds_read after an explicit vmcnt wait that
//     leaves only the ring's newer loads pending.
//   * Store: act(sum) rounded to fp16.
//
// MFMA 16x16x32 f16 layout: A lane l = row l%16, K 8(l/16)..+8; B lane l =
// column l%16, K 8(l/16)..+8; D lane l = rows 4(l/16)+i, column l%16.
#include <algorithm>
#include <stdlib.h>
#include <atomic>
#include <type_traits>

#include "i4_common.h"

namespace mcq4 {

MCQ4_SPLIT_FALLBACK_COUNTER(i4_gemv_split_fallbacks)

// Two tile shapes (template NC = weight columns per lane):
//   * NC = 8: 128-column tiles (128-byte row pieces), 4 waves per workgroup,
//     K split over workgroups.  Default.
//   * NC = 4: 64-column tiles, 16 waves per workgroup, the whole K range of a
//     tile in one workgroup when the scale/zero slots allow.  Selectable.
constexpr int I4V_LPS = 5;                // vector-memory loads per step
constexpr int I4V_GMAX = 8;               // groups per wave held in LDS
constexpr int I4V_SMAX = 16;              // K splits at most

template <int NC, int IW_ = (NC == 8 ? 4 : 16)>
struct I4vShape {
    static constexpr int IW = IW_;                              // waves per workgroup
    static constexpr int TC = 16 * NC;                          // tile columns
    static constexpr int SLOT = TC * 4 * 2;                     // fp32 scales + zeros of a tile row
    static constexpr int SZ_BYTES = IW * I4V_GMAX * SLOT;
    static constexpr int RED_BYTES = IW * 16 * TC * 4;
    static constexpr int LDS = SZ_BYTES > RED_BYTES ? SZ_BYTES : RED_BYTES;
};

struct I4GemvArgs {
    const _Float16 *X;
    int64_t ldx;
    const uint8_t *P;
    const void *scales, *zeros;
    _Float16 *Y;
    int64_t ldy;
    int M, N, nsteps, spg;    // spg = steps per group (group_size / 32)
    int spw, S;               // steps per wave, splits (grid.y)
    float *part;              // [tiles][S][M][TC] when S > 1
    uint32_t *counters;       // [tiles]; with xl, 64-bit tickets [8][4096] by blockIdx.x mod 8
    int xl;                   // XCD-local split exchange (grid.x a multiple of 8)
    uint32_t foreign;         // splits treated as run on another XCD (test switch)
};

// Scales and zeros of the lane's NC columns (fp32 slot layout: TC scales then
// TC zeros; 16-bit layouts: TC scales then TC zeros at half the size).
template <int SZ, int NC>
__device__ __forceinline__ void i4v_load_sz(const lds_u8 *slot, int c, float (&s)[NC],
                                            float (&z)[NC]) {
    constexpr int TC = 16 * NC;
    if constexpr (SZ == DT_F32) {
        typedef __attribute__((address_space(3))) float4_t lds_f4;
        const lds_f4 *sp = (const lds_f4 *)(slot + 4 * NC * c);
        const lds_f4 *zp = (const lds_f4 *)(slot + 4 * TC + 4 * NC * c);
#pragma unroll
        for (int h = 0; h < NC / 4; ++h) {
            const float4_t sv = sp[h], zv = zp[h];
#pragma unroll
            for (int i = 0; i < 4; ++i) { s[4 * h + i] = sv[i]; z[4 * h + i] = zv[i]; }
        }
    } else {
        uint32_t sv[NC / 2], zv[NC / 2];
        if constexpr (NC == 8) {
            const uint4_t a = *(const __attribute__((address_space(3))) uint4_t *)(slot + 2 * NC * c);
            const uint4_t b = *(const __attribute__((address_space(3))) uint4_t *)(slot + 2 * TC + 2 * NC * c);
#pragma unroll
            for (int i = 0; i < 4; ++i) { sv[i] = a[i]; zv[i] = b[i]; }
        } else {
            const u32x2 a = *(const __attribute__((address_space(3))) u32x2 *)(slot + 2 * NC * c);
            const u32x2 b = *(const __attribute__((address_space(3))) u32x2 *)(slot + 2 * TC + 2 * NC * c);
#pragma unroll
            for (int i = 0; i < 2; ++i) { sv[i] = a[i]; zv[i] = b[i]; }
        }
#pragma unroll
        for (int i = 0; i < NC / 2; ++i) {
            if constexpr (SZ == DT_F16) {
                const half2_t sh = bitcast<half2_t>(sv[i]), zh = bitcast<half2_t>(zv[i]);
                s[2 * i] = (float)sh[0]; s[2 * i + 1] = (float)sh[1];
                z[2 * i] = (float)zh[0]; z[2 * i + 1] = (float)zh[1];
            } else {
                s[2 * i] = __uint_as_float(sv[i] << 16); s[2 * i + 1] = __uint_as_float(sv[i] & 0xFFFF0000u);
                z[2 * i] = __uint_as_float(zv[i] << 16); z[2 * i + 1] = __uint_as_float(zv[i] & 0xFFFF0000u);
            }
        }
    }
}

template <int NC> struct WRow;
template <> struct WRow<8> { typedef u32x2 T; };
template <> struct WRow<4> { typedef uint32_t T; };

// WB = weight bits: 4 (packed[K/2][N], 32 K per step, 16x16x32 MFMA) or 8
// (int8 [K][N], 16 K per step, 16x16x16 MFMA).  A step is 16 byte rows of the
// tile in both formats.
template <int SZ, int ACT, int D, int NC, int WB, int IWT>
__global__ void __launch_bounds__(IWT * 64) __attribute__((amdgpu_waves_per_eu(3)))
i4_gemv_kernel(I4GemvArgs a) {
    typedef I4vShape<NC, IWT> Shape;
    constexpr int IW = Shape::IW, TC = Shape::TC, SLOT = Shape::SLOT;
    constexpr int KS = WB == 4 ? 32 : 16;                // K per step
    constexpr float OFF = WB == 4 ? 1024.0f : 1152.0f;  // fp16 value of code 0 in the B operand
    typedef typename std::conditional<WB == 4, uint4_t, u32x2>::type xv_t;
    typedef typename WRow<NC>::T wrow_t;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];    // Shape::LDS bytes
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    // Consecutive tiles (which share 128-byte lines when TC = 64) go to one XCD.
    const int G = (int)gridDim.x, G8 = G & ~7;
    int t = (int)blockIdx.x;
    if (t < G8) t = (t & 7) * (G8 >> 3) + (t >> 3);
    const int sp = (int)blockIdx.y;
    const int N = a.N;
    const int col0 = t * TC;
    if (a.xl && col0 >= N) return;                       // grid padding to a multiple of 8

    const int s_begin = (sp * IW + wave) * a.spw;
    const int ns = max(0, min(a.spw, a.nsteps - s_begin));

    float4_t acc[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (ns > 0) {
        // ---- scales / zeros of the wave's groups -> LDS (one copy per group) ----
        const int g_first = s_begin / a.spg;
        const int ngr = (s_begin + ns - 1) / a.spg - g_first + 1;     // <= I4V_GMAX by launch
        uint8_t *szw = smem + wave * (I4V_GMAX * SLOT);
        {
            constexpr int esz = SZ == DT_F32 ? 4 : 2;
            constexpr int per_lane = 16 / esz;                         // elements per lane copy
            constexpr int lanes_per_row = TC / per_lane;
            const bool is_z = lane >= lanes_per_row;
            const int li = is_z ? lane - lanes_per_row : lane;
            int col = col0 + li * per_lane;
            if (col >= N) col = 0;                                     // valid, never read back
            const uint8_t *src = (const uint8_t *)(is_z ? a.zeros : a.scales) + (int64_t)col * esz;
            for (int gl = 0; gl < ngr; ++gl) {
                if (lane < 2 * lanes_per_row)
                    __builtin_amdgcn_global_load_lds(
                        (void *)(src + (int64_t)(g_first + gl) * N * esz),
                        (__attribute__((address_space(3))) void *)(szw + gl * SLOT), 16, 0, 0);
            }
        }

        // ---- register ring of weight rows and activations ----
        const int ncol = col0 + NC * c < N ? col0 + NC * c : 0;
        const uint8_t *wbase = a.P + (int64_t)(s_begin * 16 + 4 * g) * N + ncol;
        const int m = min(c, a.M - 1);
        const _Float16 *xbase = a.X + (int64_t)m * a.ldx + (int64_t)s_begin * KS + (KS / 4) * g;
        wrow_t wr[D][4];
        xv_t xr[D];
        auto load_step = [&](int j, wrow_t (&w)[4], xv_t &x) {
            const uint8_t *p = wbase + (int64_t)j * 16 * N;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                w[r] = __builtin_nontemporal_load((const wrow_t *)(p + (int64_t)r * N));
            x = *(const xv_t *)(xbase + (int64_t)j * KS);
        };
#pragma unroll
        for (int d = 0; d < D; ++d) load_step(min(d, ns - 1), wr[d], xr[d]);
        // The scale/zero copies are older than the ring's loads: retire them
        // here, once, so no ds_read below waits on an LDS copy in flight.
        wait_vmcnt<D * I4V_LPS>();

        const uint32_t c64 = opaque_vgpr(0x64006400u);
        const uint32_t mlo = opaque_sgpr(0x000F000Fu);
        const half8_t ones = bitcast<half8_t>(uint4_t{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
        const half4_t ones4 = bitcast<half4_t>(u32x2{0x3C003C00u, 0x3C003C00u});
        const float4_t zf = {0.f, 0.f, 0.f, 0.f};
        float4_t P[NC], Ssum = zf;
#pragma unroll
        for (int j = 0; j < NC; ++j) P[j] = zf;

        auto step = [&](const wrow_t (&w)[4], const xv_t &xv) {
            if constexpr (WB == 8) {
                // int8: B pair of K rows 2p, 2p+1 (p = 0, 1) for column NC*c + j:
                // bytes to positions 0 and 2, then the xor flips the sign bit
                // (q + 128) and sets the 0x64 exponent bytes: fp16 1152 + q.
                const half4_t x = bitcast<half4_t>(xv);
#pragma unroll
                for (int j = 0; j < NC; ++j) {
                    const int h = j >> 2, b = j & 3;
                    const uint32_t sel = (uint32_t)b | 0x0Cu << 8 | (uint32_t)(4 + b) << 16 | 0x0Cu << 24;
                    u32x2 bq;
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        uint32_t r0, r1;
                        if constexpr (NC == 8) { r0 = w[2 * p][h]; r1 = w[2 * p + 1][h]; }
                        else { r0 = w[2 * p]; r1 = w[2 * p + 1]; }
                        bq[p] = __builtin_amdgcn_perm(r1, r0, sel) ^ 0x64806480u;
                    }
                    P[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(x, bitcast<half4_t>(bq), P[j], 0, 0, 0);
                }
                Ssum = __builtin_amdgcn_mfma_f32_16x16x16f16(x, ones4, Ssum, 0, 0, 0);
                return;
            } else {
            const half8_t x = bitcast<half8_t>(xv);
            uint32_t lo[4][NC / 4], hi[4][NC / 4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int h = 0; h < NC / 4; ++h) {
                    if constexpr (NC == 8) lo[r][h] = w[r][h];
                    else lo[r][h] = w[r];
                    hi[r][h] = lo[r][h] >> 4;
                }
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int h = j >> 2, b = j & 3;
                const uint32_t sel = (uint32_t)b | (uint32_t)b << 8 | (uint32_t)(4 + b) << 16 |
                                     (uint32_t)(4 + b) << 24;
                uint4_t bq;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    bq[r] = and_or(__builtin_amdgcn_perm(hi[r][h], lo[r][h], sel), mlo, c64);
                P[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, bitcast<half8_t>(bq), P[j], 0, 0, 0);
            }
            Ssum = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, ones, Ssum, 0, 0, 0);
            }
        };
        auto flush = [&](int gl) {
            float sv[NC], zv[NC];
            i4v_load_sz<SZ, NC>(lds_ptr(lds_addr(szw + gl * SLOT)), c, sv, zv);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const float zz = -(OFF + zv[j]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float tq = __builtin_fmaf(zz, Ssum[i], P[j][i]);
                    acc[j][i] = __builtin_fmaf(sv[j], tq, acc[j][i]);
                }
                P[j] = zf;
            }
            Ssum = zf;
        };

        // Whole blocks of D steps with unconditional (clamped) loads, so the
        // compiler's waits count exactly; then the < D remaining steps,
        // whose data is already in the ring.
        int j0 = 0;
        for (; j0 + D <= ns; j0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int j = j0 + u;
                step(wr[u], xr[u]);
                load_step(min(j + D, ns - 1), wr[u], xr[u]);
                const int sg = s_begin + j;
                if ((sg + 1) % a.spg == 0 || j == ns - 1) flush(sg / a.spg - g_first);
            }
        }
        wait_vmcnt<0>();
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int j = j0 + u;
            if (j < ns) {
                step(wr[u], xr[u]);
                const int sg = s_begin + j;
                if ((sg + 1) % a.spg == 0 || j == ns - 1) flush(sg / a.spg - g_first);
            }
        }
        wait_vmcnt<0>();
    }

    // ---- wave partials -> LDS, ordered sum over waves ----
    __syncthreads();                              // all waves done with their s/z slots
    float *red = (float *)smem;                   // [IW][16][TC]
    const int M = a.M;
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * g + i;
            if (row < M) red[(wave * 16 + row) * TC + NC * c + j] = acc[j][i];
        }
    __syncthreads();
    if (a.S == 1) {
        for (int v = tid; v < M * TC; v += IW * 64) {
            const int row = v / TC, cl = v % TC;
            if (col0 + cl >= N) continue;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < IW; ++w) sum += red[(w * 16 + row) * TC + cl];
            a.Y[(int64_t)row * a.ldy + col0 + cl] = (_Float16)activate<ACT>(sum);
        }
        return;
    }
    // Split K: this workgroup's partial goes out with write-through stores
    // (agent-scope relaxed atomic stores: global_store sc1), and once they are
    // acknowledged (vmcnt(0)) one lane takes a ticket on the tile's counter.
    // The workgroup that draws the last ticket reads every split's partial with
    // L2-bypassing loads (agent-scope atomic loads: sc1) in split order.  This
    // keeps the cross-XCD exchange to the partials themselves instead of the
    // full-L2 write-back and invalidate that an agent-scope fence costs.
    float *part = a.part + ((int64_t)t * a.S + sp) * M * TC;
    if (a.xl) {
        // Every split of this tile runs on this XCD: the partials go through its
        // L2 (plain stores, L1-bypassing loads); the ticket records each split's
        // XCD, and a split found elsewhere is recomputed (q4_common.h).
        uint64_t *cnt = (uint64_t *)a.counters + ((int)blockIdx.x & 7) * 4096 + ((int)blockIdx.x >> 3);
        const uint32_t xcc = xcc_id();
        for (int v = tid; v < M * TC; v += IW * 64) {
            const int row = v / TC, cl = v % TC;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < IW; ++w) sum += red[(w * 16 + row) * TC + cl];
            part[v] = sum;
        }
        wait_vmcnt<0>();
        __syncthreads();
        uint32_t *last_flag = (uint32_t *)smem;
        if (tid == 0) {
            const uint64_t inc = xcd_ticket_inc(xcc, sp);
            const uint64_t prev = __hip_atomic_fetch_add(cnt, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t local = xcd_ticket_local_mask(prev + inc, xcc, a.S) & ~a.foreign;
            *last_flag = (prev & 0xFF) != (uint64_t)(a.S - 1) ? 0u : 0x10000u | local;
            if ((prev & 0xFF) == (uint64_t)(a.S - 1)) {
                // Every split has drawn: the slot is free for the next launch now,
                // so its reset overlaps the sum instead of trailing it.
                __hip_atomic_store(cnt, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (local != (1u << a.S) - 1) note_split_fallback();
            }
        }
        __syncthreads();
        const uint32_t lf = *last_flag;
        if (!lf) return;
        const uint32_t local = lf & 0xFFFF;        // splits whose partial is in this L2
        const float *base = a.part + (int64_t)t * a.S * M * TC;
        for (int v = tid; v < M * TC; v += IW * 64) {
            const int row = v / TC, cl = v % TC;
            float sum = 0.f;
            for (int q0 = 0; q0 < a.S; q0 += 8) {
                float pv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pv[i] = load_l2_f32(base, (min(q0 + i, a.S - 1) * M * TC + v) * 4);
                if (local != (1u << a.S) - 1 && col0 + cl < N) {   // splits from another XCD: recompute
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (q0 + i < a.S && !((local >> (q0 + i)) & 1))
                            pv[i] = i4_dot_range<WB>(a.X + (int64_t)row * a.ldx, a.P, a.scales, a.zeros, SZ, N,
                                                     a.spg * KS, col0 + cl,
                                                     min((q0 + i) * IW * a.spw, a.nsteps) * KS,
                                                     min((q0 + i + 1) * IW * a.spw, a.nsteps) * KS);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (q0 + i < a.S) sum += pv[i];
            }
            if (col0 + cl < N) a.Y[(int64_t)row * a.ldy + col0 + cl] = (_Float16)activate<ACT>(sum);
        }
        return;
    }
    for (int v = tid; v < M * TC; v += IW * 64) {
        const int row = v / TC, cl = v % TC;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < IW; ++w) sum += red[(w * 16 + row) * TC + cl];
        __hip_atomic_store(part + v, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmcnt<0>();
    __syncthreads();                              // red is dead from here: its first word holds the flag
    uint32_t *last_flag = (uint32_t *)smem;
    if (tid == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(&a.counters[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last_flag = prev == (uint32_t)(a.S - 1) ? 1u : 0u;
        if (prev == (uint32_t)(a.S - 1)) __hip_atomic_store(&a.counters[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last_flag) return;
    const float *base = a.part + (int64_t)t * a.S * M * TC;
    for (int v = tid; v < M * TC; v += IW * 64) {
        const int row = v / TC, cl = v % TC;
        // Eight independent loads in flight at a time (clamped indices, summed
        // in split order), not one memory round trip per split.
        float sum = 0.f;
        for (int q0 = 0; q0 < a.S; q0 += 8) {
            float pv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                pv[i] = __hip_atomic_load(base + (int64_t)min(q0 + i, a.S - 1) * M * TC + v,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (q0 + i < a.S) sum += pv[i];
        }
        if (col0 + cl < N) a.Y[(int64_t)row * a.ldy + col0 + cl] = (_Float16)activate<ACT>(sum);
    }
}

struct I4GemvCfg {
    int nc, iw, spw, S;
};

// Tile shape and K split.  Default: 128-column tiles of 4 waves, one workgroup
// per CU: S = the most K splits that keep the grid within 256 workgroups (2..32
// steps per wave, at most I4V_SMAX splits).  Graph replays, us: INT4 M=16
// 4096x14336 15.3 (the previous aim of about 1024 waves gave 336 workgroups:
// 18.6), M=4 11.7 (13.7); INT8 M=16 4096x14336 21.2 (25.3); 14336x4096 and
// 4096x4096 were already at 256 workgroups.  A
// wave's steps must fit its I4V_GMAX scale/zero slots: a range of spw steps
// touches at most ceil(spw/spg) + 1 groups, or exactly spw/spg when spw is a
// multiple of spg (every range then starts on a group boundary).
// (64-column tiles of 16 waves with the whole K in one workgroup were measured
// slower: 64-byte row pieces read at about half the bandwidth of 128-byte
// pieces on MI355X.)
static I4GemvCfg i4_gemv_config(int64_t K, int64_t N, int64_t gs, int ks) {
    const int64_t nsteps = K / ks, spg = gs / ks;
    const int64_t loose = (I4V_GMAX - 1) * spg;          // any alignment
    auto fit = [&](int64_t w) {
        if (w <= loose) return w;
        return std::min<int64_t>((w + spg - 1) / spg * spg, I4V_GMAX * spg);
    };
    const int nc = 8;
    const int64_t iw = 4;
    const int64_t ntiles = (N + 16 * nc - 1) / (16 * nc);
    int64_t S = std::max<int64_t>(1, std::min<int64_t>(I4V_SMAX, 256 / ntiles));
    S = std::max(S, (nsteps + iw * 32 - 1) / (iw * 32));
    {
        int64_t spw = (nsteps + iw * S - 1) / (iw * S);
        spw = std::max<int64_t>(spw, (nsteps + iw * I4V_SMAX - 1) / (iw * I4V_SMAX));
        spw = fit(std::min<int64_t>(std::max<int64_t>(spw, 2), 32));
        S = (nsteps + iw * spw - 1) / (iw * spw);
    }
    int64_t spw = fit((nsteps + iw * S - 1) / (iw * S));
    S = (nsteps + iw * spw - 1) / (iw * spw);
    return {nc, (int)iw, (int)spw, (int)S};
}

// wb = weight bits (4: packed[K/2][N]; 8: int8 [K][N]).
bool i4_gemv_supported(int64_t M, int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                       const void *P, const void *scales, const void *zeros, int wb) {
    const int ks = wb == 4 ? 32 : 16;
    return M >= 1 && M <= 16 && K % ks == 0 && gs % ks == 0 && N % 8 == 0 &&
           (N + 63) / 64 <= COUNTER_SLOTS && ldx % 8 == 0 && ((uintptr_t)X % 16) == 0 &&
           ((uintptr_t)P % 8) == 0 && ((uintptr_t)scales % 16) == 0 &&
           ((uintptr_t)zeros % 16) == 0 && K / 32 < (1 << 24);
}

size_t i4_gemv1_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t gs);
bool i4_gemv1_supported(int64_t M, int64_t K, int64_t N, int64_t gs, const void *X, int64_t ldx,
                        const void *P, const void *scales, const void *zeros, int wb);
hipError_t launch_i4_gemv1(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                           const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K, int N, int gs,
                           int act, void *ws, hipStream_t s, int wb);

// Covers both decode kernels (i4_gemv1 when it applies, this one otherwise).
size_t i4_gemv_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t gs, int wb) {
    const I4GemvCfg c = i4_gemv_config(K, N, gs, wb == 4 ? 32 : 16);
    const int64_t tc = 16 * c.nc;
    size_t need = c.S == 1 ? 0 : COUNTER_BYTES + (size_t)((N + tc - 1) / tc) * c.S * M * tc * sizeof(float);
    if (M <= (wb == 4 ? 32 : 16) && K % 32 == 0 && gs % 32 == 0 && N % 128 == 0)
        need = std::max(need, i4_gemv1_workspace_bytes(M, K, N, gs));
    return need;
}

// Launches one instance; raises its dynamic-LDS limit once per device when the
// shape needs more than the default 64 KiB.
template <int SZ, int ACT, int D, int NC, int WB, int IW>
static hipError_t launch_one(const I4GemvArgs &a, dim3 grid, hipStream_t s) {
    constexpr size_t lds = I4vShape<NC, IW>::LDS;
    if (lds > 64 * 1024) {
        static std::atomic<uint64_t> done{0};
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        const uint64_t bit = 1ull << (dev & 63);
        if (!(done.load(std::memory_order_acquire) & bit)) {
            e = hipFuncSetAttribute((const void *)i4_gemv_kernel<SZ, ACT, D, NC, WB, IW>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
            done.fetch_or(bit, std::memory_order_acq_rel);
        }
    }
    hipLaunchKernelGGL((i4_gemv_kernel<SZ, ACT, D, NC, WB, IW>), grid, dim3(IW * 64), lds, s, a);
    return hipSuccess;
}

template <int SZ, int D, int NC, int WB, int IW>
static hipError_t launch_gemv_sz(const I4GemvArgs &a, int ntiles, int act, hipStream_t s) {
    const dim3 grid(a.xl ? (ntiles + 7) / 8 * 8 : ntiles, a.S);
    hipError_t e;
    if (act == ACT_SILU) e = launch_one<SZ, ACT_SILU, D, NC, WB, IW>(a, grid, s);
    else if (act == ACT_GELU) e = launch_one<SZ, ACT_GELU, D, NC, WB, IW>(a, grid, s);
    else e = launch_one<SZ, ACT_NONE, D, NC, WB, IW>(a, grid, s);
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

template <int NC, int WB, int IW>
static hipError_t launch_gemv_nc(const I4GemvArgs &a, int ntiles, int sz_dt, int act, hipStream_t s) {
    if (sz_dt == DT_F32) return launch_gemv_sz<DT_F32, 4, NC, WB, IW>(a, ntiles, act, s);
    if (sz_dt == DT_F16) return launch_gemv_sz<DT_F16, 4, NC, WB, IW>(a, ntiles, act, s);
    return launch_gemv_sz<DT_BF16, 4, NC, WB, IW>(a, ntiles, act, s);
}

hipError_t launch_i4_gemv(const _Float16 *X, int64_t ldx, const uint8_t *P, const void *scales,
                          const void *zeros, int sz_dt, _Float16 *Y, int64_t ldy, int M, int K,
                          int N, int gs, int act, void *ws, hipStream_t s, int wb) {
    const int ks = wb == 4 ? 32 : 16;
    // The async-copy GEMV (i4_gemv1.hip) when its shape rules hold.
    if (ldx >= K && i4_gemv1_supported(M, K, N, gs, X, ldx, P, scales, zeros, wb))
        return launch_i4_gemv1(X, ldx, P, scales, zeros, sz_dt, Y, ldy, M, K, N, gs, act, ws, s, wb);
    const I4GemvCfg c = i4_gemv_config(K, N, gs, ks);
    I4GemvArgs a;
    a.X = X; a.ldx = ldx; a.P = P; a.scales = scales; a.zeros = zeros; a.Y = Y; a.ldy = ldy;
    a.M = M; a.N = N; a.nsteps = K / ks; a.spg = gs / ks;
    a.spw = c.spw; a.S = c.S;
    a.part = nullptr; a.counters = nullptr; a.foreign = split_foreign_mask();
    const int ntiles = (N + 16 * c.nc - 1) / (16 * c.nc);
    a.xl = 0;
    if (c.S > 1) {
        if (!ws) return hipErrorInvalidValue;
        a.part = (float *)((char *)ws + COUNTER_BYTES);
        a.counters = (uint32_t *)ws;
        a.xl = !opt_is("MCQ4_XCD_LOCAL", '0') && (ntiles + 7) / 8 <= 4096;
    }
    if (wb == 8) return launch_gemv_nc<8, 8, 4>(a, ntiles, sz_dt, act, s);
    return launch_gemv_nc<8, 4, 4>(a, ntiles, sz_dt, act, s);
}

}  // namespace mcq4
