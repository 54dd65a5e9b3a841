// Shared definitions for the gfx950 block_q4_0 kernels.
//
// Block format (metalcore quantization.py:296-304, native/quant_kernels.metal:1703-1710):
// 18 bytes = fp16 scale d + 16 bytes of nibbles; byte i holds element 2i (low
// nibble) and element 2i+1 (high nibble).  Tensor layout [K/32][N][18]: the
// blocks of adjacent output columns are contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mcq4_options.h"

namespace mcq4 {

constexpr int QK = 32;       // weights per block
constexpr int BLOCK_BYTES = 18;

// Split-K workspace layout shared by both matmul kernels: a fixed area of
// per-tile arrival counters at offset 0 (zero on first use, left zero by every
// call), then the fp32 partials.  Fixing the counter area's place and size keeps
// a call's partials from ever landing where a later call, of any shape, looks
// for its counters.
constexpr int64_t COUNTER_SLOTS = 65536;
constexpr size_t COUNTER_BYTES = COUNTER_SLOTS * sizeof(uint32_t);

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

// Explicit LDS (address space 3) views: a 32-bit LDS address kept in a VGPR
// and dereferenced through these types compiles to ds_read with immediate
// offsets.
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) half8_t lds_half8;
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const lds_u8 *)p;
}
__device__ __forceinline__ const lds_u8 *lds_ptr(uint32_t addr) {
    return (const lds_u8 *)(uintptr_t)addr;
}

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From &f) {
    static_assert(sizeof(To) == sizeof(From), "size mismatch");
    return __builtin_bit_cast(To, f);
}

__device__ __forceinline__ int64_t imin64(int64_t x, int64_t y) { return x < y ? x : y; }

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}

// XCD-local split-K exchange.  gfx950 dispatches workgroup i of a grid to XCD
// (i + c) mod 8, c fixed per device, so workgroups whose linear ids agree mod 8
// share an XCD and its L2.  Partials exchanged among them can stay in that L2:
// plain stores (L1 is write-through), then L1-bypassing loads, instead of
// write-through stores and loads that go to memory.  The arrival ticket stays
// a device-coherent atomic.  Split sp adds 1 + (xcc << (8 + 3 sp)): bits 0..7
// count the arrivals and the 3-bit field of each split records the XCD it ran
// on (S <= 16 splits fit in 56 bits).  The last arrival reads the partials of
// the splits that ran on its own XCD from its L2; should the placement ever
// differ (another partition mode or part), a split from another XCD is not
// read -- its partial sits in that XCD's L2 -- but recomputed from the inputs
// by the last arrival itself, and the file's fallback counter is raised.
constexpr int XCD_SPLIT_MAX = 16;
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 7;
}
__host__ __device__ __forceinline__ uint64_t xcd_ticket_inc(uint32_t xcc, int sp) {
    return 1ull + ((uint64_t)xcc << (8 + 3 * sp));
}
// Bit q set when split q (< S) of the completed ticket `total` ran on XCD `xcc`.
__host__ __device__ __forceinline__ uint32_t xcd_ticket_local_mask(uint64_t total, uint32_t xcc, int S) {
    uint32_t m = 0;
    for (int q = 0; q < S; ++q)
        if (((total >> (8 + 3 * q)) & 7) == xcc) m |= 1u << q;
    return m;
}

// Per-file count of split-K tiles whose partials had to be recomputed (the
// placement above did not hold), readable from the host.  Each translation unit
// that uses the exchange instantiates it once with its reader's name.
#define MCQ4_SPLIT_FALLBACK_COUNTER(reader)                                                  \
    static __device__ unsigned long long g_split_fallbacks;                                  \
    __device__ __forceinline__ void note_split_fallback() {                                  \
        __hip_atomic_fetch_add(&g_split_fallbacks, 1ull, __ATOMIC_RELAXED,                   \
                               __HIP_MEMORY_SCOPE_AGENT);                                    \
    }                                                                                        \
    hipError_t reader(uint64_t *count, bool reset) {                                         \
        unsigned long long v = 0;                                                            \
        hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_split_fallbacks), sizeof(v));    \
        if (e == hipSuccess && reset) {                                                      \
            const unsigned long long z = 0;                                                  \
            e = hipMemcpyToSymbol(HIP_SYMBOL(g_split_fallbacks), &z, sizeof(z));             \
        }                                                                                    \
        *count += v;                                                                         \
        return e;                                                                            \
    }

// One output of the q4_0 product over K blocks [kb0, kb1): sum of x[k] times
// the fp16 weight (q - 8)*d, in fp32 -- the split-K recompute path of the
// exchange above (slow, taken only when a split ran on another XCD).
__device__ __forceinline__ float q4_dot_range(const _Float16 *xrow, const uint8_t *W, int N, int n,
                                                  int kb0, int kb1) {
    float acc = 0.f;
    for (int kb = kb0; kb < kb1; ++kb) {
        const uint16_t *b = (const uint16_t *)(W + ((int64_t)kb * N + n) * BLOCK_BYTES);
        const float d = (float)__builtin_bit_cast(_Float16, b[0]);
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = b[1 + i];
            for (int e = 0; e < 4; ++e) {
                const _Float16 wv = (_Float16)((float)((int)((w >> (4 * e)) & 0xF) - 8) * d);
                acc += (float)xrow[kb * QK + 4 * i + e] * (float)wv;
            }
        }
    }
    return acc;
}

// fp32 load at byte offset `off` from the workgroup-uniform `base`, bypassing
// L1 (sc0) so it is served by the XCD's L2.
__device__ __forceinline__ float load_l2_f32(const float *base, int off) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 1));
}

// Workgroup barrier that waits only for this wave's LDS traffic.  (__syncthreads
// also waits for all outstanding vector-memory operations, which would drain the
// async copies that are meant to stay in flight across the barrier; the explicit
// wait_vmcnt calls establish that the data consumed next has landed.)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// (x & mask) | bits.  With `mask` in an SGPR and `bits` in a VGPR (see
// opaque_sgpr / opaque_vgpr) this selects one v_and_or_b32; with literal
// constants gfx9 needs a separate v_and and v_or (VOP3 encodes no literal).
// Plain C on purpose: instructions written in inline asm are invisible to the
// compiler's MFMA hazard tracking, so an asm VALU write to a register that an
// in-flight MFMA will write gets clobbered.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bits) {
    return (x & mask) | bits;
}
__device__ __forceinline__ uint32_t opaque_sgpr(uint32_t v) {
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Eight nibbles (elements e0..e7 at bits 4e..4e+3 of `w`) -> fp16 halves
// 1024 + q in natural element order [e0..e7]: the even/odd nibble bytes are
// interleaved first, then each byte pair gets the 0x64 exponent byte.
__device__ __forceinline__ half8_t unpack8_1024_nat(uint32_t w) {
    const uint32_t C64 = 0x64646464u;
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t e03 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);   // e0 e1 e2 e3
    const uint32_t e47 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);   // e4 e5 e6 e7
    uint4_t r;
    r[0] = __builtin_amdgcn_perm(C64, e03, 0x04010400u);
    r[1] = __builtin_amdgcn_perm(C64, e03, 0x04030402u);
    r[2] = __builtin_amdgcn_perm(C64, e47, 0x04010400u);
    r[3] = __builtin_amdgcn_perm(C64, e47, 0x04030402u);
    return bitcast<half8_t>(r);
}

// Eight nibbles (elements e0..e7 at bits 4e..4e+3 of `w`, i.e. byte i holds
// e_{2i} low and e_{2i+1} high) and the fp16 bits of d -> eight fp16 weights
// (q-8)*d in the slot order [e0,e2,e4,e6,e1,e3,e5,e7].
//
// lo/hi isolate the even/odd nibbles one per byte; v_perm_b32 against a word
// of 0x64 bytes then builds fp16 halves 0x64qq = 1024 + q directly (one op per
// pair).  Subtracting 1032 gives q - 8 exactly, and one fp16 multiply by d
// gives the single nearest-even rounding of the exact product -- the value the
// reference's fp16 dequant produces (quantization.py:417-419: exact fp32
// product cast to fp16).
__device__ __forceinline__ half8_t dequant8_perm(uint32_t w, uint32_t dbits) {
#pragma clang fp contract(off)
    const uint32_t C64 = 0x64646464u;
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes e0 e2 e4 e6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes e1 e3 e5 e7
    const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t d2 = bitcast<half2_t>(__builtin_amdgcn_perm(dbits, dbits, 0x01000100u));
    half2_t p0 = (bitcast<half2_t>(__builtin_amdgcn_perm(C64, lo, 0x04010400u)) - off) * d2;
    half2_t p1 = (bitcast<half2_t>(__builtin_amdgcn_perm(C64, lo, 0x04030402u)) - off) * d2;
    half2_t p2 = (bitcast<half2_t>(__builtin_amdgcn_perm(C64, hi, 0x04010400u)) - off) * d2;
    half2_t p3 = (bitcast<half2_t>(__builtin_amdgcn_perm(C64, hi, 0x04030402u)) - off) * d2;
    half8_t r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// Eight nibbles (natural order e0..e7, byte i = e_{2i} | e_{2i+1} << 4) and the
// fp16 bits of d -> eight fp16 weights (q-8)*d in natural order: 1024 + q
// exactly via the 0x64 exponent byte, minus 1032 exactly, then one fp16
// multiply (the single rounding of the exact product, as the reference's fp16
// dequant).
__device__ __forceinline__ half8_t dequant8_nat(uint32_t w, half2_t d2) {
#pragma clang fp contract(off)
    const uint4_t u = bitcast<uint4_t>(unpack8_1024_nat(w));
    const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
    uint4_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = bitcast<uint32_t>((bitcast<half2_t>(u[i]) - off) * d2);
    return bitcast<half8_t>(r);
}

// Eight nibbles -> fp16 halves 1024 + q (exact) in the dequant8_perm slot order.
// Used where the -8 offset and the scale d are applied after the MFMA.
__device__ __forceinline__ half8_t unpack8_1024(uint32_t w) {
    const uint32_t C64 = 0x64646464u;
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    uint4_t r;
    r[0] = __builtin_amdgcn_perm(C64, lo, 0x04010400u);
    r[1] = __builtin_amdgcn_perm(C64, lo, 0x04030402u);
    r[2] = __builtin_amdgcn_perm(C64, hi, 0x04010400u);
    r[3] = __builtin_amdgcn_perm(C64, hi, 0x04030402u);
    return bitcast<half8_t>(r);
}

// Eight consecutive fp16 activations x0..x7 (as four dwords) reordered to the
// dequant8_perm slot order [x0,x2,x4,x6,x1,x3,x5,x7].
__device__ __forceinline__ half8_t perm_act8(uint4_t v) {
    uint4_t r;
    r[0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);  // x0, x2
    r[1] = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);  // x4, x6
    r[2] = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);  // x1, x3
    r[3] = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);  // x5, x7
    return bitcast<half8_t>(r);
}

}  // namespace mcq4
