/*
 * Independent plain-C restatement of metalcore's GGML block_q4_0 path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as a checker; never linked into the product.
 *
 * It is written separately from oracle/q4_0_ref.py (numpy) so that the two
 * restatements check each other.  fp16 conversion is done here with integer
 * bit manipulation (round to nearest even), not with a library routine.
 *
 * Reference (packages/metalcore/src/metalcore/):
 *   quantization.py:303-304  QK4_0 = 32, 18-byte blocks
 *   quantization.py:333-369  quantize_ggml_q4_0: d = amax/7 (0 -> 1),
 *                            q = round_half_even(x/d + 8) clamped to [0, 15],
 *                            byte i = q[2i] | q[2i+1] << 4, layout [K/32][N][18]
 *   quantization.py:391-419  dequantize_ggml_q4_0: W = (q - 8) * d in fp32
 *   quantization.py:452-454  matmul fallback: X @ dequant(W)
 * llama.cpp quantize_row_q4_0_ref rule (benchmark generator only):
 *   d = max_signed / -8, id = d ? 1/d : 0, q = min(15, (int8)(x*id + 8.5)).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define QK 32
#define BS 18

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even, with subnormals and inf/nan. */
uint16_t q4ref_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e = (x >> 23) & 0xFFu;
    uint32_t m = x & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    int32_t he = (int32_t)e - 127 + 15;
    if (he >= 0x1F) return (uint16_t)(sign | 0x7C00u);          /* overflow -> inf */
    if (he <= 0) {                                               /* subnormal or zero */
        if (he < -10) return (uint16_t)sign;
        uint32_t mant = m | 0x800000u;
        uint32_t shift = (uint32_t)(14 - he);                    /* 24-bit mant -> 10-bit field */
        uint32_t r = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)he << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;    /* may carry into exponent: ok */
    return (uint16_t)(sign | r);
}

float q4ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * (1.0f / 16777216.0f);               /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* Round half to even for finite floats (torch.round semantics). */
static float round_half_even(float t) {
    float fl = floorf(t);
    float diff = t - fl;                                         /* exact for |t| < 2^23 */
    if (diff > 0.5f) return fl + 1.0f;
    if (diff < 0.5f) return fl;
    return (fmodf(fl, 2.0f) == 0.0f) ? fl : fl + 1.0f;
}

static void put_block(uint8_t *blk, float d, const uint8_t q[QK]) {
    uint16_t dh = q4ref_f32_to_f16(d);
    blk[0] = (uint8_t)(dh & 0xFF);
    blk[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 16; ++i) blk[2 + i] = (uint8_t)(q[2 * i] | (q[2 * i + 1] << 4));
}

/* W: row-major fp32 [K][N]; out: [K/32][N][18]. */
void q4ref_quantize_ref(const float *W, int64_t K, int64_t N, uint8_t *out) {
    int64_t nb = K / QK;
    for (int64_t kb = 0; kb < nb; ++kb)
        for (int64_t n = 0; n < N; ++n) {
            float amax = 0.0f;
            for (int j = 0; j < QK; ++j) {
                float a = fabsf(W[(kb * QK + j) * N + n]);
                if (a > amax) amax = a;
            }
            volatile float d = amax / 7.0f;
            float dd = (d > 0.0f) ? d : 1.0f;
            uint8_t q[QK];
            for (int j = 0; j < QK; ++j) {
                volatile float t = W[(kb * QK + j) * N + n] / dd;
                volatile float t8 = t + 8.0f;
                float r = round_half_even(t8);
                if (r < 0.0f) r = 0.0f;
                if (r > 15.0f) r = 15.0f;
                q[j] = (uint8_t)r;
            }
            put_block(out + (kb * N + n) * BS, dd, q);
        }
}

void q4ref_quantize_llama(const float *W, int64_t K, int64_t N, uint8_t *out) {
    int64_t nb = K / QK;
    for (int64_t kb = 0; kb < nb; ++kb)
        for (int64_t n = 0; n < N; ++n) {
            float amax = 0.0f, mx = 0.0f;
            for (int j = 0; j < QK; ++j) {
                float v = W[(kb * QK + j) * N + n];
                if (amax < fabsf(v)) { amax = fabsf(v); mx = v; }
            }
            volatile float d = mx / -8.0f;
            volatile float id = (d != 0.0f) ? 1.0f / d : 0.0f;
            uint8_t q[QK];
            for (int j = 0; j < QK; ++j) {
                volatile float x0 = W[(kb * QK + j) * N + n] * id;
                volatile float t = x0 + 8.5f;
                int v = (int)(int8_t)(int)t;                     /* C truncation toward zero */
                q[j] = (uint8_t)(v < 15 ? v : 15);
            }
            put_block(out + (kb * N + n) * BS, d, q);
        }
}

/* blocks [K/32][N][18] -> row-major fp32 [K][N]. */
void q4ref_dequant_f32(const uint8_t *blocks, int64_t K, int64_t N, float *out) {
    int64_t nb = K / QK;
    for (int64_t kb = 0; kb < nb; ++kb)
        for (int64_t n = 0; n < N; ++n) {
            const uint8_t *b = blocks + (kb * N + n) * BS;
            float d = q4ref_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            for (int j = 0; j < QK; ++j) {
                int q = (j & 1) ? (b[2 + j / 2] >> 4) : (b[2 + j / 2] & 0xF);
                out[(kb * QK + j) * N + n] = (float)(q - 8) * d;
            }
        }
}

/* blocks -> fp16 bits [K][N]: one rounding of the exact fp32 product. */
void q4ref_dequant_f16(const uint8_t *blocks, int64_t K, int64_t N, uint16_t *out) {
    int64_t nb = K / QK;
    for (int64_t kb = 0; kb < nb; ++kb)
        for (int64_t n = 0; n < N; ++n) {
            const uint8_t *b = blocks + (kb * N + n) * BS;
            float d = q4ref_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            for (int j = 0; j < QK; ++j) {
                int q = (j & 1) ? (b[2 + j / 2] >> 4) : (b[2 + j / 2] & 0xF);
                out[(kb * QK + j) * N + n] = q4ref_f32_to_f16((float)(q - 8) * d);
            }
        }
}

/* X: fp16 bits row-major [M][K]; Y: float64 [M][N] = X @ dequant(W), summed in double. */
void q4ref_matmul_f64(const uint16_t *X, int64_t M, int64_t K, const uint8_t *blocks,
                      int64_t N, double *Y) {
    int64_t nb = K / QK;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) Y[m * N + n] = 0.0;
    for (int64_t kb = 0; kb < nb; ++kb)
        for (int64_t n = 0; n < N; ++n) {
            const uint8_t *b = blocks + (kb * N + n) * BS;
            double d = (double)q4ref_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            for (int j = 0; j < QK; ++j) {
                int q = (j & 1) ? (b[2 + j / 2] >> 4) : (b[2 + j / 2] & 0xF);
                double w = (double)(q - 8) * d;
                for (int64_t m = 0; m < M; ++m)
                    Y[m * N + n] += (double)q4ref_f16_to_f32(X[m * K + kb * QK + j]) * w;
            }
        }
}
