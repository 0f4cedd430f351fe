/* Plain-C restatement of the reference's INT8 per-token quantizer.
 *
 * TEST INFRASTRUCTURE ONLY: built by oracle/Makefile into oracle/libfa_oracle.so
 * and loaded by tests/ to cross-check oracle/quant.py.  Not part of the
 * product library.
 *
 * Follows /root/reference/flash_attn_triton/triton_kernel/attention_kernel_int8.py:
 *   _round_i8        :27-30   x >= 0 ? floor(x + 0.5) : ceil(x - 0.5), fp32
 *   _quantize_rows   :33-39   s = max(amax, 1) / 127; x = q / s      (Q form)
 *   _quantize_k_rows :58-79   s = max(amax, 1) / 127; x = k * (1/s)  (K form)
 * Compiled with -O2 -fno-fast-math -ffp-contract=off so every float
 * operation is a single IEEE-754 binary32 operation with round-to-nearest-even.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* IEEE half -> float, exact (every binary16 value is representable). */
static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float f = (float)man * 5.9604644775390625e-8f; /* exact: man < 2^10 */
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static int8_t round_i8(float x) {
    volatile float y = (x >= 0.0f) ? floorf(x + 0.5f) : ceilf(x - 0.5f);
    return (int8_t)(int)y;
}

/* mode 0: K form (multiply by the fp32 reciprocal); mode 1: Q form (divide). */
static void quantize_rows(const uint16_t* x, int8_t* x8, float* s, int64_t rows,
                          int64_t dim, int mode) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* row = x + r * dim;
        float amax = 0.0f;
        for (int64_t d = 0; d < dim; ++d) {
            float a = fabsf(half_to_float(row[d]));
            if (a > amax) amax = a;
        }
        volatile float clamped = amax > 1.0f ? amax : 1.0f;
        volatile float scale = clamped / 127.0f;
        volatile float inv = 1.0f / scale;
        for (int64_t d = 0; d < dim; ++d) {
            float v = half_to_float(row[d]);
            volatile float q = mode == 0 ? v * inv : v / scale;
            x8[r * dim + d] = round_i8(q);
        }
        s[r] = scale;
    }
}

void oracle_quantize_k_rows_f16(const uint16_t* k, int8_t* k8, float* s, int64_t rows,
                                int64_t dim) {
    quantize_rows(k, k8, s, rows, dim, 0);
}

void oracle_quantize_q_rows_f16(const uint16_t* q, int8_t* q8, float* s, int64_t rows,
                                int64_t dim) {
    quantize_rows(q, q8, s, rows, dim, 1);
}
