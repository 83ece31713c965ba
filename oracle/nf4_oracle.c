/*
 * CPU oracle for the NF4 dequantization path. TEST INFRASTRUCTURE ONLY: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only to
 * produce expected results (or, in bench.py, as the timed CPU baseline). The product path never
 * calls it.
 *
 * Restates the reference kernel skc_nf4_dequant_kernel (solution/nf4.py:27-48) on the CPU:
 *   for the packed byte b at flat byte offset i:
 *     block  = (2*i) / blocksize                       (solution/nf4.py:36, flat index)
 *     nested: scale = fp32(code2[absmax_u8[block]] * absmax2[block / blocksize2])
 *             scale = fp32(scale + offset)             (two roundings, no FMA: nf4.py:39-41,84)
 *     plain:  scale = absmax_f32[block]                (nf4.py:42-43)
 *     out[2i]   = fp16_rne(fp32(code[b >> 4] * scale)) (high nibble first: nf4.py:44,46)
 *     out[2i+1] = fp16_rne(fp32(code[b & 15] * scale)) (nf4.py:45-46)
 * Built with -ffp-contract=off so the compiler cannot fuse the multiply and the add.
 * The fp32 -> fp16 conversion below is written out bit by bit (round to nearest, ties to
 * even, subnormals kept, overflow to infinity) so it does not depend on the host compiler's
 * _Float16 support; tests pin it against numpy's independent conversion.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* IEEE-754 binary32 -> binary16, round to nearest even. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) {                       /* inf or NaN */
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));  /* quiet NaN, payload kept */
    }
    int32_t e = (int32_t)exp - 127 + 15;      /* rebiased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);       /* overflow (exp field >= 31) */
    if (e <= 0) {                             /* fp16 subnormal or zero */
        if (e < -10) return (uint16_t)sign;   /* below half the smallest subnormal */
        uint32_t m = man | 0x800000u;         /* implicit bit */
        int shift = 14 - e;                   /* bits dropped: 13 + (1 - e) */
        uint32_t kept = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (kept & 1u))) kept += 1u;
        return (uint16_t)(sign | kept);       /* a carry into bit 10 gives the smallest normal */
    }
    uint32_t kept = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t out = sign | ((uint32_t)e << 10) | kept;
    if (rem > 0x1000u || (rem == 0x1000u && (kept & 1u))) out += 1u;  /* carry may reach inf */
    return (uint16_t)out;
}

/* binary16 -> binary32 (exact). */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (man == 0) {
            out = sign;
        } else {                               /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            out = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1Fu) {
        out = sign | 0x7F800000u | (man << 13);
    } else {
        out = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

/* One 64-bit flat byte offset -> its scale (solution/nf4.py:36-43). */
static inline float nf4_scale(int64_t byte, const uint8_t* absmax_u8, const float* absmax_f32,
                              const float* absmax2, const float* code2, float offset, int nested,
                              int64_t blocksize, int64_t blocksize2) {
    int64_t block = (2 * byte) / blocksize;
    if (nested) {
        float s = code2[absmax_u8[block]] * absmax2[block / blocksize2];
        return s + offset;
    }
    return absmax_f32[block];
}

/* Dequantize n_bytes packed bytes into 2*n_bytes fp16 values (as uint16 bit patterns). */
void oracle_nf4_dequant(const uint8_t* packed, const uint8_t* absmax_u8, const float* absmax_f32,
                        const float* absmax2, const float* code2, float offset, const float* code,
                        uint16_t* out, int64_t n_bytes, int nested, int64_t blocksize,
                        int64_t blocksize2, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static) if (nthreads != 1)
#endif
    for (int64_t i = 0; i < n_bytes; ++i) {
        float scale = nf4_scale(i, absmax_u8, absmax_f32, absmax2, code2, offset, nested,
                                blocksize, blocksize2);
        uint8_t b = packed[i];
        float hi = code[b >> 4] * scale;
        float lo = code[b & 15] * scale;
        out[2 * i] = oracle_f32_to_f16(hi);
        out[2 * i + 1] = oracle_f32_to_f16(lo);
    }
}

/* Vector helpers used by the checks: bulk fp16 <-> fp32. */
void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
