// Device-side building blocks shared by the NF4 kernels (gfx950, wave64).
//
// Arithmetic contract (bit-exact with solution/nf4.py:31-48):
//   nested scale = fp32(fp32(code2[q] * absmax2[block / blocksize2]) + offset)  (no FMA)
//   weight       = fp16_rne(fp32(code[nibble] * scale)), high nibble = even element.
// The whole library is compiled with -ffp-contract=off, so no multiply-add pair below is
// fused unless it is written as an explicit fma.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "decik_nf4.h"

namespace dk {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Weight descriptor as the kernels see it (host fills it from dk_nf4_weight).
struct NF4Dev {
    const uint8_t* packed;
    const uint8_t* absmax8;   // nested codes
    const float* absmaxf;     // plain fp32 absmax
    const float* absmax2;
    const float* code2;
    const float* offset;
    const float* code;
    int64_t n, k;
    int32_t blocksize, blocksize2;
    int32_t bs_shift, bs2_shift;  // log2 of the block sizes, -1 if not a power of two
};

__device__ __forceinline__ int64_t block_of(const NF4Dev& w, int64_t flat) {
    return w.bs_shift >= 0 ? (flat >> w.bs_shift) : flat / w.blocksize;
}

__device__ __forceinline__ int64_t group_of(const NF4Dev& w, int64_t block) {
    return w.bs2_shift >= 0 ? (block >> w.bs2_shift) : block / w.blocksize2;
}

// fp32 -> two fp16 (round to nearest even) packed with `a` in the low half.
__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
    half2_t h;
    h.x = (_Float16)a;
    h.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, h);
}

// The fp32 scale of the block `block` (solution/nf4.py:37-43). `code2` may point to LDS.
template <bool NESTED>
__device__ __forceinline__ float block_scale(const NF4Dev& w, int64_t block, const float* code2,
                                             float offset) {
    if constexpr (NESTED) {
        const float s = code2[w.absmax8[block]] * w.absmax2[group_of(w, block)];
        return s + offset;
    } else {
        return w.absmaxf[block];
    }
}

// Dequantize 4 packed bytes (8 weights, one scale) into 4 dwords of fp16 pairs: dword d holds
// byte d's high-nibble weight in its low half and low-nibble weight in its high half, which is
// the element order of the unpacked row. `lut` is the 16-entry code book (LDS).
__device__ __forceinline__ void dequant4(uint32_t word, float s, const float* lut, uint32_t* o) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t b = (word >> (8 * j)) & 0xFFu;
        o[j] = pack_half2(lut[b >> 4] * s, lut[b & 15u] * s);
    }
}

// 16 packed bytes (32 weights, one scale) -> 16 dwords.
__device__ __forceinline__ void dequant16(u32x4_t p, float s, const float* lut, uint32_t* o) {
    dequant4(p.x, s, lut, o + 0);
    dequant4(p.y, s, lut, o + 4);
    dequant4(p.z, s, lut, o + 8);
    dequant4(p.w, s, lut, o + 12);
}

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4_t mfma16x16x16(half4_t a, half4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// The wave's lane-group layout of v_mfma_f32_16x16x32_f16 (CDNA3/4):
//   A operand: lane l holds A[l % 16][8 * (l / 16) + e], e = 0..7
//   B operand: lane l holds B[8 * (l / 16) + e][l % 16]
//   C/D:       lane l holds D[4 * (l / 16) + r][l % 16], r = 0..3

}  // namespace dk
