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
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
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
    uint32_t packed_bytes, absmax_bytes, absmax2_bytes;  // buffer sizes (fused GEMM: < 2^31)
};

// Raw buffer loads (gfx9 resource word 3 = 0x00020000): an offset at or past the buffer's size
// reads 0, so edge tiles need no branches around their loads -- invalid lanes load at kOOB.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;

// Buffer offset that reads zeros unless `ok`: sets bit 31 (every buffer here is < 2^31 bytes).
// Written as arithmetic so the compiler keeps one load instead of branching around two.
__device__ __forceinline__ uint32_t off_if(bool ok, uint32_t off) {
    return off | ((uint32_t)!ok << 31);
}

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t bload128(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x2_t bload64(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload8(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
// 16 bytes per lane straight into LDS: lane l's data lands at lds_wave_base + 16 * l (the base
// must be the same for the whole wave). Past-the-end offsets write zeros.
__device__ __forceinline__ void bload128_lds(rsrc_t r, void* lds_wave_base, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_wave_base, 16, (int)off, 0, 0, 0);
}

// 1 or 4 bytes per lane straight into LDS; each lane's value occupies a dword slot, at
// lds_wave_base + 4 * l, whatever the load size.
__device__ __forceinline__ void bload8_lds(rsrc_t r, void* lds_wave_base, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_wave_base, 1, (int)off, 0, 0, 0);
}
__device__ __forceinline__ void bload32_lds(rsrc_t r, void* lds_wave_base, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_wave_base, 4, (int)off, 0, 0, 0);
}

// Wait until at most n vector-memory operations are outstanding (global loads and the
// buffer -> LDS loads above). Written as inline asm with a memory clobber so the compiler keeps
// memory operations on their side of it.
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// Work-group barrier for LDS hand-offs: this wave's LDS writes complete, then s_barrier. Unlike
// __syncthreads() it carries no release fence, which would wait for every outstanding global ->
// LDS load (vmcnt(0)) and so serialize the prefetch; loads the next phase reads are covered by
// an explicit wait_vmcnt before the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float bloadf(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

__device__ __forceinline__ int64_t block_of(const NF4Dev& w, int64_t flat) {
    return w.bs_shift >= 0 ? (flat >> w.bs_shift) : flat / w.blocksize;
}

__device__ __forceinline__ int64_t group_of(const NF4Dev& w, int64_t block) {
    return w.bs2_shift >= 0 ? (block >> w.bs2_shift) : block / w.blocksize2;
}

// fp32 -> two fp16 (round to nearest even) packed with `a` in the low half. The empty asm hides
// a product feeding the conversion from the compiler, which would otherwise fold fp16(x * y)
// into v_fma_mix*_f16 with a +0 addend -- that turns a -0 product into +0.
__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
    asm("" : "+v"(a), "+v"(b));
    half2_t h;
    h.x = (_Float16)a;
    h.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, h);
}

// fp32 -> fp16 (round to nearest even), the value opaque to the compiler (see pack_half2).
__device__ __forceinline__ _Float16 to_half(float x) {
    asm("" : "+v"(x));
    return (_Float16)x;
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

// Code-book lookups with cheap addresses. The kernels keep their 16-entry code books in a static
// __shared__ array, whose LDS address is a compile-time constant that folds into the ds_read
// offset; code book g occupies bytes 64 g .. 64 g + 63, so every lookup address fits in a byte.
// nib_addrs turns a packed dword into two words of such byte addresses (4 * nibble + 64 g):
// `hi` for the high nibbles of its 4 bytes, `lo` for the low ones; each lookup then costs one
// v_bfe_u32. The empty asm keeps the compiler from folding the masks back into per-lookup
// shift-and pairs.
__device__ __forceinline__ void nib_addrs(uint32_t w, uint32_t gbase4, uint32_t& hi, uint32_t& lo) {
    hi = ((w >> 2) & 0x3C3C3C3Cu) | gbase4;
    lo = ((w << 2) & 0x3C3C3C3Cu) | gbase4;
    asm("" : "+v"(hi), "+v"(lo));
}

// 8 x byte e of w (the byte-pair code-book offset) in one SDWA instruction
__device__ __forceinline__ uint32_t byte_x8(uint32_t w, int e) {
    uint32_t r;
    switch (e) {
        case 0: asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(r) : "v"(w)); break;
        case 1: asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(r) : "v"(w)); break;
        case 2: asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(r) : "v"(w)); break;
        default: asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(r) : "v"(w)); break;
    }
    return r;
}

__device__ __forceinline__ float lut_at(const float* lut, uint32_t addrs, int byte) {
    return *(const float*)((const char*)lut + __builtin_amdgcn_ubfe(addrs, 8 * byte, 8));
}

// Dequantize 4 packed bytes (8 weights, one scale) with a static-LDS code book (see nib_addrs):
// dword j = fp16 pair (high nibble of byte j, low nibble of byte j).
__device__ __forceinline__ void dequant4s(uint32_t word, float s, const float* lut, uint32_t* o) {
    uint32_t hi, lo;
    nib_addrs(word, 0u, hi, lo);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_half2(lut_at(lut, hi, j) * s, lut_at(lut, lo, j) * s);
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

// SwiGLU arithmetic (solution/swiglu.py:15-37), shared by the elementwise kernels and the fused
// GEMM epilogues so both give the same bits: fp32 from fp16 inputs, one fp16 rounding. The
// sigmoid uses the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each, far
// below the fp16 output rounding), three instructions instead of a full-precision expf and
// division: in a GEMM epilogue nothing hides this arithmetic.
__device__ __forceinline__ float swiglu_sigmoid(float g) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}

// fp16 pairs: h = (g sigmoid(g)) u
__device__ __forceinline__ uint32_t swiglu_fwd2(uint32_t g2, uint32_t u2) {
    const half2_t g = __builtin_bit_cast(half2_t, g2), u = __builtin_bit_cast(half2_t, u2);
    const float g0 = (float)g.x, g1 = (float)g.y;
    return pack_half2(g0 * swiglu_sigmoid(g0) * (float)u.x, g1 * swiglu_sigmoid(g1) * (float)u.y);
}

// one element: dup = G g s, dgate = G u s (1 + g (1 - s)), s = sigmoid(g)
__device__ __forceinline__ void swiglu_bwd1(float G, float g, float u, float& dg, float& du) {
    const float s = swiglu_sigmoid(g);
    du = G * g * s;
    dg = G * u * s * (1.0f + g * (1.0f - s));
    asm("" : "+v"(du), "+v"(dg));  // keep a later fp16 conversion off v_fma_mix (see pack_half2)
}

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4_t mfma16x16x16(half4_t a, half4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_f16 (gfx950), with g = l / 32:
//   A operand: lane l holds A[l % 32][8 g + e], e = 0..7
//   B operand: lane l holds B[8 g + e][l % 32]
//   C/D:       lane l holds D[8 (r / 4) + 4 g + (r % 4)][l % 32], r = 0..15
// With A row i taken from weight row arow_to_n(i) (a permutation of 0..31), lane l's 16
// accumulators are the 16 consecutive weight rows 16 g + r.
__device__ __forceinline__ int arow_to_n(int i) {
    return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3);
}

// The wave's lane-group layout of v_mfma_f32_16x16x32_f16 (CDNA3/4):
//   A operand: lane l holds A[l % 16][8 * (l / 16) + e], e = 0..7
//   B operand: lane l holds B[8 * (l / 16) + e][l % 16]
//   C/D:       lane l holds D[4 * (l / 16) + r][l % 16], r = 0..3

}  // namespace dk
