// Helpers shared by the fused dequant-GEMM kernels (forward and input gradient).
#pragma once

#include "dk_internal.h"

namespace dk {

__device__ __forceinline__ int xcd_logical_id() {
    // The dispatcher deals work-groups to the 8 XCDs round-robin. Renumber them so that logical
    // ids that are consecutive run on one XCD (and share its L2). gridDim.x is a multiple of 8.
    const int nwg = gridDim.x, bid = blockIdx.x;
    return (bid & 7) * (nwg >> 3) + (bid >> 3);
}

// Pin a wave-uniform 32- or 64-bit value (a pointer: an SGPR pair) in scalar registers: the empty
// asm hides where the value came from, so the compiler can neither re-load it from memory later
// -- inside a loop that would be a scalar load, whose out-of-order return forces a wait on every
// outstanding LDS read -- nor move it to a VGPR.
template <typename T>
__device__ __forceinline__ T sgpr(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values only");
    asm volatile("" : "+s"(v));
    return v;
}

__device__ __forceinline__ uint32_t perm_lo(uint32_t lo_src, uint32_t hi_src) {
    // low 16 bits of lo_src, then low 16 bits of hi_src
    return __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
}

__device__ __forceinline__ uint32_t perm_hi(uint32_t lo_src, uint32_t hi_src) {
    // high 16 bits of lo_src, then high 16 bits of hi_src
    return __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
}

__device__ __forceinline__ float4_t chunk4(const float16_t& v, int q) {
    switch (q) {
        case 0: return __builtin_shufflevector(v, v, 0, 1, 2, 3);
        case 1: return __builtin_shufflevector(v, v, 4, 5, 6, 7);
        case 2: return __builtin_shufflevector(v, v, 8, 9, 10, 11);
        default: return __builtin_shufflevector(v, v, 12, 13, 14, 15);
    }
}

__device__ __forceinline__ float16_t join4(float4_t a, float4_t b, float4_t c, float4_t d) {
    typedef float float8_t __attribute__((ext_vector_type(8)));
    const float8_t ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    const float8_t cd = __builtin_shufflevector(c, d, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

// Ring refills spread over a step. A step's loads are split into parts, issued in the order
// packed weights, their statistics, then the activation chunks (the weights come from HBM, the
// activation tiles mostly from L2, so the weights get the longest flight). Issue index i goes
// after MFMA (i / 4) * (MB / 2) of one slice: for i % 4 == 0, slice 3 of the step three before
// (once that step's barrier has freed the ring slots), otherwise slice i % 4 - 1 of the step two
// before; each slice then issues at most two loads, and the eight waves' loads no longer meet
// in one slice.
__host__ __device__ constexpr int spread_slice(int i) { return i % 4 == 0 ? 3 : i % 4 - 1; }
// the part of issue index i, for a step of `chunks` activation chunks (parts 0 .. chunks - 1),
// the packed weights (part chunks) and their statistics (part chunks + 1)
__host__ __device__ constexpr int spread_part(int i, int chunks) {
    return i == 0 ? chunks : (i == 1 ? chunks + 1 : i - 2);
}
// loads of one step issued by the time the parts after MFMA 0 of slice `slice` (of the step two
// before) are out, counting the slice-3 parts of the step before that first (slice < 0: those
// only); the statistics part is `stats_loads` loads
__host__ __device__ constexpr int spread_loads(int parts, int stats_loads, int slice) {
    int n = 0;
    for (int i = 0; i < parts; ++i) {
        const int s = spread_slice(i);
        if (s == 3 || s < slice || (s == slice && i < 4)) n += i == 1 ? stats_loads : 1;
    }
    return n;
}

template <typename V>
struct AccChunks;
template <>
struct AccChunks<float4_t> {
    static constexpr int n = 1;
    static __device__ __forceinline__ float4_t get(const float4_t& v, int) { return v; }
    static __device__ __forceinline__ void set(float4_t& v, int, float4_t c) { v = c; }
};
template <>
struct AccChunks<float16_t> {
    static constexpr int n = 4;
    static __device__ __forceinline__ float4_t get(const float16_t& v, int q) { return chunk4(v, q); }
    static __device__ __forceinline__ void set(float16_t& v, int q, float4_t c) {
        const float16_t w = join4(c, c, c, c);
        switch (q) {
            case 0: v = __builtin_shufflevector(v, w, 16, 17, 18, 19, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15); break;
            case 1: v = __builtin_shufflevector(v, w, 0, 1, 2, 3, 20, 21, 22, 23, 8, 9, 10, 11, 12, 13, 14, 15); break;
            case 2: v = __builtin_shufflevector(v, w, 0, 1, 2, 3, 4, 5, 6, 7, 24, 25, 26, 27, 12, 13, 14, 15); break;
            default: v = __builtin_shufflevector(v, w, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 28, 29, 30, 31); break;
        }
    }
};

}  // namespace dk
