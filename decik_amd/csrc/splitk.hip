// Split-K epilogue of the fused GEMMs: sums the per-split fp32 partial slabs in split order
// (deterministic: the same additions in the same order on every run, whatever order the
// work-groups of the GEMM ran in), adds the bias, rounds once and stores fp16 (or fp32).
// One thread per 8 consecutive output columns of one row (rows are ncols / 8 threads apart in
// the flat index), so every thread has work whatever the row length, and every load and store
// instruction is contiguous across the wave.
#include "dk_internal.h"

namespace dk {

constexpr int kReduceThreads = 256;

// Sum of the split slabs at C (2 or 4) consecutive columns of one row, in split order: the
// narrow form for reductions too small to fill the GPU at 8 columns a thread.
template <int C>
__device__ __forceinline__ void sum_splits_n(const ReduceArgs& a, const float* base, int col, float (&v)[C]) {
    using vec_t = float __attribute__((ext_vector_type(C)));
    constexpr int kBatch = 16;  // splits whose loads are in flight together
#pragma unroll
    for (int e = 0; e < C; ++e) v[e] = 0.0f;
    for (int s0 = 0; s0 < a.splits; s0 += kBatch) {
        vec_t l[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (s0 + u < a.splits) l[u] = *(const vec_t*)(base + (int64_t)(s0 + u) * a.slab + col);
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (s0 + u < a.splits)
#pragma unroll
                for (int e = 0; e < C; ++e) v[e] += l[u][e];
    }
}

// Sum of the split slabs at 8 consecutive columns of one row, in split order.
__device__ __forceinline__ void sum_splits(const ReduceArgs& a, const float* base, int col, float4_t& v0, float4_t& v1) {
    constexpr int kBatch = 16;  // splits whose loads are in flight together
    v0 = float4_t{0.f, 0.f, 0.f, 0.f};
    v1 = v0;
    for (int s0 = 0; s0 < a.splits; s0 += kBatch) {
        float4_t l0[kBatch], l1[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (s0 + u < a.splits) {
                const float4_t* p = (const float4_t*)(base + (int64_t)(s0 + u) * a.slab + col);
                // plain loads: the slabs were written just before and are read back from the
                // caches (non-temporal loads measured 2-3.5 us slower per reduction)
                l0[u] = *p;
                l1[u] = *(p + 1);
            }
        }
        // the additions stay in split order
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (s0 + u < a.splits) {
                v0 += l0[u];
                v1 += l1[u];
            }
        }
    }
}

__device__ __forceinline__ void add_bias(const ReduceOut& o, int oc, float4_t& v0, float4_t& v1) {
    if (o.bias != nullptr) {
        const half8_t b = *(const half8_t*)(o.bias + oc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v0[e] += (float)b[e];
            v1[e] += (float)b[e + 4];
        }
    }
}

// fp32 -> fp16 -> fp32: the value the projection stores as fp16
__device__ __forceinline__ float4_t round16(float4_t v) {
    float4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (float)to_half(v[e]);
    return r;
}

__global__ __launch_bounds__(kReduceThreads) void splitk_reduce_kernel(const ReduceArgs a) {
    const int chunks = a.ncols >> 3;
    const int64_t item = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;
    if (item >= (int64_t)a.m * chunks) return;
    const int row = (int)(item / chunks);
    const float* base = a.partials + (int64_t)row * a.ncols;
    const int col = (int)(item - (int64_t)row * chunks) << 3;
    int g = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.nout && col >= a.o[i].col_begin) g = i;
    const ReduceOut& o = a.o[g];
    const int oc = col - o.col_begin;
    if ((a.rope_mask >> g) & 1) {
        // RoPE (solution/attn.py:27-66 on this projection's fp16 output): the thread of a chunk in
        // the first half of a head also finishes the partner chunk head_dim / 2 further on
        // (head_dim % 16 == 0: chunks never straddle the halves); the other half's threads are idle
        const int D = a.head_dim, half = D >> 1;
        const int d = oc % D;
        if (d >= half) return;
        float4_t x0, x1, y0, y1;  // this chunk (x) and its partner (y), columns d .. d + 7, + half
        sum_splits(a, base, col, x0, x1);
        sum_splits(a, base, col + half, y0, y1);
        add_bias(o, oc, x0, x1);
        add_bias(o, oc + half, y0, y1);
        x0 = round16(x0);
        x1 = round16(x1);
        y0 = round16(y0);
        y1 = round16(y1);
        const float* cr = a.cos + (int64_t)row * D;
        const float* sr = a.sin + (int64_t)row * D;
        uint32_t ox[4], oy[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float rx[2], ry[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int j = e + q;
                const float xv = j < 4 ? x0[j] : x1[j - 4];
                const float yv = j < 4 ? y0[j] : y1[j - 4];
                // x cos + rotate_half(x) sin, the two products rounded before the sum:
                // rotate_half = [-y, x] for the first half and its partner
                const float a0 = xv * cr[d + j], b0 = (-yv) * sr[d + j];
                const float a1 = yv * cr[d + half + j], b1 = xv * sr[d + half + j];
                rx[q] = a0 + b0;
                ry[q] = a1 + b1;
            }
            ox[e >> 1] = pack_half2(rx[0], rx[1]);
            oy[e >> 1] = pack_half2(ry[0], ry[1]);
        }
        _Float16* dst = a.rope_out[g] + ((int64_t)(oc / D) * a.m + row) * D + d;
        *(u32x4_t*)dst = u32x4_t{ox[0], ox[1], ox[2], ox[3]};
        *(u32x4_t*)(dst + half) = u32x4_t{oy[0], oy[1], oy[2], oy[3]};
        return;
    }
    float4_t v0, v1;
    sum_splits(a, base, col, v0, v1);
    add_bias(o, oc, v0, v1);
    if (a.out_fp32) {
        float* dst = (float*)o.out + (int64_t)row * o.ld + oc;
        *(float4_t*)dst = v0;
        *(float4_t*)(dst + 4) = v1;
    } else {
        _Float16* dst = (_Float16*)o.out + (int64_t)row * o.ld + oc;
        *(u32x4_t*)dst = u32x4_t{pack_half2(v0[0], v0[1]), pack_half2(v0[2], v0[3]),
                                 pack_half2(v1[0], v1[1]), pack_half2(v1[2], v1[3])};
    }
}

// The same sums with C columns a thread (no RoPE epilogue): each output adds its splits in the
// same order as in splitk_reduce_kernel, so the bits are the same.
template <int C>
__global__ __launch_bounds__(kReduceThreads) void splitk_reduce_narrow_kernel(const ReduceArgs a) {
    const int chunks = a.ncols / C;
    const int64_t item = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;
    if (item >= (int64_t)a.m * chunks) return;
    const int row = (int)(item / chunks);
    const int col = (int)(item - (int64_t)row * chunks) * C;
    int g = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.nout && col >= a.o[i].col_begin) g = i;
    const ReduceOut& o = a.o[g];
    const int oc = col - o.col_begin;  // groups start at multiples of 8: a chunk lies in one group
    float v[C];
    sum_splits_n<C>(a, a.partials + (int64_t)row * a.ncols, col, v);
    if (o.bias != nullptr)
#pragma unroll
        for (int e = 0; e < C; ++e) v[e] += (float)o.bias[oc + e];
    if (a.out_fp32) {
        float* dst = (float*)o.out + (int64_t)row * o.ld + oc;
#pragma unroll
        for (int e = 0; e < C; ++e) dst[e] = v[e];
    } else {
        uint32_t* dst = (uint32_t*)((_Float16*)o.out + (int64_t)row * o.ld + oc);
#pragma unroll
        for (int e = 0; e < C; e += 2) dst[e >> 1] = pack_half2(v[e], v[e + 1]);
    }
}

// Reductions of fewer chunks than this run the narrow kernel (a quarter of the columns a thread,
// four times the threads): below it the eight-column kernel leaves most CUs idle.
constexpr int64_t kNarrowReduceChunks = 256 * kReduceThreads;

hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s) {
    if (a.m <= 0 || a.ncols <= 0) return hipSuccess;
    const int64_t items = (int64_t)a.m * (a.ncols >> 3);
    if (a.rope_mask == 0 && items < kNarrowReduceChunks) {
        const int64_t n2 = items * 4;
        hipLaunchKernelGGL(splitk_reduce_narrow_kernel<2>, dim3((unsigned)((n2 + kReduceThreads - 1) / kReduceThreads)),
                           dim3(kReduceThreads), 0, s, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((items + kReduceThreads - 1) / kReduceThreads)),
                       dim3(kReduceThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dk
