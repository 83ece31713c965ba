// Split-K epilogue of the fused GEMMs: sums the per-split fp32 partial slabs in split order
// (deterministic: the same additions in the same order on every run, whatever order the
// work-groups of the GEMM ran in), adds the bias, rounds once and stores fp16 (or fp32).
// One thread per 8 consecutive output columns of one row (rows are ncols / 8 threads apart in
// the flat index), so every thread has work whatever the row length, and every load and store
// instruction is contiguous across the wave.
#include "dk_internal.h"

namespace dk {

constexpr int kReduceThreads = 256;

__global__ __launch_bounds__(kReduceThreads) void splitk_reduce_kernel(const ReduceArgs a) {
    const int chunks = a.ncols >> 3;
    const int64_t item = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;
    if (item >= (int64_t)a.m * chunks) return;
    const int row = (int)(item / chunks);
    const float* base = a.partials + (int64_t)row * a.ncols;
    constexpr int kBatch = 16;  // splits whose loads are in flight together
    {
        const int col = (int)(item - (int64_t)row * chunks) << 3;
        float4_t v0 = {0.f, 0.f, 0.f, 0.f}, v1 = v0;
        for (int s0 = 0; s0 < a.splits; s0 += kBatch) {
            float4_t l0[kBatch], l1[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                if (s0 + u < a.splits) {
                    const float4_t* p = (const float4_t*)(base + (int64_t)(s0 + u) * a.slab + col);
                    // plain loads: the slabs were written just before and are read back from
                    // the caches (non-temporal loads measured 2-3.5 us slower per reduction)
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
        int g = 0;
#pragma unroll
        for (int i = 1; i < kMaxGroups; ++i)
            if (i < a.nout && col >= a.o[i].col_begin) g = i;
        const ReduceOut& o = a.o[g];
        const int oc = col - o.col_begin;
        if (o.bias != nullptr) {
            const half8_t b = *(const half8_t*)(o.bias + oc);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v0[e] += (float)b[e];
                v1[e] += (float)b[e + 4];
            }
        }
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
}

hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s) {
    if (a.m <= 0 || a.ncols <= 0) return hipSuccess;
    const int64_t items = (int64_t)a.m * (a.ncols >> 3);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((items + kReduceThreads - 1) / kReduceThreads)),
                       dim3(kReduceThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dk
