// SwiGLU between the gate/up and down projections (solution/swiglu.py:15-37, the reference's
// example kernels): fwd out = fp16(g sigmoid(g) u); bwd dup = G g s, dgate = G u s (1 + g (1 - s)),
// all in fp32, 8 elements per thread with 16-byte loads and stores.
#include "dk_internal.h"

namespace dk {

constexpr int kEwThreads = 256;

__global__ __launch_bounds__(kEwThreads) void swiglu_fwd_kernel(const _Float16* __restrict__ g,
                                                                 const _Float16* __restrict__ u,
                                                                 _Float16* __restrict__ o,
                                                                 int64_t n) {
    const int64_t i0 = ((int64_t)blockIdx.x * kEwThreads + threadIdx.x) * 8;
    if (i0 + 8 <= n) {
        const half8_t gv = *(const half8_t*)(g + i0);
        const half8_t uv = *(const half8_t*)(u + i0);
        const u32x4_t g4 = __builtin_bit_cast(u32x4_t, gv), u4 = __builtin_bit_cast(u32x4_t, uv);
        *(u32x4_t*)(o + i0) = u32x4_t{swiglu_fwd2(g4[0], u4[0]), swiglu_fwd2(g4[1], u4[1]),
                                      swiglu_fwd2(g4[2], u4[2]), swiglu_fwd2(g4[3], u4[3])};
    } else {
        for (int64_t i = i0; i < n; ++i) {
            const uint32_t h = swiglu_fwd2(__builtin_bit_cast(uint16_t, g[i]), __builtin_bit_cast(uint16_t, u[i]));
            o[i] = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
        }
    }
}

__global__ __launch_bounds__(kEwThreads) void swiglu_bwd_kernel(const _Float16* __restrict__ gr,
                                                                 const _Float16* g,
                                                                 const _Float16* u,
                                                                 _Float16* dg, _Float16* du,
                                                                 int64_t n) {
    // dg/du may alias g/u: each thread reads its 8 elements before writing them
    const int64_t i0 = ((int64_t)blockIdx.x * kEwThreads + threadIdx.x) * 8;
    if (i0 + 8 <= n) {
        const half8_t Gv = *(const half8_t*)(gr + i0);
        const half8_t gv = *(const half8_t*)(g + i0);
        const half8_t uv = *(const half8_t*)(u + i0);
        half8_t dgv, duv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float dgf, duf;
            swiglu_bwd1((float)Gv[e], (float)gv[e], (float)uv[e], dgf, duf);
            dgv[e] = (_Float16)dgf;
            duv[e] = (_Float16)duf;
        }
        *(half8_t*)(dg + i0) = dgv;
        *(half8_t*)(du + i0) = duv;
    } else {
        for (int64_t i = i0; i < n; ++i) {
            float dgf, duf;
            swiglu_bwd1((float)gr[i], (float)g[i], (float)u[i], dgf, duf);
            du[i] = (_Float16)duf;
            dg[i] = (_Float16)dgf;
        }
    }
}

static inline int ew_grid(int64_t n) { return (int)((n + 8 * kEwThreads - 1) / (8 * kEwThreads)); }

hipError_t launch_swiglu_fwd(const _Float16* g, const _Float16* u, _Float16* o, int64_t n,
                             hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_fwd_kernel, dim3(ew_grid(n)), dim3(kEwThreads), 0, s, g, u, o, n);
    return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const _Float16* gr, const _Float16* g, const _Float16* u,
                             _Float16* dg, _Float16* du, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(ew_grid(n)), dim3(kEwThreads), 0, s, gr, g, u, dg, du, n);
    return hipGetLastError();
}

}  // namespace dk
