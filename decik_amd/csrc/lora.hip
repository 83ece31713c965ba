// Rank-r LoRA products around the fused GEMMs (r = 16 for q/v in the reference run).
//
// The reference runs peft's branch as fp16 matmuls (solution/attn.py:225-228 forward,
// :251-257 backward). Here:
//   lora_down:  U  = fp16(X . A^T)                 [m, r]   (the forward epilogue adds s U.B^T)
//   lora_gu:    GU = fp16(s * dY . B)              [m, r]   (the backward epilogue adds GU.A)
//   lora_wgrad: dB = s * dY^T . U  (fp32 [n, r]),  dA = GU^T . X  (fp32 [r, k])
// These are ~2% of the flops of the projection they ride on. lora_down / lora_gu use one
// work-group per token row (the contraction is spread over the 256 threads, then reduced with
// cross-lane shuffles and LDS); the weight gradients reduce over tokens inside one work-group
// per 16 output columns (16 token slices reduced through LDS), so no atomics and the summation
// order is fixed.
#include "dk_internal.h"

namespace dk {

constexpr int kLoraThreads = 256;

// Sum `v[0..R)` over the 256 threads of the work-group; thread 0..R-1 returns the total of
// component tid in *out.
template <int R>
__device__ __forceinline__ void block_reduce(float (&v)[R], float* red, float* out) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int t = 0; t < R; ++t) {
        float x = v[t];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
        v[t] = x;
    }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < R; ++t) red[wave * R + t] = v[t];
    }
    __syncthreads();
    if (tid < R) *out = ((red[tid] + red[R + tid]) + red[2 * R + tid]) + red[3 * R + tid];
}

// U[m, t] = fp16(sum_k X[m, k] A[t, k]); one work-group per row m, 8 consecutive k per thread.
template <int R>
__global__ __launch_bounds__(kLoraThreads) void lora_down_kernel(const _Float16* __restrict__ x,
                                                                 int64_t k, int64_t ldx,
                                                                 const _Float16* __restrict__ a,
                                                                 _Float16* __restrict__ u) {
    __shared__ float red[4 * R];
    const int64_t m = blockIdx.x;
    const _Float16* xr = x + m * ldx;
    float acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = 0.0f;
    for (int64_t k0 = 8 * threadIdx.x; k0 < k; k0 += 8 * kLoraThreads) {
        if (k0 + 8 <= k) {
            const half8_t xv = *(const half8_t*)(xr + k0);
#pragma unroll
            for (int t = 0; t < R; ++t) {
                const half8_t av = *(const half8_t*)(a + (int64_t)t * k + k0);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[t] = __builtin_fmaf((float)xv[e], (float)av[e], acc[t]);
            }
        } else {
            for (int64_t kk = k0; kk < k; ++kk)
#pragma unroll
                for (int t = 0; t < R; ++t)
                    acc[t] = __builtin_fmaf((float)xr[kk], (float)a[(int64_t)t * k + kk], acc[t]);
        }
    }
    float tot;
    block_reduce<R>(acc, red, &tot);
    if (threadIdx.x < R) u[m * R + threadIdx.x] = (_Float16)tot;
}

// GU[m, t] = fp16(s * sum_n dY[m, n] B[n, t]); one work-group per row m.
template <int R>
__global__ __launch_bounds__(kLoraThreads) void lora_gu_kernel(const _Float16* __restrict__ dy,
                                                               int64_t lddy, int64_t n,
                                                               const _Float16* __restrict__ b,
                                                               float scale,
                                                               _Float16* __restrict__ gu) {
    __shared__ float red[4 * R];
    const int64_t m = blockIdx.x;
    const _Float16* dr = dy + m * lddy;
    float acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = 0.0f;
    for (int64_t j = threadIdx.x; j < n; j += kLoraThreads) {
        const float g = (float)dr[j];
        const _Float16* br = b + j * R;
#pragma unroll
        for (int t = 0; t < R; t += 8) {
            const half8_t bv = *(const half8_t*)(br + t);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[t + e] = __builtin_fmaf(g, (float)bv[e], acc[t + e]);
        }
    }
    float tot;
    block_reduce<R>(acc, red, &tot);
    if (threadIdx.x < R) gu[m * R + threadIdx.x] = to_half(scale * tot);
}

// C[c, t] = scale * sum_m Q[m, c] P[m, t] over all m, for 16 columns c per work-group:
// thread = (column c0 + tid % 16, token slice tid / 16); slices reduced in LDS in fixed order.
// transpose_out: write C as [t][c] (row stride ldc) instead of [c][t].
template <int R>
__global__ __launch_bounds__(kLoraThreads) void lora_wgrad_kernel(
    const _Float16* __restrict__ q, int64_t ldq, const _Float16* __restrict__ p, int64_t m_rows,
    int64_t ncols, float scale, float* __restrict__ c, int64_t ldc, int transpose_out) {
    __shared__ float red[16][16][R + 1];
    const int tid = threadIdx.x;
    const int cl = tid & 15, slice = tid >> 4;
    const int64_t col = (int64_t)blockIdx.x * 16 + cl;
    float acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = 0.0f;
    if (col < ncols) {
        for (int64_t m = slice; m < m_rows; m += 16) {
            const float qv = (float)q[m * ldq + col];
            const _Float16* pr = p + m * R;
#pragma unroll
            for (int t = 0; t < R; t += 8) {
                const half8_t pv = *(const half8_t*)(pr + t);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[t + e] = __builtin_fmaf(qv, (float)pv[e], acc[t + e]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < R; ++t) red[slice][cl][t] = acc[t];
    __syncthreads();
    // thread (cl, t-part) sums the 16 slices of column cl for t = tid / 16 (+16 ...)
    for (int t = slice; t < R; t += 16) {
        float s = 0.0f;
#pragma unroll
        for (int sl = 0; sl < 16; ++sl) s += red[sl][cl][t];
        if (col < ncols) {
            if (transpose_out) c[(int64_t)t * ldc + col] = scale * s;
            else c[col * ldc + t] = scale * s;
        }
    }
}

#define DK_RANK_CASES(X) X(16) X(32)

hipError_t launch_lora_down(const _Float16* x, int64_t m, int64_t k, int64_t ldx, const _Float16* a,
                            int rank, _Float16* u, hipStream_t s) {
    if (m == 0) return hipSuccess;
#define X(R) \
    if (rank == R) { hipLaunchKernelGGL((lora_down_kernel<R>), dim3(m), dim3(kLoraThreads), 0, s, x, k, ldx, a, u); return hipGetLastError(); }
    DK_RANK_CASES(X)
#undef X
    return hipErrorInvalidValue;
}

hipError_t launch_lora_bwd(const _Float16* dy, int64_t lddy, const _Float16* u, const _Float16* x,
                           int64_t ldx, const _Float16* b, int64_t m, int64_t n, int64_t k, int rank,
                           float scale, _Float16* gu, float* da, float* db, hipStream_t s) {
    if (m == 0) return hipSuccess;
#define X(R)                                                                                        \
    if (rank == R) {                                                                                \
        hipLaunchKernelGGL((lora_gu_kernel<R>), dim3(m), dim3(kLoraThreads), 0, s, dy, lddy, n, b,  \
                           scale, gu);                                                              \
        if (db != nullptr)                                                                          \
            hipLaunchKernelGGL((lora_wgrad_kernel<R>), dim3((n + 15) / 16), dim3(kLoraThreads), 0, \
                               s, dy, lddy, u, m, n, scale, db, (int64_t)R, 0);                     \
        if (da != nullptr)                                                                          \
            hipLaunchKernelGGL((lora_wgrad_kernel<R>), dim3((k + 15) / 16), dim3(kLoraThreads), 0, \
                               s, x, ldx, gu, m, k, 1.0f, da, k, 1);                                \
        return hipGetLastError();                                                                   \
    }
    DK_RANK_CASES(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
