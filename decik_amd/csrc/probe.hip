// Dense fp16 MFMA rate of this device: a loop of v_mfma_f32_32x32x16_f16 on register operands,
// 8 waves per work-group, two A fragments x four B fragments per wave (eight independent
// accumulators, each MFMA reusing the B operand of the previous one). No memory traffic in the
// loop; the sums are stored so nothing is removed. The bench reports the GEMM kernels' rates
// against this measured ceiling beside the published peak.
#include "dk_internal.h"

namespace dk {

constexpr int kProbeThreads = 512;

__global__ __launch_bounds__(kProbeThreads, 1) void mfma_peak_kernel(float* __restrict__ out, int iters) {
    const int lane = threadIdx.x & 63;
    half8_t a0, a1, b[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a0[e] = (_Float16)(0.001f * (lane + e));
        a1[e] = (_Float16)(0.002f * (lane - e));
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q][e] = (_Float16)(0.0005f * (q + e - lane));
    }
    float16_t acc[2][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[0][q] = acc[1][q] = float16_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc[0][q] = mfma32x32x16(a0, b[q], acc[0][q]);
            acc[1][q] = mfma32x32x16(a1, b[q], acc[1][q]);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[0][q][r] + acc[1][q][r];
    out[(int64_t)blockIdx.x * kProbeThreads + threadIdx.x] = s;
}

hipError_t launch_mfma_peak(int64_t work_groups, int iters, float* out, hipStream_t s) {
    hipLaunchKernelGGL(mfma_peak_kernel, dim3((unsigned)work_groups), dim3(kProbeThreads), 0, s, out, iters);
    return hipGetLastError();
}

}  // namespace dk
