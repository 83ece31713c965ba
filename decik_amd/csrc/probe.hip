// Measured ceilings of this device, for reporting the kernels against them.
//
// Dense fp16 MFMA rate: a loop of v_mfma_f32_32x32x16_f16 on register operands,
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

// HBM streaming rate with the access pattern of the dequantization kernel: each thread handles
// UNITS 16-byte chunks 4 KB apart (every load or store instruction covers 1 KB contiguous per
// wave) and issues all its loads first. mode bits 0-1: 0 read only (one float per work-group is
// written, so the loads stay), 1 write only (fill), 2 copy; bit 2: plain instead of
// non-temporal stores; bit 3: plain instead of non-temporal loads; bits 4-5: 4, 8 or 16 chunks
// per thread. The caller takes the best of the variants as the device's ceiling.
constexpr int kHbmThreads = 256;

template <int UNITS>
__global__ __launch_bounds__(kHbmThreads) void hbm_probe_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                                int64_t chunks, int mode, float* __restrict__ sums) {
    constexpr int kHbmUnits = UNITS;
    const bool plain = (mode & 4) != 0, plain_loads = (mode & 8) != 0;
    mode &= 3;
    const int64_t base = (int64_t)blockIdx.x * kHbmThreads * kHbmUnits + threadIdx.x;
    u32x4_t v[kHbmUnits];
    if (mode != 1) {
#pragma unroll
        for (int u = 0; u < kHbmUnits; ++u) {
            const int64_t c = base + (int64_t)u * kHbmThreads;
            v[u] = c >= chunks ? u32x4_t{0u, 0u, 0u, 0u}
                               : (plain_loads ? src[c] : __builtin_nontemporal_load(src + c));
        }
    } else {
#pragma unroll
        for (int u = 0; u < kHbmUnits; ++u) v[u] = u32x4_t{(uint32_t)u, 1u, 2u, 3u};
    }
    if (mode == 0) {
        uint32_t x = 0;
#pragma unroll
        for (int u = 0; u < kHbmUnits; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
        if (x == 0x9E3779B9u) sums[blockIdx.x] = (float)x;  // practically never: keeps the loads
        return;
    }
#pragma unroll
    for (int u = 0; u < kHbmUnits; ++u) {
        const int64_t c = base + (int64_t)u * kHbmThreads;
        if (c < chunks) {
            if (plain) dst[c] = v[u];
            else __builtin_nontemporal_store(v[u], dst + c);
        }
    }
}

template <int UNITS>
static hipError_t launch_hbm_probe_t(const void* src, void* dst, int64_t bytes, int mode, float* sums, hipStream_t s) {
    const int64_t chunks = bytes / 16;
    const int64_t per_wg = (int64_t)kHbmThreads * UNITS;
    const int64_t grid = (chunks + per_wg - 1) / per_wg;
    hipLaunchKernelGGL(hbm_probe_kernel<UNITS>, dim3((unsigned)grid), dim3(kHbmThreads), 0, s, (const u32x4_t*)src,
                       (u32x4_t*)dst, chunks, mode & 15, sums);
    return hipGetLastError();
}

hipError_t launch_hbm_probe(const void* src, void* dst, int64_t bytes, int mode, float* sums, hipStream_t s) {
    switch ((mode >> 4) & 3) {
        case 0: return launch_hbm_probe_t<4>(src, dst, bytes, mode, sums, s);
        case 1: return launch_hbm_probe_t<8>(src, dst, bytes, mode, sums, s);
        case 2: return launch_hbm_probe_t<16>(src, dst, bytes, mode, sums, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dk
