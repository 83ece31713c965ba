// Fused NF4 dequant x fp16 product for launches with few token rows (m <= kGemvMaxM): the same
// Y = X.W^T + bias as nf4_fwd_kernel (solution/nf4.py:93-96) for the small-M regime (one token
// when decoding, a handful in a short batch), where the product is bound by reading the packed
// weight once. The MFMA kernels pad such launches to 32-token tiles and dequantize every weight
// for one useful multiply-add; here each weight is dequantized once and used for every token in
// fp32 dot products.
//
// Each wave owns RW consecutive weight rows (four waves per work-group): lane l takes 16-byte
// chunks l, l + 64, ... of each row (32 weights of one block each; every load instruction reads
// 1 KB contiguous of one row), dequantizes them to the reference's fp16 bits through a byte-pair
// code book (one 8-byte LDS read per packed byte), and accumulates v_dot2_f32_f16 products with
// the matching 32 values of every token row of X (fp32 accumulation). One X fragment serves the
// RW rows: with RW = 4, X (read from the caches) costs a quarter of what it costs with a row per
// wave, where it was read four times for every packed byte (7B gate at one token: 23 -> 18 us).
// Launches with few rows (long ones: 7B down) keep RW = 1 for enough waves to cover the memory
// latency. A butterfly reduction over the wave's lanes finishes each dot product; lanes 0..RW-1
// add the bias, round once to fp16 and store.
#include "dk_internal.h"

namespace dk {

constexpr int kGemvThreads = 256;  // four waves

template <int MT, bool NESTED, int kGemvRows>
__global__ __launch_bounds__(kGemvThreads) void nf4_gemv_kernel(const FwdArgs a) {
    // byte-pair code books: entry 256 g + b holds (code_g[b >> 4], code_g[b & 15]), the two
    // weights of packed byte b
    __shared__ float2_t lut2[256 * kMaxGroups];
    for (int gg = 0; gg < a.ngroups; ++gg) {
        const float* code = a.g[gg].w.code;
        lut2[256 * gg + threadIdx.x] = float2_t{code[threadIdx.x >> 4], code[threadIdx.x & 15]};
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    // this wave's first row among the launch's rows (groups back to back, col_begin = first row;
    // groups have n % 8 == 0, so a wave's rows lie in one group)
    const int row0 = (blockIdx.x * (kGemvThreads / 64) + wave) * kGemvRows;
    if (row0 >= a.ncols) return;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && row0 >= a.g[i].col_begin) gi = i;
    const FwdGroupDev& G = a.g[gi];
    const NF4Dev& W = G.w;
    const int n0 = row0 - G.col_begin;
    const int K = a.k, M = a.m;
    const int64_t rowb = (int64_t)(K >> 1);  // packed bytes per row
    const char* book = (const char*)(lut2 + 256 * gi);
    const float offset = NESTED ? *W.offset : 0.0f;

    float acc[kGemvRows][MT];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
    // chunk c = 16 packed bytes = 32 weights of one block (k % 32 == 0, blocks >= 32, aligned)
    for (int c = lane; c < (K >> 5); c += 64) {
        u32x4_t p[kGemvRows];
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) p[r] = *(const u32x4_t*)(W.packed + (int64_t)(n0 + r) * rowb + 16 * c);
        float s[kGemvRows];
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) {
            const int64_t blk = ((int64_t)(n0 + r) * K + 32 * c) >> W.bs_shift;
            if constexpr (NESTED) {
                s[r] = W.code2[W.absmax8[blk]] * W.absmax2[blk >> W.bs2_shift];
                s[r] = s[r] + offset;
            } else {
                s[r] = W.absmaxf[blk];
            }
        }
        // the 32 X values of this chunk for every token row (elements copied to scalars:
        // hipcc compiles __builtin_bit_cast of a vector element v[j] as element 0 whatever j is)
        uint32_t xs[MT][16];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < M) {
                const u32x4_t* xp = (const u32x4_t*)(a.x + (int64_t)m * a.ldx + 32 * c);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const u32x4_t xv = xp[e];
                    xs[m][4 * e + 0] = xv[0];
                    xs[m][4 * e + 1] = xv[1];
                    xs[m][4 * e + 2] = xv[2];
                    xs[m][4 * e + 3] = xv[3];
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) xs[m][q] = 0u;
            }
        }
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) {
            // the reference's fp16 bits of the row's 32 weights: pair q of dword e = weights
            // 8 e + 2 q, + 1
            const uint32_t pw[4] = {p[r][0], p[r][1], p[r][2], p[r][3]};
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float2_t cv = *(const float2_t*)(book + (((pw[e] >> (8 * q)) & 0xFFu) << 3));
                    const uint32_t w2 = pack_half2(cv.x * s[r], cv.y * s[r]);
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        acc[r][m] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w2),
                                                           __builtin_bit_cast(half2_t, xs[m][4 * e + q]), acc[r][m],
                                                           false);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) acc[r][m] += __shfl_xor(acc[r][m], o, 64);
    if (lane < kGemvRows) {
        // lane r stores row n0 + r (the butterfly left every lane with every total)
        float v[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            v[m] = acc[0][m];
#pragma unroll
            for (int r = 1; r < kGemvRows; ++r)
                if (lane == r) v[m] = acc[r][m];
        }
        const int n = n0 + lane;
        const float b = G.bias != nullptr ? (float)G.bias[n] : 0.0f;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < M) G.y[(int64_t)m * G.ldy + n] = to_half(v[m] + b);
    }
}

template <int MT, int RW>
static hipError_t launch_gemv_rw(const FwdArgs& a, hipStream_t s) {
    const int rows_per_wg = (kGemvThreads / 64) * RW;
    const int grid = (a.ncols + rows_per_wg - 1) / rows_per_wg;
    if (a.nested)
        hipLaunchKernelGGL((nf4_gemv_kernel<MT, true, RW>), dim3(grid), dim3(kGemvThreads), 0, s, a);
    else
        hipLaunchKernelGGL((nf4_gemv_kernel<MT, false, RW>), dim3(grid), dim3(kGemvThreads), 0, s, a);
    return hipGetLastError();
}

// four rows per wave while that still gives four waves per SIMD on a 256-CU device
template <int MT>
static hipError_t launch_gemv_t(const FwdArgs& a, hipStream_t s) {
    return a.ncols >= 4 * 4 * 1024 ? launch_gemv_rw<MT, 4>(a, s) : launch_gemv_rw<MT, 1>(a, s);
}

hipError_t launch_gemv(const FwdArgs& a, hipStream_t s) {
    if (a.m < 1 || a.m > kGemvMaxM || a.glu) return hipErrorInvalidValue;
    for (int g = 0; g < a.ngroups; ++g)
        if (a.g[g].lora_u != nullptr) return hipErrorInvalidValue;
    if (a.m == 1) return launch_gemv_t<1>(a, s);
    if (a.m == 2) return launch_gemv_t<2>(a, s);
    if (a.m <= 4) return launch_gemv_t<4>(a, s);
    return launch_gemv_t<8>(a, s);
}

}  // namespace dk
