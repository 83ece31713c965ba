// Fused NF4 dequant x fp16 product for launches with few token rows (m <= kGemvMaxM): the same
// Y = X.W^T + bias as nf4_fwd_kernel (solution/nf4.py:93-96) for the small-M regime (one token
// when decoding, a handful in a short batch), where the product is bound by reading the packed
// weight once. The MFMA kernels pad such launches to 32-token tiles and dequantize every weight
// for one useful multiply-add; here each weight is dequantized once and used for every token in
// fp32 dot products.
//
// One wave per weight row (four per work-group): lane l takes 16-byte chunks l, l + 64, ... of the
// row (32 weights of one block each; every load instruction reads 1 KB contiguous), dequantizes
// them to the reference's fp16 bits through a byte-pair code book (one 8-byte LDS read per packed
// byte), and accumulates v_dot2_f32_f16 products with the matching 32 values of every token row of
// X (fp32 accumulation). A butterfly reduction over
// the wave's lanes finishes each dot product; lane 0 adds the bias, rounds once to fp16 and stores.
#include "dk_internal.h"

namespace dk {

constexpr int kGemvThreads = 256;  // four waves, one weight row each

template <int MT, bool NESTED>
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

    // this wave's row among the launch's rows (groups back to back, col_begin = first row)
    const int row = blockIdx.x * (kGemvThreads / 64) + wave;
    if (row >= a.ncols) return;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && row >= a.g[i].col_begin) gi = i;
    const FwdGroupDev& G = a.g[gi];
    const NF4Dev& W = G.w;
    const int n = row - G.col_begin;
    const int K = a.k, M = a.m;
    const u32x4_t* prow = (const u32x4_t*)(W.packed + (int64_t)n * (K >> 1));
    const int64_t flat0 = (int64_t)n * K;
    const char* book = (const char*)(lut2 + 256 * gi);
    const float offset = NESTED ? *W.offset : 0.0f;

    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    // chunk c = 16 packed bytes = 32 weights of one block (k % 32 == 0, blocks >= 32, aligned)
    for (int c = lane; c < (K >> 5); c += 64) {
        const u32x4_t p = prow[c];
        const int64_t blk = (flat0 + 32 * c) >> W.bs_shift;
        float s;
        if constexpr (NESTED) {
            s = W.code2[W.absmax8[blk]] * W.absmax2[blk >> W.bs2_shift];
            s = s + offset;
        } else {
            s = W.absmaxf[blk];
        }
        // the reference's fp16 bits of the 32 weights: pair q of dword e = weights 8 e + 2 q, + 1
        uint32_t w[16];
        const uint32_t pw[4] = {p[0], p[1], p[2], p[3]};
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float2_t cv = *(const float2_t*)(book + (((pw[e] >> (8 * q)) & 0xFFu) << 3));
                w[4 * e + q] = pack_half2(cv.x * s, cv.y * s);
            }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < M) {
                const u32x4_t* xp = (const u32x4_t*)(a.x + (int64_t)m * a.ldx + 32 * c);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const u32x4_t xv = xp[e];
                    // elements copied to scalars first: hipcc compiles __builtin_bit_cast of a
                    // vector element (v[j]) as element 0 whatever j is
                    const uint32_t xs[4] = {xv[0], xv[1], xv[2], xv[3]};
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[m] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w[4 * e + q]),
                                                        __builtin_bit_cast(half2_t, xs[q]), acc[m], false);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o, 64);
    if (lane == 0) {
        const float b = G.bias != nullptr ? (float)G.bias[n] : 0.0f;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < M) G.y[(int64_t)m * G.ldy + n] = to_half(acc[m] + b);
    }
}

template <int MT>
static hipError_t launch_gemv_t(const FwdArgs& a, hipStream_t s) {
    const int grid = (a.ncols + kGemvThreads / 64 - 1) / (kGemvThreads / 64);
    if (a.nested)
        hipLaunchKernelGGL((nf4_gemv_kernel<MT, true>), dim3(grid), dim3(kGemvThreads), 0, s, a);
    else
        hipLaunchKernelGGL((nf4_gemv_kernel<MT, false>), dim3(grid), dim3(kGemvThreads), 0, s, a);
    return hipGetLastError();
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
