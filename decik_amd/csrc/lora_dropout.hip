// LoRA dropout around the rank-r products (the packed-mask path of LoRAPairFromNorm,
// solution/attn.py:129-180, 183-203, 251-271):
//   keep_pack:    bits[r, c / 8] bit (c % 8) = keep[r, c]            (skc_keep_pack_kernel)
//   inputs:       xq = fp16(x * (keep_q * scale_q)), xv likewise      (skc_lora_inputs_kernel)
//   input_grad:   out = (g_q * keep_q) * sq + (g_v * keep_v) * sv      (skc_lora_input_grad_kernel)
//                 in fp32 from the fp16 input gradients of both branches
//   lora_up:      G = fp16(GU . A)  [m, k]  (a branch's input gradient before the dropout mask)
// All elementwise in fp32 with the reference's order of operations (no FMA: the library is
// compiled with -ffp-contract=off), so the masks, inputs and input gradient are bit-exact.
// Each thread takes one mask byte (8 elements): 16- or 32-byte loads and stores.
#include "dk_internal.h"

namespace dk {

constexpr int kDropThreads = 256;

__global__ __launch_bounds__(kDropThreads) void lora_keep_pack_kernel(const uint8_t* __restrict__ kq,
                                                                      const uint8_t* __restrict__ kv,
                                                                      uint8_t* __restrict__ bq,
                                                                      uint8_t* __restrict__ bv,
                                                                      int64_t nbytes) {
    const int64_t i = (int64_t)blockIdx.x * kDropThreads + threadIdx.x;
    if (i >= nbytes) return;
    const u32x2_t q = *(const u32x2_t*)(kq + 8 * i), v = *(const u32x2_t*)(kv + 8 * i);
    uint32_t oq = 0, ov = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // byte j of the 8 (0 or 1 for a bool mask) shifted to bit j, as the reference ORs them
        oq |= ((q[j >> 2] >> (8 * (j & 3))) & 0xFFu) << j;
        ov |= ((v[j >> 2] >> (8 * (j & 3))) & 0xFFu) << j;
    }
    bq[i] = (uint8_t)oq;
    bv[i] = (uint8_t)ov;
}

template <bool X32>
__global__ __launch_bounds__(kDropThreads) void lora_dropout_inputs_kernel(
    const void* __restrict__ x, const uint8_t* __restrict__ bq, const uint8_t* __restrict__ bv,
    const float* __restrict__ scale_q, const float* __restrict__ scale_v, _Float16* __restrict__ xq,
    _Float16* __restrict__ xv, int64_t nbytes) {
    const int64_t i = (int64_t)blockIdx.x * kDropThreads + threadIdx.x;
    if (i >= nbytes) return;
    const float sq = *scale_q, sv = *scale_v;
    const uint32_t mq = bq[i], mv = bv[i];
    float xf[8];
    if constexpr (X32) {
        const float4_t a = *(const float4_t*)((const float*)x + 8 * i);
        const float4_t b = *(const float4_t*)((const float*)x + 8 * i + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xf[e] = a[e];
            xf[e + 4] = b[e];
        }
    } else {
        const half8_t h = *(const half8_t*)((const _Float16*)x + 8 * i);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = (float)h[e];
    }
    half8_t oq, ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        // the dropout value keep * scale is 0 or the scale exactly; x * 0 keeps x's sign
        const float dq = (float)((mq >> e) & 1u) * sq;
        const float dv = (float)((mv >> e) & 1u) * sv;
        oq[e] = (_Float16)(xf[e] * dq);
        ov[e] = (_Float16)(xf[e] * dv);
    }
    *(half8_t*)(xq + 8 * i) = oq;
    *(half8_t*)(xv + 8 * i) = ov;
}

__global__ __launch_bounds__(kDropThreads) void lora_input_grad_kernel(
    const _Float16* __restrict__ gq, const _Float16* __restrict__ gv, const uint8_t* __restrict__ bq,
    const uint8_t* __restrict__ bv, float sq, float sv, float* __restrict__ out, int64_t nbytes) {
    const int64_t i = (int64_t)blockIdx.x * kDropThreads + threadIdx.x;
    if (i >= nbytes) return;
    const uint32_t mq = bq[i], mv = bv[i];
    const half8_t a = *(const half8_t*)(gq + 8 * i), b = *(const half8_t*)(gv + 8 * i);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float tq = ((float)a[e] * (float)((mq >> e) & 1u)) * sq;
        const float tv = ((float)b[e] * (float)((mv >> e) & 1u)) * sv;
        o[e] = tq + tv;
    }
    *(float4_t*)(out + 8 * i) = float4_t{o[0], o[1], o[2], o[3]};
    *(float4_t*)(out + 8 * i + 4) = float4_t{o[4], o[5], o[6], o[7]};
}

// G[m, k] = fp16(sum_t GU[m, t] A[t, k]), fp32 accumulation in t order; one thread per 8
// consecutive k of one row.
template <int R>
__global__ __launch_bounds__(kDropThreads) void lora_up_kernel(const _Float16* __restrict__ gu,
                                                               const _Float16* __restrict__ a,
                                                               _Float16* __restrict__ out, int64_t m,
                                                               int64_t k) {
    const int64_t i = (int64_t)blockIdx.x * kDropThreads + threadIdx.x;  // chunk of 8 outputs
    const int64_t chunks = k / 8;
    if (i >= m * chunks) return;
    const int64_t row = i / chunks, k0 = (i - row * chunks) * 8;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const float g = (float)gu[row * R + t];
        const half8_t av = *(const half8_t*)(a + (int64_t)t * k + k0);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = acc[e] + g * (float)av[e];
    }
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (_Float16)acc[e];
    *(half8_t*)(out + row * k + k0) = o;
}

static inline unsigned drop_grid(int64_t n) { return (unsigned)((n + kDropThreads - 1) / kDropThreads); }

hipError_t launch_lora_keep_pack(const uint8_t* kq, const uint8_t* kv, uint8_t* bq, uint8_t* bv,
                                 int64_t nbytes, hipStream_t s) {
    if (nbytes == 0) return hipSuccess;
    hipLaunchKernelGGL(lora_keep_pack_kernel, dim3(drop_grid(nbytes)), dim3(kDropThreads), 0, s, kq, kv, bq, bv,
                       nbytes);
    return hipGetLastError();
}

hipError_t launch_lora_dropout_inputs(const void* x, bool x32, const uint8_t* bq, const uint8_t* bv,
                                      const float* sq, const float* sv, _Float16* xq, _Float16* xv,
                                      int64_t nbytes, hipStream_t s) {
    if (nbytes == 0) return hipSuccess;
    if (x32)
        hipLaunchKernelGGL(lora_dropout_inputs_kernel<true>, dim3(drop_grid(nbytes)), dim3(kDropThreads), 0, s, x, bq,
                           bv, sq, sv, xq, xv, nbytes);
    else
        hipLaunchKernelGGL(lora_dropout_inputs_kernel<false>, dim3(drop_grid(nbytes)), dim3(kDropThreads), 0, s, x,
                           bq, bv, sq, sv, xq, xv, nbytes);
    return hipGetLastError();
}

hipError_t launch_lora_input_grad(const _Float16* gq, const _Float16* gv, const uint8_t* bq, const uint8_t* bv,
                                  float sq, float sv, float* out, int64_t nbytes, hipStream_t s) {
    if (nbytes == 0) return hipSuccess;
    hipLaunchKernelGGL(lora_input_grad_kernel, dim3(drop_grid(nbytes)), dim3(kDropThreads), 0, s, gq, gv, bq, bv,
                       sq, sv, out, nbytes);
    return hipGetLastError();
}

hipError_t launch_lora_up(const _Float16* gu, const _Float16* a, int rank, _Float16* out, int64_t m, int64_t k,
                          hipStream_t s) {
    const int64_t n = m * (k / 8);
    if (n == 0) return hipSuccess;
    if (rank == 16)
        hipLaunchKernelGGL(lora_up_kernel<16>, dim3(drop_grid(n)), dim3(kDropThreads), 0, s, gu, a, out, m, k);
    else
        hipLaunchKernelGGL(lora_up_kernel<32>, dim3(drop_grid(n)), dim3(kDropThreads), 0, s, gu, a, out, m, k);
    return hipGetLastError();
}

}  // namespace dk
