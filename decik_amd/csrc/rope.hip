// Rotary position embedding of the attention inputs (skc_rope_fwd_kernel / skc_rope_bwd_kernel,
// solution/attn.py:27-86), one launch each way for q and k:
//   forward:  q = fp32(q_base) + fp32(q_lora);  out = q * cos + rotate_half(q) * sin   (fp32)
//             stored fp16 head-major [H, T, D] (as SDPA takes it); k likewise without LoRA
//   backward: d = g * cos + rotate_half^T(g * sin), fp32, rounded to fp16 once, token-major
// rotate_half(q)[d] = -q[d + D/2] for d < D/2, q[d - D/2] otherwise. Elementwise fp32 in the
// reference's order (no FMA: the library is compiled with -ffp-contract=off), so bit-exact.
// One thread per 8 consecutive d of one (token, head): 16-byte loads and stores; D % 16 == 0, so
// the 8 values and their partners lie in one half of the head.
#include "dk_internal.h"

namespace dk {

constexpr int kRopeThreads = 256;

// Work item w of a launch: q items first (n_tok * hq * D / 8), then k items.
__global__ __launch_bounds__(kRopeThreads) void rope_fwd_kernel(const RopeArgs a) {
    const int64_t w = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x;
    const int cpd = a.d / 8;  // chunks per head
    const int64_t nq = a.n_tok * a.hq * cpd;
    const bool isq = w < nq;
    const int64_t wi = isq ? w : w - nq;
    const int heads = isq ? a.hq : a.hk;
    if (wi >= a.n_tok * heads * cpd) return;
    const int64_t t = wi / (heads * cpd);
    const int rem = (int)(wi - t * heads * cpd);
    const int h = rem / cpd, d0 = (rem - h * cpd) * 8;
    const int half = a.d / 2;
    const int dj0 = d0 < half ? d0 + half : d0 - half;  // the partners of d0 .. d0 + 7
    const _Float16* base = isq ? a.q_base : a.k;
    const _Float16* lora = isq ? a.q_lora : nullptr;
    const int64_t ld = isq ? a.ldq : a.ldk;
    const _Float16* row = base + t * ld + (int64_t)h * a.d;
    const half8_t bi = *(const half8_t*)(row + d0), bj = *(const half8_t*)(row + dj0);
    float qi[8], qj[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        qi[e] = (float)bi[e];
        qj[e] = (float)bj[e];
    }
    if (lora != nullptr) {
        const _Float16* lrow = lora + t * a.ldl + (int64_t)h * a.d;
        const half8_t li = *(const half8_t*)(lrow + d0), lj = *(const half8_t*)(lrow + dj0);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qi[e] = qi[e] + (float)li[e];
            qj[e] = qj[e] + (float)lj[e];
        }
    }
    const float4_t c0 = *(const float4_t*)(a.cos + t * a.d + d0), c1 = *(const float4_t*)(a.cos + t * a.d + d0 + 4);
    const float4_t s0 = *(const float4_t*)(a.sin + t * a.d + d0), s1 = *(const float4_t*)(a.sin + t * a.d + d0 + 4);
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float c = e < 4 ? c0[e] : c1[e - 4], s = e < 4 ? s0[e] : s1[e - 4];
        const float rot = d0 < half ? -qj[e] : qj[e];
        o[e] = (_Float16)(qi[e] * c + rot * s);
    }
    _Float16* out = (isq ? a.q_out : a.k_out) + ((int64_t)h * a.n_tok + t) * a.d + d0;
    *(half8_t*)out = o;
}

__global__ __launch_bounds__(kRopeThreads) void rope_bwd_kernel(const RopeArgs a) {
    const int64_t w = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x;
    const int cpd = a.d / 8;
    const int64_t nq = a.n_tok * a.hq * cpd;
    const bool isq = w < nq;
    const int64_t wi = isq ? w : w - nq;
    const int heads = isq ? a.hq : a.hk;
    if (wi >= a.n_tok * heads * cpd) return;
    const int64_t t = wi / (heads * cpd);
    const int rem = (int)(wi - t * heads * cpd);
    const int h = rem / cpd, d0 = (rem - h * cpd) * 8;
    const int half = a.d / 2;
    const int dj0 = d0 < half ? d0 + half : d0 - half;
    const _Float16* g = (isq ? a.grad_q : a.grad_k) + ((int64_t)h * a.n_tok + t) * a.d;
    const half8_t gi = *(const half8_t*)(g + d0), gj = *(const half8_t*)(g + dj0);
    const float* cr = a.cos + t * a.d;
    const float* sr = a.sin + t * a.d;
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = (float)gi[e] * cr[d0 + e];
        const float y = (float)gj[e] * sr[dj0 + e];
        o[e] = (_Float16)(x + (d0 < half ? y : -y));
    }
    _Float16* out = (isq ? a.dq : a.dk) + t * (isq ? a.lddq : a.lddk) + (int64_t)h * a.d + d0;
    *(half8_t*)out = o;
}

hipError_t launch_rope(const RopeArgs& a, bool backward, hipStream_t s) {
    const int64_t items = a.n_tok * (int64_t)(a.hq + a.hk) * (a.d / 8);
    if (items == 0) return hipSuccess;
    const unsigned grid = (unsigned)((items + kRopeThreads - 1) / kRopeThreads);
    if (backward)
        hipLaunchKernelGGL(rope_bwd_kernel, dim3(grid), dim3(kRopeThreads), 0, s, a);
    else
        hipLaunchKernelGGL(rope_fwd_kernel, dim3(grid), dim3(kRopeThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dk
