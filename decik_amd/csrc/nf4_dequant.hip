// Standalone NF4 dequantization (HBM-bound): packed uint8 + double-quant statistics -> fp16.
//
// Replaces skc_nf4_dequant_kernel (solution/nf4.py:27-48). Each thread owns 16 packed bytes
// (32 weights; with blocksize % 32 == 0 they share one scale), loads them with one 16-byte
// load, and writes 64 bytes of fp16 with four 16-byte stores. The 16-entry code book lives in
// LDS. Several weights can share one launch (dk_nf4_dequant_batched): the grid is the
// concatenation of each weight's work-groups.
#include "dk_internal.h"

namespace dk {

__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_kernel(const DequantArgs a) {
    __shared__ float lut[16];
    const int tid = threadIdx.x;
    const int bid = blockIdx.x;
    // pick this work-group's weight (uniform, scalar selects)
    int wi = 0;
#pragma unroll
    for (int j = 1; j < kMaxDequantBatch; ++j)
        if (j < a.count && bid >= a.wg_begin[j]) wi = j;
    NF4Dev w = a.w[0];
    uint16_t* out = a.out[0];
    int64_t nbytes = a.nbytes[0];
    int wg0 = a.wg_begin[0];
#pragma unroll
    for (int j = 1; j < kMaxDequantBatch; ++j)
        if (j == wi) {
            w = a.w[j];
            out = a.out[j];
            nbytes = a.nbytes[j];
            wg0 = a.wg_begin[j];
        }
    if (tid < 16) lut[tid] = w.code[tid];
    __syncthreads();

    const bool nested = w.absmax8 != nullptr;
    const float offset = nested ? *w.offset : 0.0f;
    const int64_t b0 = ((int64_t)(bid - wg0) * kDequantThreads + tid) * 16;
    if (b0 >= nbytes) return;

    if (a.fast[wi] && b0 + 16 <= nbytes) {
        const u32x4_t p = __builtin_nontemporal_load((const u32x4_t*)(w.packed + b0));
        const int64_t blk = block_of(w, 2 * b0);
        const float s = nested ? block_scale<true>(w, blk, w.code2, offset)
                               : block_scale<false>(w, blk, w.code2, offset);
        uint32_t o[16];
        dequant16(p, s, lut, o);
        u32x4_t* dst = (u32x4_t*)(out + 2 * b0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4_t v = {o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
            __builtin_nontemporal_store(v, dst + q);
        }
    } else {
        // generic path: any even blocksize, unaligned pointers, the tail of the tensor
        const int64_t end = b0 + 16 < nbytes ? b0 + 16 : nbytes;
        for (int64_t i = b0; i < end; ++i) {
            const int64_t blk = block_of(w, 2 * i);
            const float s = nested ? block_scale<true>(w, blk, w.code2, offset)
                                   : block_scale<false>(w, blk, w.code2, offset);
            const uint32_t b = w.packed[i];
            const uint32_t v = pack_half2(lut[b >> 4] * s, lut[b & 15u] * s);
            out[2 * i] = (uint16_t)(v & 0xFFFFu);
            out[2 * i + 1] = (uint16_t)(v >> 16);
        }
    }
}

}  // namespace dk
