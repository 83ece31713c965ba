// Standalone NF4 dequantization (HBM-bound): packed uint8 + double-quant statistics -> fp16.
//
// Replaces skc_nf4_dequant_kernel (solution/nf4.py:27-48). A work-group covers
// kDequantUnits x 256 units of one packed dword (8 weights; with a power-of-two blocksize >= 32
// a unit lies in one block, so it has one scale). The work-group first forms the scale of each
// of its blocks once (one thread per block: statistics loads, fp32 scale into an LDS table)
// while its packed loads are in flight; each thread then unpacks and writes 16 bytes of fp16 per
// unit with a non-temporal store. Per-unit statistics loads (two small loads per unit) made the
// kernel issue three loads per store; with the table it streams HBM-resident weights at 5.8
// TB/s instead of 4.4. Consecutive lanes own consecutive units, so every load and store
// instruction is contiguous per wave. The code book and the code2 table sit in LDS. Loads are buffer
// loads relative to the work-group's first byte, so offsets stay 32-bit for any tensor size
// and past-the-end reads give zeros. Several weights can share one launch
// (dk_nf4_dequant_batched): the grid is the concatenation of each weight's work-groups.
#include "gemm_common.h"

namespace dk {

__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_kernel(const DequantArgs a) {
    __shared__ float lut[16];
    __shared__ float c2[256];
    const int tid = threadIdx.x;
    const int bid = blockIdx.x;
    int wi = 0;  // this work-group's weight
#pragma unroll
    for (int j = 1; j < kMaxDequantBatch; ++j)
        if (j < a.count && bid >= a.wg_begin[j]) wi = j;
    wi = __builtin_amdgcn_readfirstlane(wi);
    const NF4Dev& w = a.w[wi];
    const bool nested = w.absmax8 != nullptr;
    if (tid < 16) lut[tid] = w.code[tid];
    if (nested) c2[tid] = w.code2[tid];
    const float offset = nested ? *w.offset : 0.0f;
    const int64_t nbytes = a.nbytes[wi];
    uint16_t* const out = a.out[wi];
    constexpr int64_t kSpan = (int64_t)kDequantThreads * 4 * kDequantUnits;  // bytes per work-group
    const int64_t base = (int64_t)(bid - a.wg_begin[wi]) * kSpan;
    __syncthreads();

    if (!a.fast[wi]) {
        // generic path: any even blocksize, unaligned pointers
        const int64_t end = base + kSpan < nbytes ? base + kSpan : nbytes;
        for (int64_t i = base + tid; i < end; i += kDequantThreads) {
            const int64_t blk = block_of(w, 2 * i);
            const float s = nested ? block_scale<true>(w, blk, c2, offset) : block_scale<false>(w, blk, c2, offset);
            const uint32_t b = w.packed[i];
            const uint32_t v = pack_half2(lut[b >> 4] * s, lut[b & 15u] * s);
            out[2 * i] = (uint16_t)(v & 0xFFFFu);
            out[2 * i + 1] = (uint16_t)(v >> 16);
        }
        return;
    }

    // fast path: units of one packed dword (8 weights, one scale) per lane; each load instruction
    // reads 256 contiguous bytes per wave and each store writes 1 KB contiguous per wave
    const int64_t left = nbytes - base;  // > 0
    const uint32_t span = (uint32_t)(left < kSpan ? left : kSpan);
    const rsrc_t prs = make_rsrc(w.packed + base, span);
    const uint32_t bs_shift = sgpr((uint32_t)w.bs_shift);
    const int64_t blk0 = (2 * base) >> bs_shift;  // first block of the work-group
    // The work-group's block scales, once per block: thread i computes block blk0 + i (and
    // blk0 + i + 256, ...) into an LDS table, so each unit reads its scale from LDS instead of
    // issuing two global loads of its own. Order: statistics loads, then the packed loads, then
    // the scales are formed while the packed bytes are in flight.
    const int64_t blk_end = (2 * (base + (int64_t)span) - 1) >> bs_shift;  // last block touched
    const int nbw = (int)(blk_end - blk0 + 1);
    constexpr int kSB = 2 * kDequantThreads * 4 * kDequantUnits / 32;  // blocks per span at blocksize 32
    constexpr int kSPT = (kSB + kDequantThreads - 1) / kDequantThreads;  // scales per thread
    __shared__ float sct[kSB];
    uint32_t q8[kSPT];
    float a2[kSPT];
#pragma unroll
    for (int j = 0; j < kSPT; ++j) {
        const int i = tid + j * kDequantThreads;
        const int64_t blk = blk0 + i;
        const bool ok = i < nbw;
        if (nested) {
            q8[j] = ok ? (uint32_t)w.absmax8[blk] : 0u;
            a2[j] = ok ? w.absmax2[group_of(w, blk)] : 0.0f;
        } else {
            q8[j] = 0;
            a2[j] = ok ? w.absmaxf[blk] : 0.0f;
        }
    }
    asm volatile("" ::: "memory");  // the packed loads stay behind the statistics loads
    uint32_t p[kDequantUnits];
#pragma unroll
    for (int u = 0; u < kDequantUnits; ++u) {
        const uint32_t off = (uint32_t)(u * kDequantThreads + tid) * 4u;  // within the span
        p[u] = __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(off + 4u <= span ? off : kOOB), 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kSPT; ++j) {
        const int i = tid + j * kDequantThreads;
        if (i < nbw) sct[i] = nested ? c2[q8[j]] * a2[j] + offset : a2[j];  // two roundings (no contraction)
    }
    lds_barrier();
#pragma unroll
    for (int u = 0; u < kDequantUnits; ++u) {
        const uint32_t off = (uint32_t)(u * kDequantThreads + tid) * 4u;
        if (off >= span) break;
        if (off + 4u > span) {
            // the tensor's last, partial unit
            for (int64_t i = base + off; i < nbytes; ++i) {
                const int64_t blk = block_of(w, 2 * i);
                const float s = nested ? block_scale<true>(w, blk, c2, offset) : block_scale<false>(w, blk, c2, offset);
                const uint32_t b = w.packed[i];
                const uint32_t v = pack_half2(lut[b >> 4] * s, lut[b & 15u] * s);
                out[2 * i] = (uint16_t)(v & 0xFFFFu);
                out[2 * i + 1] = (uint16_t)(v >> 16);
            }
            break;
        }
        const float s = sct[((2 * (base + off)) >> bs_shift) - blk0];
        uint32_t o[4];
        dequant4(p[u], s, lut, o);
        __builtin_nontemporal_store(u32x4_t{o[0], o[1], o[2], o[3]}, (u32x4_t*)(out + 2 * (base + off)));
    }
}

// fp32 scale of every block (solution/nf4.py:37-43): nested
// fp32(fp32(code2[q] * absmax2[block / blocksize2]) + offset), plain absmax itself. The same two
// roundings as the dequantization, so a plain-statistics dequantization with these scales gives
// bit-identical weights.
__global__ __launch_bounds__(256) void nf4_block_scales_kernel(const NF4Dev w, int64_t nblocks, float* out) {
    __shared__ float c2[256];
    const bool nested = w.absmax8 != nullptr;
    if (nested) c2[threadIdx.x] = w.code2[threadIdx.x];
    __syncthreads();
    const float offset = nested ? *w.offset : 0.0f;
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    out[b] = nested ? block_scale<true>(w, b, c2, offset) : block_scale<false>(w, b, c2, offset);
}

hipError_t launch_block_scales(const NF4Dev& w, int64_t nblocks, float* out, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t grid = (nblocks + 255) / 256;
    hipLaunchKernelGGL(nf4_block_scales_kernel, dim3((unsigned)grid), dim3(256), 0, s, w, nblocks, out);
    return hipGetLastError();
}

}  // namespace dk
