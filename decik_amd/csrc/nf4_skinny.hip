// Fused NF4 dequant x fp16 product for forward launches of few token rows (m <= 32): the same
// Y = X.W^T + bias as the other forward kernels (solution/nf4.py:93-96) in the regime where the
// call is bound by streaming the packed weight from HBM once (decoding, short batches). The
// MFMA kernels for many tokens pad such launches to 224-288-token tiles; here the token count
// is padded only to 16 (MT = 1) or 32 (MT = 2) and the kernel is organised around the weight
// stream:
//
// - A work-group (8 waves) owns RT row tiles of 16 weight rows (RT = 4; 5 or 6 where 64-row
//   groups would overrun one work-group per CU, so that a tall weight runs in one round instead of
//   two whose second is mostly idle) and one contiguous range of the contraction (split-K over
//   work-groups only where the rows alone cannot fill the GPU).
//   Its waves take the range's 128-wide super-steps in turn, so every wave streams whole rows
//   and the fp32 tiles of the 8 waves are summed through LDS in wave order at the end.
// - Per super-step a lane loads 16 contiguous packed bytes (32 weights, one block: blocks are
//   powers of two >= 32) of each of its 4 rows -- lanes 16 g .. 16 g + 15 read bytes
//   16 g .. 16 g + 15 of the step's 64-byte row segment, so each load instruction covers 16 rows
//   x 64 contiguous bytes -- and the matching 64 bytes of X for each 16-token block. The next
//   super-step's loads are issued before this one is computed.
// - v_mfma_f32_16x16x32_f16 with A = dequantized weights (16 rows x 32), B = X^T (32 x 16
//   tokens). MFMA t (t = 0..3) of a super-step contracts lane group g's dword t, i.e. k =
//   k0 + 32 g + 8 t + e (a permutation of the step's 128 k that A and B share).
// - Dequantization as in the other kernels: byte-pair code book in LDS (one 8-byte read per
//   packed byte), fp32 multiply by the block scale, one fp16 rounding: the reference's bits.
#include "gemm_common.h"

namespace dk {

constexpr int kSkWaves = 8;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkStep = 128;   // contraction per super-step

// the waves' fp32 tiles for the reduction (rows padded to 16 RT + 1 floats)
__host__ __device__ constexpr size_t skinny_smem_bytes(int mt, int rt) {
    return (size_t)kSkWaves * 16 * mt * (16 * rt + 1) * 4;
}

template <int MT, bool NESTED, int RT>
__global__ __launch_bounds__(kSkThreads) void nf4_skinny_kernel(const FwdArgs a) {
    constexpr int kSkRows = 16 * RT;  // weight rows per work-group
    constexpr int kSkPad = kSkRows + 1;
    __shared__ float2_t lut2[256];  // byte-pair code book of this work-group's weight
    __shared__ float c2[256];       // nested statistics: the code2 table
    extern __shared__ __attribute__((aligned(16))) float red[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;

    const int rg = (int)blockIdx.x / a.splits;  // row group over all groups' rows
    const int split = (int)blockIdx.x - rg * a.splits;
    int gi = 0;
#pragma unroll
    for (int q = 1; q < kMaxGroups; ++q)
        if (q < a.ngroups && rg >= a.g[q].tile_begin) gi = q;
    gi = __builtin_amdgcn_readfirstlane(gi);
    const FwdGroupDev& G = a.g[gi];
    const NF4Dev& W = G.w;
    const int M = a.m, K = a.k, N = (int)W.n, ldx = (int)a.ldx;
    const int n0 = (rg - G.tile_begin) * kSkRows;

    {
        const float* book = W.code;
        if (tid < 256) lut2[tid] = float2_t{book[tid >> 4], book[tid & 15]};
        if (NESTED && tid >= 256) c2[tid - 256] = W.code2[tid - 256];
    }
    const float offset = NESTED ? *W.offset : 0.0f;

    const rsrc_t wrs = make_rsrc(W.packed, W.packed_bytes);
    const rsrc_t ars = make_rsrc(NESTED ? (const void*)W.absmax8 : (const void*)W.absmaxf, W.absmax_bytes);
    const rsrc_t a2rs = make_rsrc(W.absmax2, NESTED ? W.absmax2_bytes : 0u);
    const rsrc_t xrs = make_rsrc(a.x, a.x_bytes);
    const uint32_t bs_shift = W.bs_shift, bs2_shift = W.bs2_shift;

    // this lane's rows (A row i of tile r) and token rows (B column i of token block b)
    uint32_t wbase[RT];
    bool rok[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int row = n0 + 16 * r + i;
        rok[r] = row < N;
        wbase[r] = (uint32_t)(rok[r] ? row : 0) * (uint32_t)K + 32u * (uint32_t)g;  // flat element index
    }
    bool tok[MT];
#pragma unroll
    for (int b = 0; b < MT; ++b) tok[b] = 16 * b + i < M;

    const int total = (K + kSkStep - 1) / kSkStep;
    const int s0 = split * a.ksteps_per_split;
    const int s1 = min(total, s0 + a.ksteps_per_split);

    float4_t acc[RT][MT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int b = 0; b < MT; ++b) acc[r][b] = float4_t{};

    // loads of one super-step: packed bytes and block scale of each row, X of each token block
    struct Step {
        u32x4_t p[RT];
        float s[RT];
        uint32_t q8[RT];  // nested: absmax codes (the scale is completed after the wait)
        u32x4_t x[MT][4];
    };
    auto load = [&](int ss, Step& st) __attribute__((always_inline)) {
        const int k = ss * kSkStep + 32 * g;
        const bool kok = ss < s1 && k < K;  // K % 32 == 0: a lane's 32 k are wholly in or out
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint32_t el = wbase[r] + (uint32_t)ss * kSkStep;
            st.p[r] = bload128(wrs, off_if(kok && rok[r], el >> 1));
            const uint32_t blk = el >> bs_shift;
            if constexpr (NESTED) {
                st.q8[r] = bload8(ars, off_if(kok && rok[r], blk));
                st.s[r] = bloadf(a2rs, off_if(kok && rok[r], (blk >> bs2_shift) * 4u));
            } else {
                st.s[r] = bloadf(ars, off_if(kok && rok[r], blk * 4u));
            }
        }
#pragma unroll
        for (int b = 0; b < MT; ++b)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                st.x[b][t] = bload128(xrs, off_if(kok && tok[b], (uint32_t)((tok[b] ? 16 * b + i : 0) * ldx + k + 8 * t) * 2u));
    };
    auto compute = [&](const Step& st) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            float s = st.s[r];
            if constexpr (NESTED) s = c2[st.q8[r]] * s + offset;  // two roundings (no contraction)
            if (!rok[r]) s = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t w = st.p[r][t];
                u32x4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float2_t cv = *(const float2_t*)((const char*)lut2 + (((w >> (8 * e)) & 0xFFu) << 3));
                    o[e] = pack_half2(cv.x * s, cv.y * s);
                }
                const half8_t av = __builtin_bit_cast(half8_t, o);
#pragma unroll
                for (int b = 0; b < MT; ++b)
                    acc[r][b] = mfma16x16x32(av, __builtin_bit_cast(half8_t, st.x[b][t]), acc[r][b]);
            }
        }
    };

    // this wave's super-steps: s0 + wave, s0 + wave + 8, ... (the loads of the next are in flight
    // while one is computed; past the range they read zeros)
    // Ping-pong: a step is computed while the next one's loads are in flight. The scheduling
    // barriers keep the loads ahead of the computation (the compiler otherwise sinks them below
    // it and every step waits a full memory round trip).
    Step sa, sb;
    int ss = s0 + wave;
    load(ss, sa);
    __syncthreads();  // the code book in LDS (the first step's loads are already in flight)
    while (ss < s1) {
        load(ss + kSkWaves, sb);
        __builtin_amdgcn_sched_barrier(0);
        compute(sa);
        __builtin_amdgcn_sched_barrier(0);
        if (ss + kSkWaves >= s1) break;
        load(ss + 2 * kSkWaves, sa);
        __builtin_amdgcn_sched_barrier(0);
        compute(sb);
        __builtin_amdgcn_sched_barrier(0);
        ss += 2 * kSkWaves;
    }

    // lane holds D[4 g + r'][i] of tile r, token block b: weight row n0 + 16 r + 4 g + r',
    // token 16 b + i. Stage as red[wave][token][row] (rows padded to 65 floats).
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int b = 0; b < MT; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                red[(wave * 16 * MT + 16 * b + i) * kSkPad + 16 * r + 4 * g + q] = acc[r][b][q];
    __syncthreads();
    const bool split_out = a.splits > 1;
    for (int t = tid; t < 16 * MT * kSkRows; t += kSkThreads) {
        const int m = t / kSkRows, row = t - m * kSkRows;  // consecutive threads: consecutive rows
        const int n = n0 + row;
        if (m >= M || n >= N) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kSkWaves; ++w) v += red[(w * 16 * MT + m) * kSkPad + row];
        if (split_out) {
            a.partials[((int64_t)split * M + m) * a.ncols + G.col_begin + n] = v;
        } else {
            if (G.bias != nullptr) v += (float)G.bias[n];
            G.y[(int64_t)m * G.ldy + n] = to_half(v);
        }
    }
}

template <int MT, bool NESTED, int RT>
static hipError_t launch_skinny_t(const FwdArgs& a, int grid, hipStream_t s) {
    const size_t lds = skinny_smem_bytes(MT, RT);
    const hipError_t e = allow_dynamic_lds((const void*)nf4_skinny_kernel<MT, NESTED, RT>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((nf4_skinny_kernel<MT, NESTED, RT>), dim3(grid), dim3(kSkThreads), lds, s, a);
    return hipGetLastError();
}

template <int RT>
static hipError_t launch_skinny_rt(const FwdArgs& a, int grid, hipStream_t s) {
    if (a.m <= 16) return a.nested ? launch_skinny_t<1, true, RT>(a, grid, s) : launch_skinny_t<1, false, RT>(a, grid, s);
    return a.nested ? launch_skinny_t<2, true, RT>(a, grid, s) : launch_skinny_t<2, false, RT>(a, grid, s);
}

hipError_t launch_skinny(const FwdArgs& a, int row_tiles, int grid, hipStream_t s) {
    if (a.m < 1 || a.m > kSkinnyMaxM || a.glu) return hipErrorInvalidValue;
    for (int g = 0; g < a.ngroups; ++g)
        if (a.g[g].lora_u != nullptr) return hipErrorInvalidValue;
    switch (row_tiles) {
        case 4: return launch_skinny_rt<4>(a, grid, s);
        case 5: return launch_skinny_rt<5>(a, grid, s);
        case 6: return launch_skinny_rt<6>(a, grid, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dk
