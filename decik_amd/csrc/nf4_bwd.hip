// Fused NF4 dequant x fp16 GEMM, input gradient (replaces dequantize_nf4 + matmul,
// solution/nf4.py:99-104, and the summed input gradients of solution/mlp.py:106-109):
//
//     dX[m, k] = sum_g sum_n dY_g[m, n] W_g[n, k]  (+ sum_g GU_g[m, t] A_g[t, k] for LoRA)
//
// The contraction runs over weight rows, so the weight must be read transposed: each step the
// work-group unpacks a 64 x 256 weight tile into LDS (row-major fp16), and every wave reads 8
// rows x 4 columns per lane (ds_read_b64) and transposes them into MFMA operands with
// v_perm_b32 (output columns interleaved by 4, so each lane ends with 16 consecutive outputs of
// one row). dY (BM x 64 fp16) is staged in LDS, double-buffered. Split-K over the contraction
// with a deterministic last-arriver reduction (gemm_common.h).
#include "gemm_common.h"

namespace dk {

template <int MT, bool NESTED>
__global__ __launch_bounds__(kGemmThreads, 1) void nf4_bwd_kernel(const BwdArgs a) {
    constexpr int BM = 16 * MT;
    constexpr int DBUF = BM * 128;   // bytes of one dY buffer (BM rows x 64 fp16)
    constexpr int WBUF = 64 * 512;   // bytes of one weight buffer (64 rows x 256 fp16)
    constexpr int DCH = BM * 8;      // 16-byte chunks per dY tile
    constexpr int DPT = (DCH + kGemmThreads - 1) / kGemmThreads;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* ds = smem;
    uint8_t* wt = smem + 2 * DBUF;
    float* lut = (float*)(wt + 2 * WBUF);    // [kMaxGroups][16]
    float* c2 = lut + 16 * kMaxGroups;        // [kMaxGroups][256]
    int* flag = (int*)(c2 + 256 * kMaxGroups);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, lg = lane >> 4;

    const int L = xcd_logical_id();
    if (L >= a.m_tiles * a.k_tiles * a.splits) return;
    const int m_tile = L % a.m_tiles;
    const int rest = L / a.m_tiles;
    const int k_tile = rest % a.k_tiles;
    const int split = rest / a.k_tiles;
    const int M = a.m, K = a.k;
    const int m0 = m_tile * BM;
    const int k0 = k_tile * kBwdBN;         // work-group's first output column
    const int kw0 = k0 + 64 * wave;         // wave's first output column
    const int cs0 = split * a.csteps_per_split;
    const int cs1 = min(a.csteps, cs0 + a.csteps_per_split);

    // each group's code books (groups may come from different QuantStates)
#pragma unroll
    for (int g = 0; g < kMaxGroups; ++g) {
        if (g >= a.ngroups) break;
        if (tid < 16) lut[16 * g + tid] = a.g[g].w.code[tid];
        if constexpr (NESTED) c2[256 * g + tid] = a.g[g].w.code2[tid];
    }

    u32x4_t dr[DPT];
    u32x4_t wraw[2];
    uint32_t wq[2];
    float wa[2];
    bool wok[2];
    float woff = 0.0f;
    int wgi = 0;  // group of the step held in the load registers

    auto load_step = [&](int s) {
        BwdGroupDev G = a.g[0];
        int gi = 0;
#pragma unroll
        for (int i = 1; i < kMaxGroups; ++i)
            if (i < a.ngroups && s >= a.g[i].step_begin) {
                G = a.g[i];
                gi = i;
            }
        wgi = gi;
        const int n0 = (s - G.step_begin) * kBwdBC;
        const int N = (int)G.w.n;
        const rsrc_t drs = make_rsrc(G.dy, G.dy_bytes);
#pragma unroll
        for (int i = 0; i < DPT; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c = q & 7;
            const int gm = m0 + row, gn = n0 + 8 * c;
            const uint32_t off = (q < DCH && gm < M && gn < N) ? (uint32_t)(gm * (int)G.lddy + gn) * 2u : kOOB;
            dr[i] = bload128(drs, off);
        }
        const rsrc_t wrs = make_rsrc(G.w.packed, G.w.packed_bytes);
        const rsrc_t ars = make_rsrc(NESTED ? (const void*)G.w.absmax8 : (const void*)G.w.absmaxf,
                                     G.w.absmax_bytes);
        const rsrc_t a2rs = make_rsrc(G.w.absmax2, G.w.absmax2_bytes);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c = q & 7;
            const int n = n0 + row, kk = k0 + 32 * c;
            wok[i] = n < N && kk < K;
            const uint32_t flat = (uint32_t)n * (uint32_t)K + (uint32_t)kk;
            const uint32_t blk = flat >> G.w.bs_shift;
            wraw[i] = bload128(wrs, wok[i] ? flat >> 1 : kOOB);
            if constexpr (NESTED) {
                wq[i] = bload8(ars, wok[i] ? blk : kOOB);
                wa[i] = bloadf(a2rs, wok[i] ? (blk >> G.w.bs2_shift) * 4u : kOOB);
            } else {
                wq[i] = 0;
                wa[i] = bloadf(ars, wok[i] ? blk * 4u : kOOB);
            }
        }
        woff = NESTED ? *G.w.offset : 0.0f;
    };
    auto store_step = [&](int buf) {
#pragma unroll
        for (int i = 0; i < DPT; ++i) {
            const int q = tid + kGemmThreads * i;
            if (q < DCH) {
                const int row = q >> 3, c = q & 7;
                *(u32x4_t*)(ds + buf * DBUF + row * 128 + ((c ^ ((row >> 1) & 7)) << 4)) = dr[i];
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c = q & 7;
            float s;
            if constexpr (NESTED) s = wok[i] ? c2[256 * wgi + wq[i]] * wa[i] + woff : 0.0f;
            else s = wa[i];
            uint32_t o[16];
            dequant16(wraw[i], s, lut + 16 * wgi, o);
            const int sw = ((row >> 4) & 1) << 3;
#pragma unroll
            for (int p = 0; p < 4; ++p)
                *(u32x4_t*)(wt + buf * WBUF + row * 512 + (((4 * c + p) ^ sw) << 4)) =
                    u32x4_t{o[4 * p], o[4 * p + 1], o[4 * p + 2], o[4 * p + 3]};
        }
    };

    float4_t acc_flat[MT * 4];
    float4_t (&acc)[MT][4] = *reinterpret_cast<float4_t(*)[MT][4]>(&acc_flat);
#pragma unroll
    for (int t = 0; t < MT * 4; ++t) acc_flat[t] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (cs0 < cs1) load_step(cs0);
    __syncthreads();  // code books
    if (cs0 < cs1) store_step(0);
    __syncthreads();

    for (int s = cs0; s < cs1; ++s) {
        const int buf = (s - cs0) & 1;
        const bool more = s + 1 < cs1;
        if (more) load_step(s + 1);
        const uint8_t* wb = wt + buf * WBUF;
        const uint8_t* db = ds + buf * DBUF;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            // 8 weight rows x 4 columns per lane -> A operands of 4 interleaved column blocks
            u32x2_t h[8];
            const int sw = (lg & 1) << 3;
            const int chunk = 8 * wave + (l16 >> 1);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int row = 16 * lg + 8 * jj + e;
                h[e] = *(const u32x2_t*)(wb + row * 512 + ((chunk ^ sw) << 4) + ((l16 & 1) << 3));
            }
            half8_t aop[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                uint32_t d[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t lo = h[2 * q][b >> 1], hi = h[2 * q + 1][b >> 1];
                    d[q] = (b & 1) ? perm_hi(lo, hi) : perm_lo(lo, hi);
                }
                aop[b] = __builtin_bit_cast(half8_t, u32x4_t{d[0], d[1], d[2], d[3]});
            }
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int row = 16 * i + l16;
                const half8_t bo =
                    *(const half8_t*)(db + row * 128 + (((2 * lg + jj) ^ ((l16 >> 1) & 7)) << 4));
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[i][b] = mfma16x16x32(aop[b], bo, acc[i][b]);
            }
        }
        if (more) store_step(buf ^ 1);
        __syncthreads();
    }

    if (a.splits > 1) {
        const int tile = k_tile * a.m_tiles + m_tile;
        if (!splitk_finish(acc_flat, a.partials, a.counters, tile, a.splits, split, flag, a.partial_bytes)) return;
    }

    // ---- epilogue: LoRA input-gradient terms GU_g . A_g, rounding, stores
    if (a.lora_rank > 0) {
        const int R = a.lora_rank;
#pragma unroll
        for (int g = 0; g < kMaxGroups; ++g) {
            if (g >= a.ngroups) break;
            const BwdGroupDev& G = a.g[g];
            if (G.lora_gu == nullptr) continue;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int kc = kw0 + 4 * l16 + b;
                for (int t0 = 0; t0 < R; t0 += 16) {
                    half4_t av;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        av[e] = kc < K ? G.lora_a[(int64_t)(t0 + 4 * lg + e) * K + kc] : (_Float16)0;
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        const int m = m0 + 16 * i + l16;
                        const half4_t gv = m < M ? *(const half4_t*)(G.lora_gu + (int64_t)m * R + t0 + 4 * lg)
                                                 : half4_t{0, 0, 0, 0};
                        acc[i][b] = mfma16x16x16(av, gv, acc[i][b]);
                    }
                }
            }
        }
    }
    const int kb = kw0 + 16 * lg;  // this lane's 16 consecutive output columns: t = 4 r + b
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = m0 + 16 * i + l16;
        if (m >= M) continue;
        float v[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) v[t] = acc[i][t & 3][t >> 2];
        if (a.dx_fp32) {
            float* row = (float*)a.dx + (int64_t)m * a.lddx + kb;
            if (kb + 16 <= K) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(float4_t*)(row + 4 * q) = float4_t{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            } else {
                for (int t = 0; t < 16 && kb + t < K; ++t) row[t] = v[t];
            }
        } else {
            _Float16* row = (_Float16*)a.dx + (int64_t)m * a.lddx + kb;
            uint32_t o[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t] = pack_half2(v[2 * t], v[2 * t + 1]);
            if (kb + 16 <= K) {
                *(u32x4_t*)(row) = u32x4_t{o[0], o[1], o[2], o[3]};
                *(u32x4_t*)(row + 8) = u32x4_t{o[4], o[5], o[6], o[7]};
            } else {
                for (int t = 0; t < 16 && kb + t < K; ++t) row[t] = (_Float16)v[t];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// launch

template <int MT>
static size_t bwd_smem() { return 2 * (16 * MT) * 128 + 2 * 64 * 512 + (16 + 256) * 4 * kMaxGroups + 16; }

template <int MT, bool NESTED>
static hipError_t launch_bwd_t(const BwdArgs& a, int grid, hipStream_t s) {
    static bool attr = false;
    const size_t sm = bwd_smem<MT>();
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)nf4_bwd_kernel<MT, NESTED>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((nf4_bwd_kernel<MT, NESTED>), dim3(grid), dim3(kGemmThreads), sm, s, a);
    return hipGetLastError();
}


hipError_t launch_bwd(const BwdArgs& a, int mt, int grid, hipStream_t s) {
#define X(T) \
    if (mt == T) return a.nested ? launch_bwd_t<T, true>(a, grid, s) : launch_bwd_t<T, false>(a, grid, s);
    X(1) X(2) X(4) X(8) X(13)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
