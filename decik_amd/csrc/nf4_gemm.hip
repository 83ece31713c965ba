// Fused NF4 dequant x fp16 GEMM on gfx950 MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation).
//
// Forward  (replaces dequantize_nf4 + F.linear, solution/nf4.py:93-96):
//     Y[m, n] = sum_k X[m, k] W[n, k] + bias[n] + s * sum_t U[m, t] B[n, t]
//   The dequantized weight is the MFMA A operand (rows n), X the B operand (columns m), so
//   D = W.X^T = Y^T. Each wave owns 64 weight rows for the whole tile: it loads their packed
//   bytes straight from HBM (16 bytes = 32 consecutive k per lane), unpacks them in registers
//   and feeds them to the MFMA; no fp16 weight is written anywhere. The X tile (BM x 128 fp16)
//   is staged in LDS, double-buffered, and shared by the 4 waves.
//
// Backward (replaces dequantize_nf4 + matmul, solution/nf4.py:99-104, and the summed input
//   gradients of solution/mlp.py:106-109): dX[m, k] = sum_g sum_n dY_g[m, n] W_g[n, k].
//   The contraction runs over weight rows, so the weight must be read transposed: each step the
//   work-group unpacks a 64 x 256 weight tile into LDS (row-major fp16), and every wave reads 8
//   rows x 4 columns per lane (ds_read_b64) and transposes them into MFMA operands with
//   v_perm_b32. dY (BM x 64 fp16) is staged in LDS like X in the forward.
//
// Permutation freedom: an MFMA sums over its 32 contraction slots in any order, so lanes take
// contraction indices that make their global loads contiguous; A and B always use the same
// mapping. Output columns are interleaved so that each lane ends up owning 16 consecutive
// outputs of one row, stored with two 16-byte stores.
//
// Split-K: when the output has too few tiles to fill the GPU, the contraction is split; each
// work-group writes its fp32 partial tile, and the last one to finish (an atomic counter per
// tile) adds all partials in split order (deterministic), runs the epilogue and resets the
// counter to 0.
#include "dk_internal.h"

namespace dk {

namespace {

__device__ __forceinline__ int xcd_logical_id() {
    // The dispatcher deals work-groups to the 8 XCDs round-robin. Renumber them so that logical
    // ids that are consecutive run on one XCD (and share its L2). gridDim.x is a multiple of 8.
    const int nwg = gridDim.x, bid = blockIdx.x;
    return (bid & 7) * (nwg >> 3) + (bid >> 3);
}

__device__ __forceinline__ uint32_t perm_lo(uint32_t lo_src, uint32_t hi_src) {
    // low 16 bits of lo_src, then low 16 bits of hi_src
    return __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
}

__device__ __forceinline__ uint32_t perm_hi(uint32_t lo_src, uint32_t hi_src) {
    // high 16 bits of lo_src, then high 16 bits of hi_src
    return __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
}

template <int MT>
__device__ __forceinline__ bool splitk_finish(float4_t (&acc)[MT][4], float* partials,
                                              int32_t* counters, int tile, int splits,
                                              int split, int* flag) {
    const int tid = threadIdx.x;
    float* base = partials + (int64_t)tile * splits * (MT * 4 * kGemmThreads * 4);
    float* mine = base + (int64_t)split * (MT * 4 * kGemmThreads * 4);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *(float4_t*)(mine + ((i * 4 + j) * kGemmThreads + tid) * 4) = acc[i][j];
    __threadfence();
    __syncthreads();
    if (tid == 0) *flag = (atomicAdd(counters + tile, 1) == splits - 1);
    __syncthreads();
    if (!*flag) return false;
    __threadfence();
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float4_t sum = {0.f, 0.f, 0.f, 0.f};
            for (int s = 0; s < splits; ++s) {
                const float4_t v = s == split
                    ? acc[i][j]
                    : __builtin_nontemporal_load(
                          (const float4_t*)(base + (int64_t)s * (MT * 4 * kGemmThreads * 4) +
                                            ((i * 4 + j) * kGemmThreads + tid) * 4));
                sum += v;
            }
            acc[i][j] = sum;
        }
    if (tid == 0) counters[tile] = 0;
    return true;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// forward

template <int MT, bool NESTED>
__global__ __launch_bounds__(kGemmThreads, 1) void nf4_fwd_kernel(const FwdArgs a) {
    constexpr int BM = 16 * MT;
    constexpr int XBUF = BM * 256;  // bytes of one X buffer (BM rows x 128 fp16)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* xs = smem;
    float* lut = (float*)(smem + 2 * XBUF);
    float* c2 = lut + 16;
    int* flag = (int*)(c2 + 256);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, lg = lane >> 4;

    const int L = xcd_logical_id();
    if (L >= a.m_tiles * a.n_tiles * a.splits) return;
    const int m_tile = L % a.m_tiles;
    const int rest = L / a.m_tiles;
    const int n_tile = rest % a.n_tiles;
    const int split = rest / a.n_tiles;

    FwdGroupDev G = a.g[0];
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && n_tile >= a.g[i].tile_begin) G = a.g[i];
    const NF4Dev& W = G.w;
    const int M = a.m, K = a.k;
    const int64_t N = W.n;
    const int m0 = m_tile * BM;
    const int64_t nw0 = (int64_t)(n_tile - G.tile_begin) * kFwdBN + wave * 64;
    const int ks0 = split * a.ksteps_per_split;
    const int ks1 = min(a.ksteps, ks0 + a.ksteps_per_split);

    if (tid < 16) lut[tid] = W.code[tid];
    if constexpr (NESTED) c2[tid] = W.code2[tid];
    const float offset = NESTED ? *W.offset : 0.0f;

    // ---- per-step loaders
    u32x4_t xr[MT];
    u32x4_t wraw[4];
    uint32_t wq[4];
    float wa[4];
    bool wok[4];

    auto load_x = [&](int ks) {
        const int k0 = ks * kFwdBK;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 4, c = q & 15;
            const int gm = m0 + row, gk = k0 + 8 * c;
            xr[i] = (gm < M && gk < K) ? *(const u32x4_t*)(a.x + (int64_t)gm * a.ldx + gk)
                                       : u32x4_t{0u, 0u, 0u, 0u};
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 4, c = q & 15;
            *(u32x4_t*)(xs + buf * XBUF + row * 256 + ((c ^ (row & 15)) << 4)) = xr[i];
        }
    };
    auto load_w = [&](int ks) {
        const int krun = ks * kFwdBK + 32 * lg;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t row = nw0 + 4 * l16 + j;
            wok[j] = row < N && krun < K;
            if (wok[j]) {
                const int64_t flat = row * K + krun;
                wraw[j] = *(const u32x4_t*)(W.packed + (flat >> 1));
                const int64_t blk = block_of(W, flat);
                if constexpr (NESTED) {
                    wq[j] = W.absmax8[blk];
                    wa[j] = W.absmax2[group_of(W, blk)];
                } else {
                    wq[j] = 0;
                    wa[j] = W.absmaxf[blk];
                }
            } else {
                wraw[j] = u32x4_t{0u, 0u, 0u, 0u};
                wq[j] = 0;
                wa[j] = 0.0f;
            }
        }
    };

    float4_t acc[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (ks0 < ks1) {
        load_x(ks0);
        load_w(ks0);
    }
    __syncthreads();  // code books in LDS
    if (ks0 < ks1) store_x(0);
    __syncthreads();

    for (int ks = ks0; ks < ks1; ++ks) {
        const int buf = (ks - ks0) & 1;
        // unpack this step's weights into MFMA A operands
        half8_t wop[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float s;
            if constexpr (NESTED) s = wok[j] ? c2[wq[j]] * wa[j] + offset : 0.0f;
            else s = wa[j];
            uint32_t o[16];
            dequant16(wraw[j], s, lut, o);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                wop[j][jj] = __builtin_bit_cast(
                    half8_t, u32x4_t{o[4 * jj], o[4 * jj + 1], o[4 * jj + 2], o[4 * jj + 3]});
        }
        const bool more = ks + 1 < ks1;
        if (more) {
            load_x(ks + 1);
            load_w(ks + 1);
        }
        const uint8_t* xb = xs + buf * XBUF;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            half8_t xo[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                xo[jj] = *(const half8_t*)(xb + (16 * i + l16) * 256 + (((4 * lg + jj) ^ l16) << 4));
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) acc[i][j] = mfma16x16x32(wop[j][jj], xo[jj], acc[i][j]);
        }
        if (more) store_x(buf ^ 1);
        __syncthreads();
    }

    if (a.splits > 1) {
        const int tile = n_tile * a.m_tiles + m_tile;
        if (!splitk_finish<MT>(acc, a.partials, a.counters, tile, a.splits, split, flag)) return;
    }

    // ---- epilogue: LoRA term, bias, fp16 rounding, stores
    if (G.lora_u != nullptr) {
        const int R = a.lora_rank;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t row = nw0 + 4 * l16 + j;
            for (int t0 = 0; t0 < R; t0 += 16) {
                const half4_t bl = row < N ? *(const half4_t*)(G.lora_b + row * R + t0 + 4 * lg)
                                           : half4_t{0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const int m = m0 + 16 * i + l16;
                    const half4_t uu = m < M ? *(const half4_t*)(G.lora_u + (int64_t)m * R + t0 + 4 * lg)
                                             : half4_t{0, 0, 0, 0};
                    const float4_t t = mfma16x16x16(bl, uu, float4_t{0.f, 0.f, 0.f, 0.f});
                    acc[i][j] += G.lora_scale * t;
                }
            }
        }
    }
    const int64_t nb = nw0 + 16 * lg;  // this lane's 16 consecutive output columns
    float bias[16];
#pragma unroll
    for (int t = 0; t < 16; ++t)
        bias[t] = (G.bias != nullptr && nb + t < N) ? (float)G.bias[nb + t] : 0.0f;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = m0 + 16 * i + l16;
        if (m >= M) continue;
        uint32_t o[8];
#pragma unroll
        for (int t = 0; t < 16; t += 2) {
            // column t = 4 r + j  ->  acc[i][j][r]
            const float v0 = acc[i][t & 3][t >> 2] + bias[t];
            const float v1 = acc[i][(t + 1) & 3][(t + 1) >> 2] + bias[t + 1];
            o[t >> 1] = pack_half2(v0, v1);
        }
        _Float16* yrow = G.y + (int64_t)m * G.ldy + nb;
        if (nb + 16 <= N) {
            *(u32x4_t*)(yrow) = u32x4_t{o[0], o[1], o[2], o[3]};
            *(u32x4_t*)(yrow + 8) = u32x4_t{o[4], o[5], o[6], o[7]};
        } else {
            for (int t = 0; t < 16 && nb + t < N; ++t)
                yrow[t] = __builtin_bit_cast(_Float16, (uint16_t)((o[t >> 1] >> (16 * (t & 1))) & 0xFFFFu));
        }
    }
}

// ------------------------------------------------------------------------------------------
// backward (input gradient)

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
        const int64_t n0 = (int64_t)(s - G.step_begin) * kBwdBC;
        const int64_t N = G.w.n;
#pragma unroll
        for (int i = 0; i < DPT; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c = q & 7;
            const int gm = m0 + row;
            const int64_t gn = n0 + 8 * c;
            dr[i] = (q < DCH && gm < M && gn < N)
                        ? *(const u32x4_t*)(G.dy + (int64_t)gm * G.lddy + gn)
                        : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c = q & 7;
            const int64_t n = n0 + row;
            const int kk = k0 + 32 * c;
            wok[i] = n < N && kk < K;
            if (wok[i]) {
                const int64_t flat = n * K + kk;
                wraw[i] = *(const u32x4_t*)(G.w.packed + (flat >> 1));
                const int64_t blk = block_of(G.w, flat);
                if constexpr (NESTED) {
                    wq[i] = G.w.absmax8[blk];
                    wa[i] = G.w.absmax2[group_of(G.w, blk)];
                } else {
                    wq[i] = 0;
                    wa[i] = G.w.absmaxf[blk];
                }
            } else {
                wraw[i] = u32x4_t{0u, 0u, 0u, 0u};
                wq[i] = 0;
                wa[i] = 0.0f;
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

    float4_t acc[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

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
        if (!splitk_finish<MT>(acc, a.partials, a.counters, tile, a.splits, split, flag)) return;
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
static size_t fwd_smem() { return 2 * (16 * MT) * 256 + (16 + 256) * 4 + 16; }
template <int MT>
static size_t bwd_smem() { return 2 * (16 * MT) * 128 + 2 * 64 * 512 + (16 + 256) * 4 * kMaxGroups + 16; }

template <int MT, bool NESTED>
static hipError_t launch_fwd_t(const FwdArgs& a, int grid, hipStream_t s) {
    static bool attr = false;
    const size_t sm = fwd_smem<MT>();
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)nf4_fwd_kernel<MT, NESTED>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((nf4_fwd_kernel<MT, NESTED>), dim3(grid), dim3(kGemmThreads), sm, s, a);
    return hipGetLastError();
}

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

#define DK_MT_CASES(X) X(1) X(2) X(4) X(8) X(13)

hipError_t launch_fwd(const FwdArgs& a, int mt, int grid, hipStream_t s) {
#define X(T) \
    if (mt == T) return a.nested ? launch_fwd_t<T, true>(a, grid, s) : launch_fwd_t<T, false>(a, grid, s);
    DK_MT_CASES(X)
#undef X
    return hipErrorInvalidValue;
}

hipError_t launch_bwd(const BwdArgs& a, int mt, int grid, hipStream_t s) {
#define X(T) \
    if (mt == T) return a.nested ? launch_bwd_t<T, true>(a, grid, s) : launch_bwd_t<T, false>(a, grid, s);
    DK_MT_CASES(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
