// Fused NF4 dequant x fp16 GEMM, forward (replaces dequantize_nf4 + F.linear,
// solution/nf4.py:93-96; the LoRA term of solution/attn.py:225-228 rides in the epilogue):
//
//     Y[m, n] = sum_k X[m, k] W[n, k] + bias[n] + sum_t U[m, t] fp16(s * B[n, t])
//
// MFMA v_mfma_f32_32x32x16_f16 with fp32 accumulation. The dequantized weight is the A operand
// (32 weight rows per block), X the B operand (32 token rows per block), so D = W.X^T = Y^T.
// Work-group = 4 waves; tile = 32*MB token rows x 256 weight rows, 64 weight rows per wave.
// Each wave loads its own weight rows' packed bytes (16 bytes = 32 consecutive k per lane and
// step), unpacks them in registers and feeds them to the MFMA: no fp16 weight is ever written.
// The X tile (32*MB rows x 64 k, fp16) is staged in LDS, double-buffered, shared by the waves.
//
// Software pipeline (one wave per SIMD, so the wave itself must overlap its latencies): while
// the MFMAs of step s run, the wave unpacks step s+1's weights (VALU + code-book lookups in
// LDS) in slices between the MFMAs and reads the next token block's X fragments one block
// ahead. Global loads run ahead of use and go straight into LDS rings (buffer_load ... lds):
// X tiles and, per wave, the packed weights with their block statistics; each step ends with
// one explicit wait on them and a barrier.
//
// Contraction order: an MFMA sums its 16 contraction slots in any order, so lane group g takes
// k = 32 g + 8 jj + e (jj = MFMA index within the 64-wide step): its 32 weights are one
// contiguous 16-byte load. A rows follow arow_to_n, so each lane ends with 16 consecutive
// output columns of one token row (two 16-byte stores).
#include "gemm_common.h"

namespace dk {

constexpr int kFwdSmemHeader = 2048;  // code books + split-K flag; X buffers follow
constexpr int kFwdWSlot = 3072;       // per wave and step: 2 KB packed, 2 x 256 B codes, 2 x 256 B absmax2

// Per token block and wave: 8 MFMAs, 4 X fragment reads and 1/MB of the step's unpacking
// (64 code-book lookups, ~260 VALU).
template <int MB>
constexpr int kFwdDsPerMfma = (4 + 64 / MB + 7) / 8;
template <int MB>
constexpr int kFwdValuPerMfma = (270 / MB + 7) / 8;

template <int MB, bool NESTED>
__global__ __launch_bounds__(kGemmThreads, 1) void nf4_fwd_kernel(const FwdArgs a) {
    constexpr int BM = 32 * MB;
    constexpr int XBUF = BM * 128;  // bytes of one X buffer
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* lut = (float*)smem;  // at LDS address 0: the lookup address is nibble * 4
    float* c2 = lut + 16;
    int* flag = (int*)(c2 + 256);
    uint8_t* xs = smem + kFwdSmemHeader;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;

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
    const int M = a.m, K = a.k, N = (int)W.n;
    const int m0 = m_tile * BM;
    const int nw0 = (n_tile - G.tile_begin) * kFwdBN + wave * 64;
    const int ks0 = split * a.ksteps_per_split;
    const int ks1 = min(a.ksteps, ks0 + a.ksteps_per_split);

    if (tid < 16) lut[tid] = W.code[tid];
    if constexpr (NESTED) c2[tid] = W.code2[tid];
    const float offset = NESTED ? *W.offset : 0.0f;

    const rsrc_t xrs = make_rsrc(a.x, a.x_bytes);
    const rsrc_t wrs = make_rsrc(W.packed, W.packed_bytes);
    const rsrc_t ars = make_rsrc(NESTED ? (const void*)W.absmax8 : (const void*)W.absmaxf, W.absmax_bytes);
    const rsrc_t a2rs = make_rsrc(W.absmax2, W.absmax2_bytes);
    const int wrow0 = nw0 + arow_to_n(l32);  // this lane's A row in block 0 (block 1: +32)
    const int xsw = (l32 >> 1) & 7;           // LDS swizzle of this lane's X rows

    // ---- loaders: every global load goes straight into LDS (buffer_load ... lds), two steps
    // ahead, so the only waits on global memory are the explicit one per step below.
    //   X tiles: ring of 3 buffers shared by the work-group.
    //   Weights: per-wave ring of 3 slots holding each lane's 2 x 16 packed bytes, its 2 absmax
    //   codes and 2 absmax2 values (plain weights: 2 fp32 absmax); read back by the same lane.
    uint8_t* wring = xs + 3 * XBUF + wave * (3 * kFwdWSlot);
    auto xbuf = [&](int t) -> uint8_t* { return xs + ((t - ks0) % 3) * XBUF; };
    auto wslot = [&](int t) -> uint8_t* { return wring + ((t - ks0) % 3) * kFwdWSlot; };
    auto load_x = [&](int t) {  // X tile of step t
        const int k0 = t * kFwdBK;
        uint8_t* dst = xbuf(t);
#pragma unroll
        for (int h = 0; h < MB; ++h) {
            // wave-contiguous LDS destination: chunk q lands at q * 16 = row * 128 + pc * 16
            const int q = tid + kGemmThreads * h;
            const int row = q >> 3, pc = q & 7;
            const int c = pc ^ ((row >> 1) & 7);  // the logical k chunk stored at this position
            const int gm = m0 + row, gk = k0 + 8 * c;
            bload128_lds(xrs, dst + (kGemmThreads * h + 64 * wave) * 16,
                         (gm < M && gk < K) ? (uint32_t)(gm * (int)a.ldx + gk) * 2u : kOOB);
        }
    };
    auto load_w = [&](int t) {  // this lane's packed weights and statistics of step t
        const int krun = t * kFwdBK + 32 * g;
        uint8_t* slot = wslot(t);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int row = wrow0 + 32 * b;
            const bool ok = row < N && krun < K;
            const uint32_t flat = (uint32_t)row * (uint32_t)K + (uint32_t)krun;
            const uint32_t blk = flat >> W.bs_shift;
            bload128_lds(wrs, slot + b * 1024, ok ? flat >> 1 : kOOB);
            if constexpr (NESTED) {
                bload8_lds(ars, slot + 2048 + b * 256, ok ? blk : kOOB);
                bload32_lds(a2rs, slot + 2560 + b * 256, ok ? (blk >> W.bs2_shift) * 4u : kOOB);
            } else {
                bload32_lds(ars, slot + 2560 + b * 256, ok ? blk * 4u : kOOB);
            }
        }
    };
    const bool rowok0 = wrow0 < N, rowok1 = wrow0 + 32 < N;
    // fp32 scale of block b for step t (0 past the end of the weight)
    auto scale_of = [&](int t, int b) -> float {
        const uint8_t* slot = wslot(t);
        const float a2 = *(const float*)(slot + 2560 + b * 256 + 4 * lane);
        const bool ok = (b ? rowok1 : rowok0) && t * kFwdBK + 32 * g < K;
        if constexpr (NESTED) {
            const uint32_t q = slot[2048 + b * 256 + 4 * lane];
            const float sc = c2[q] * a2 + offset;
            return ok ? sc : 0.0f;
        } else {
            return a2;  // past the end the load wrote 0
        }
    };
    auto wpacked = [&](int t, int b) -> u32x4_t {
        return *(const u32x4_t*)(wslot(t) + b * 1024 + 16 * lane);
    };
    auto xfrag = [&](const uint8_t* xb, int i, int jj) -> half8_t {
        return *(const half8_t*)(xb + (32 * i + l32) * 128 + (((4 * g + jj) ^ xsw) << 4));
    };

    float16_t acc[MB * 2];  // [token block i][weight block b] at i * 2 + b
#pragma unroll
    for (int t = 0; t < MB * 2; ++t) acc[t] = float16_t{};

    half8_t wop[2][4];  // A operands of the current step
    // Issue order matters for the waits: weights first, then X, for every step.
    load_w(ks0);
    load_x(ks0);
    load_w(ks0 + 1);
    load_x(ks0 + 1);
    constexpr int WL = NESTED ? 6 : 4;  // global loads per step for the weights (per lane)
    wait_vmcnt<MB + WL>();  // X(ks0) and W(ks0) have landed
    lds_barrier();         // ... for every wave; code books in LDS
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        uint32_t o[16];
        dequant16(wpacked(ks0, b), scale_of(ks0, b), lut, o);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
            wop[b][jj] = __builtin_bit_cast(half8_t, u32x4_t{o[4 * jj], o[4 * jj + 1], o[4 * jj + 2], o[4 * jj + 3]});
    }
    load_w(ks0 + 2);
    load_x(ks0 + 2);
    wait_vmcnt<MB + WL>();  // X(ks0 + 1), W(ks0 + 1) have landed
    lds_barrier();

    // One step: MFMAs on X(t) and the current operands; in slices between them, step t+1's
    // weights are unpacked. The body is one basic block, so the scheduler can interleave it;
    // loads past k read zeros and are never used.
    for (int t = ks0; t < ks1; ++t) {
        const uint8_t* xb = xbuf(t);
        const u32x4_t p0 = wpacked(t + 1, 0), p1 = wpacked(t + 1, 1);
        const float sn0 = scale_of(t + 1, 0), sn1 = scale_of(t + 1, 1);
        uint32_t on[2][16];
        half8_t xf[2][4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) xf[0][jj] = xfrag(xb, 0, jj);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            if (i + 1 < MB) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) xf[(i + 1) & 1][jj] = xfrag(xb, i + 1, jj);
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
                for (int b = 0; b < 2; ++b) acc[i * 2 + b] = mfma32x32x16(wop[b][jj], xf[i & 1][jj], acc[i * 2 + b]);
#pragma unroll
                for (int ch = 0; ch < 8; ++ch) {
                    if ((ch * MB * 4) / 8 == i * 4 + jj)
                        dequant4((ch >> 2 ? p1 : p0)[ch & 3], (ch >> 2) ? sn1 : sn0, lut,
                                 &on[ch >> 2][4 * (ch & 3)]);
                }
            }
            // Issue order within the token block: each MFMA followed by LDS reads (code-book
            // lookups, the next block's X fragments) and unpacking VALU work; nothing moves
            // across blocks, which bounds the live registers.
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                      // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, kFwdDsPerMfma<MB>, 0);    // LDS read
                __builtin_amdgcn_sched_group_barrier(0x002, kFwdValuPerMfma<MB>, 0);  // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                wop[b][jj] = __builtin_bit_cast(
                    half8_t, u32x4_t{on[b][4 * jj], on[b][4 * jj + 1], on[b][4 * jj + 2], on[b][4 * jj + 3]});
        lds_barrier();  // every wave is done with X(t) and W(t+1): their buffers are reused next
        load_w(t + 3);
        load_x(t + 3);
        // X(t+1) and W(t+2) have landed: only X(t+2), W(t+3), X(t+3) may still be in flight
        wait_vmcnt<2 * MB + WL>();
        lds_barrier();
    }
    wait_vmcnt<0>();

    if (a.splits > 1) {
        const int tile = n_tile * a.m_tiles + m_tile;
        if (!splitk_finish(acc, a.partials, a.counters, tile, a.splits, split, flag, a.partial_bytes)) return;
    }

    // ---- epilogue: LoRA term, bias, one fp16 rounding, stores
    if (G.lora_u != nullptr) {
        // s * U.B^T accumulates straight into the MFMA accumulators; the scale is folded into
        // the B operand (exact for power-of-two scales such as alpha / r = 2).
        const int R = a.lora_rank;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int row = wrow0 + 32 * b;
            for (int t0 = 0; t0 < R; t0 += 16) {
                half8_t bl = row < N ? *(const half8_t*)(G.lora_b + (int64_t)row * R + t0 + 8 * g)
                                     : half8_t{};
#pragma unroll
                for (int e = 0; e < 8; ++e) bl[e] = (_Float16)((float)bl[e] * G.lora_scale);
#pragma unroll
                for (int i = 0; i < MB; ++i) {
                    const int m = m0 + 32 * i + l32;
                    const half8_t uu = m < M ? *(const half8_t*)(G.lora_u + (int64_t)m * R + t0 + 8 * g)
                                             : half8_t{};
                    acc[i * 2 + b] = mfma32x32x16(bl, uu, acc[i * 2 + b]);
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int nb = nw0 + 32 * b + 16 * g;  // this lane's 16 consecutive output columns
        float bias[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) bias[r] = (G.bias != nullptr && nb + r < N) ? (float)G.bias[nb + r] : 0.0f;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int m = m0 + 32 * i + l32;
            if (m >= M) continue;
            uint32_t o[8];
#pragma unroll
            for (int r = 0; r < 16; r += 2) o[r >> 1] = pack_half2(acc[i * 2 + b][r] + bias[r], acc[i * 2 + b][r + 1] + bias[r + 1]);
            _Float16* yrow = G.y + (int64_t)m * G.ldy + nb;
            if (nb + 16 <= N) {
                *(u32x4_t*)(yrow) = u32x4_t{o[0], o[1], o[2], o[3]};
                *(u32x4_t*)(yrow + 8) = u32x4_t{o[4], o[5], o[6], o[7]};
            } else {
                for (int r = 0; r < 16 && nb + r < N; ++r)
                    yrow[r] = __builtin_bit_cast(_Float16, (uint16_t)((o[r >> 1] >> (16 * (r & 1))) & 0xFFFFu));
            }
        }
    }
}

template <int MB>
static size_t fwd_smem() { return kFwdSmemHeader + 3 * (32 * MB) * 128 + 4 * 3 * kFwdWSlot; }

template <int MB, bool NESTED>
static hipError_t launch_fwd_t(const FwdArgs& a, int grid, hipStream_t s) {
    static bool attr = false;
    const size_t sm = fwd_smem<MB>();
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)nf4_fwd_kernel<MB, NESTED>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((nf4_fwd_kernel<MB, NESTED>), dim3(grid), dim3(kGemmThreads), sm, s, a);
    return hipGetLastError();
}

hipError_t launch_fwd(const FwdArgs& a, int mb, int grid, hipStream_t s) {
#define X(T) \
    if (mb == T) return a.nested ? launch_fwd_t<T, true>(a, grid, s) : launch_fwd_t<T, false>(a, grid, s);
    X(1) X(2) X(4) X(7)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
