// Fused NF4 dequant x fp16 product for launches with one to eight token rows: the same
// Y = X.W^T + bias as nf4_fwd_kernel (solution/nf4.py:93-96) in the decoding regime, where the
// call is bound by streaming the packed weight from HBM once. The MFMA kernels pad such launches
// to 32-token tiles and dequantize every weight for one useful multiply-add; here each weight is
// dequantized once and used for every token in fp32 dot products (v_dot2_f32_f16).
//
// The kernel is organised around keeping as much of the weight in flight as HBM needs:
// - Token rows: a work-group computes one, two or four (MT); launches of five to eight rows take
//   two work-groups per row range, one per four token rows, so that X stays four rows of LDS.
// - A work-group (four waves; eight where X of long rows would limit a CU to 12 waves) owns
//   `rows` consecutive weight rows of one group. Their packed bytes are contiguous ([n, k / 2]
//   row-major), so the work-group streams one contiguous range of 16-byte chunks (32 weights of
//   one block each: blocks are powers of two >= 32 and k % 32 == 0): thread t of T takes chunks
//   t, t + T, ..., so every load instruction reads 4 KB contiguous, and all of a thread's chunk
//   loads (and their block scales) are issued before any is used -- the whole weight of a 7B
//   projection is in flight at once.
// - X (m x k fp16) is copied to LDS by the work-group while the weight loads are in flight, in
//   a transposed order: 16-byte piece e of the 64-byte k-range p of a chunk goes to slot
//   e * (k / 32) + p, so the lanes of a wave (consecutive chunks, consecutive p) read
//   consecutive 16-byte slots -- no LDS bank conflicts -- where the natural order would put 64
//   bytes between neighbouring lanes.
// - Each chunk's dot products (fp32) go to an LDS slot; 16 lanes of a wave then sum each row's
//   slots in a fixed order (lane j: slots j, j + 16, ...; then four DPP steps across the 16), add
//   the bias, round once to fp16 and store. The summation order depends only on k: every call
//   gives the same bits.
// - Dequantization as in the other kernels: byte-pair code book in LDS (one 8-byte read per
//   packed byte), fp32 multiply by the block scale, one fp16 rounding: the reference's bits.
#include "dk_internal.h"

namespace dk {

constexpr int kGemvThreads = 256;  // four waves
constexpr int kGemvMaxChunks = 8;  // chunks (16-byte loads) per thread
constexpr size_t kGemvWideLds = 40 * 1024;  // LDS per work-group past which it takes eight waves

// LDS bytes of a launch: code book, X of the token rows, the chunk partial sums
static size_t gemv_smem_bytes(int mt, int k, int chunks) {
    // dynamic part: nested code2 table (256 floats), X, sums (the code book is static)
    return 256 * sizeof(float) + (size_t)mt * k * 2 + (size_t)mt * chunks * sizeof(float);
}

// x plus the x of the lane that DPP control CTRL names (all rows and banks, no bound control)
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false);
    return x + __builtin_bit_cast(float, o);
}

// The sum of v over the 16 lanes of a DPP row: every lane of the row receives a sum of all 16,
// each in a fixed order (pairs, then quads, then across quads).
__device__ __forceinline__ float row16_sum(float v) {
    v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v = dpp_add<0x124>(v);  // row_ror:4
    return dpp_add<0x128>(v);  // row_ror:8
}

template <int MT, bool NESTED, int CPT, int TH>
__global__ __launch_bounds__(TH) void nf4_gemv_kernel(const FwdArgs a, const int rows_per_wg, const uint32_t cpr_inv,
                                                       const int tg_shift) {
    // byte-pair code book (static: its address is a constant the LDS reads take as an offset)
    __shared__ float2_t lut2[256];
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* c2 = (float*)smem;                        // nested: code2 table
    _Float16* xs = (_Float16*)(smem + 256 * 4);      // [MT][k], transposed 16-byte pieces
    // token groups: with tg_shift = 1, work-groups 2 b and 2 b + 1 take the same weight rows for
    // token rows 0..MT-1 and MT..2 MT-1 (X of MT rows per work-group)
    const int tg = (int)blockIdx.x & ((1 << tg_shift) - 1);
    const int bid = (int)blockIdx.x >> tg_shift;
    const int K = a.k, M = min(MT, a.m - MT * tg);
    const _Float16* const xg = a.x + (int64_t)(MT * tg) * a.ldx;
    float* part = (float*)(xs + MT * K);             // [MT][rows * cpr]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
    int gi = 0;
#pragma unroll
    for (int q = 1; q < kMaxGroups; ++q)
        if (q < a.ngroups && bid >= a.g[q].tile_begin) gi = q;
    const FwdGroupDev& G = a.g[gi];
    const NF4Dev& W = G.w;
    const int N = (int)W.n;
    const int n0 = (bid - G.tile_begin) * rows_per_wg;
    const int rows = min(rows_per_wg, N - n0);
    const int cpr = K >> 5;                 // chunks per row
    const int nch = rows * cpr;             // chunks of this work-group
    const uint32_t c0 = (uint32_t)n0 * (uint32_t)cpr;  // first chunk (flat over the weight)

    // Load order: the thread's chunk loads and block statistics first, so that the HBM round trip
    // starts before anything else; then its code-book entries and X of every token row, straight
    // into LDS (no registers), which arrive while the chunks are in flight. Vector memory
    // operations complete in order: one wait for all of them precedes the code book's LDS writes.
    const rsrc_t wrs = make_rsrc(W.packed, W.packed_bytes);
    const rsrc_t ars = make_rsrc(NESTED ? (const void*)W.absmax8 : (const void*)W.absmaxf, W.absmax_bytes);
    const rsrc_t a2rs = make_rsrc(W.absmax2, NESTED ? W.absmax2_bytes : 0u);
    const uint32_t bs_shift = W.bs_shift, bs2_shift = W.bs2_shift;
    u32x4_t p[CPT];
    float s[CPT];
    uint32_t q8[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + TH * i;
        const bool ok = c < nch;
        const uint32_t ch = c0 + (uint32_t)c;
        p[i] = bload128(wrs, off_if(ok, ch * 16u));
        const uint32_t blk = (ch * 32u) >> bs_shift;
        if constexpr (NESTED) {
            q8[i] = bload8(ars, off_if(ok, blk));
            s[i] = bloadf(a2rs, off_if(ok, (blk >> bs2_shift) * 4u));
        } else {
            s[i] = bloadf(ars, off_if(ok, blk * 4u));
        }
    }
    asm volatile("" ::: "memory");  // the chunk loads go out first
    const float b_hi = W.code[(tid & 255) >> 4], b_lo = W.code[tid & 15];
    const float c2v = NESTED ? W.code2[tid & 255] : 0.0f;
    const float offset = NESTED ? *W.offset : 0.0f;
    {
        // slot e * cpr + p of a token row holds its 16-byte piece e of k-range p (source bytes
        // 16 (4 p + e)): each load instruction of a wave fills 64 consecutive slots of one piece
        const uint32_t xbytes = (uint32_t)K * 2u;
        for (int m = 0; m < MT; ++m) {
            const rsrc_t xr = make_rsrc(xg + (int64_t)min(m, M - 1) * a.ldx, m < M ? xbytes : 0u);
            uint8_t* xm = (uint8_t*)xs + (size_t)m * xbytes;
            for (int p0 = 64 * wave; p0 < cpr; p0 += TH)
                if (p0 + lane < cpr)  // rows past m: zeros (descriptor of size 0)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        bload128_lds(xr, xm + (size_t)(e * cpr + p0) * 16, (4u * (uint32_t)(p0 + lane) + (uint32_t)e) * 16u);
        }
    }

    // code book and nested code2 table; the barrier (without the release fence of
    // __syncthreads) then publishes every wave's share of them and of X
    wait_vmcnt<0>();
    if (tid < 256) {
        lut2[tid] = float2_t{b_hi, b_lo};
        if constexpr (NESTED) c2[tid] = c2v;
    }
    lds_barrier();

    // k-range p (chunk within its row) of the thread's chunk i: advanced by 256 chunks a step
    // tid % cpr and TH % cpr without a division: cpr_inv = ceil(2^20 / cpr), exact for
    // numerators below 512 while cpr <= 2048 (the error term n (cpr_inv cpr - 2^20) stays below 2^20)
    int pk = tid - (int)__umul24((uint32_t)cpr, __umul24((uint32_t)tid, cpr_inv) >> 20);
    const int dp = TH - cpr * (int)(((uint32_t)TH * cpr_inv) >> 20);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + TH * i;
        float sc = s[i];
        if constexpr (NESTED) sc = c2[q8[i]] * sc + offset;  // two roundings (no contraction)
        const int pc = c < nch ? pk : 0;
        pk += dp;
        if (pk >= cpr) pk -= cpr;
        // the 32 X values of this chunk for every token row: dword j of piece e holds
        // X[32 p + 8 e + 2 j] and X[32 p + 8 e + 2 j + 1]. One or two token rows: all four
        // pieces read up front; more rows: piece by piece (16 registers a row otherwise)
        constexpr bool kXAll = MT <= 2;
        u32x4_t xv[kXAll ? MT : 1][4];
        if constexpr (kXAll)
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[m][e] = *(const u32x4_t*)(xs + m * K + (e * cpr + pc) * 8);
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            u32x4_t xe[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m)
                xe[m] = kXAll ? xv[kXAll ? m : 0][e] : *(const u32x4_t*)(xs + m * K + (e * cpr + pc) * 8);
            const uint32_t w = p[i][e];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // packed byte 4 e + q: weights 32 p + 8 e + 2 q (high nibble) and + 1
                const float2_t cv = *(const float2_t*)((const char*)lut2 + byte_x8(w, q));
                const half2_t w2 = __builtin_bit_cast(half2_t, pack_half2(cv.x * sc, cv.y * sc));
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    // elements copied to a scalar first: hipcc compiles __builtin_bit_cast of a
                    // vector element v[j] as element 0 whatever j is
                    const uint32_t xq = xe[m][q];
                    acc[m] = __builtin_amdgcn_fdot2(w2, __builtin_bit_cast(half2_t, xq), acc[m], false);
                }
            }
        }
        // the chunk's sums go to LDS at once (kept in registers to the end, the compiler sinks
        // their arithmetic below everything and holds every chunk's operands meanwhile)
        if (c < nch)
#pragma unroll
            for (int m = 0; m < MT; ++m) part[m * nch + c] = acc[m];
    }
    lds_barrier();

    // each row's sum in a fixed order: a wave sums four rows at once, 16 lanes each; lane j of a
    // row adds its slots j, j + 16, ... in turn, then the 16 lanes combine in four DPP steps
    // (lane j with lanes j ^ 1, j ^ 2, then rotations by 4 and 8 within the 16), and lane 0 of
    // the 16 stores. The order depends only on k.
    const int sub = lane >> 4, j16 = lane & 15;
    for (int r0 = 4 * wave; r0 < rows; r0 += TH / 16) {
        const int r = r0 + sub;
        float v[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            v[m] = 0.0f;
            if (r < rows) {
                // four reads in flight at a time, added in slot order
                const float* pr = part + m * nch + r * cpr;
                int q = j16;
                for (; q + 48 < cpr; q += 64) {
                    const float t0 = pr[q], t1 = pr[q + 16], t2 = pr[q + 32], t3 = pr[q + 48];
                    v[m] += t0;
                    v[m] += t1;
                    v[m] += t2;
                    v[m] += t3;
                }
                for (; q < cpr; q += 16) v[m] += pr[q];
            }
            v[m] = row16_sum(v[m]);
        }
        if (j16 == 0 && r < rows) {
            const int n = n0 + r;
            const float b = G.bias != nullptr ? (float)G.bias[n] : 0.0f;
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m < M) G.y[(int64_t)(MT * tg + m) * G.ldy + n] = to_half(v[m] + b);
        }
    }
}

// Work-group shape of a launch: `threads` per work-group, `cpt` chunk loads per thread and
// `rows` rows per work-group (rows * cpr <= threads * cpt).
struct GemvShape {
    int cpt, rows, threads = kGemvThreads;
};

// The fewest loads per thread whose rows fill at least 95% of them, else the best fill (4 to 8
// loads per thread): the shape that bounds the LDS a launch of contraction k needs.
static GemvShape gemv_shape_bound(int k) {
    const int cpr = k >> 5;
    GemvShape best{0, 0};
    double best_fill = -1.0;
    for (int cpt = 4; cpt <= kGemvMaxChunks; ++cpt) {
        const int rows = kGemvThreads * cpt / cpr;
        if (rows < 1) continue;
        const double fill = (double)rows * cpr / (kGemvThreads * cpt);
        if (fill >= 0.95) return GemvShape{cpt, rows};
        if (fill > best_fill + 1e-9) {
            best_fill = fill;
            best = GemvShape{cpt, rows};
        }
    }
    return best;
}

// Token rows a work-group of a launch of m rows computes (X rows past m read as zeros); past
// four rows two work-groups share each weight row range, one per four token rows
static int gemv_mt(int64_t m) { return m <= 1 ? 1 : m <= 2 ? 2 : 4; }

// Whether the GEMV takes a launch of m token rows and contraction k (a row must fit one
// work-group's loads, X of the token rows and the sums must fit LDS).
bool gemv_fits(int64_t m, int64_t k) {
    if (m < 1 || m > kGemvMaxM || k <= 0 || k % 32 != 0 || k > kGemvThreads * kGemvMaxChunks * 32) return false;
    const GemvShape sh = gemv_shape_bound((int)k);
    return sh.rows >= 1 && gemv_smem_bytes(gemv_mt(m), (int)k, sh.rows * (int)(k >> 5)) <= 158 * 1024;
}

// The shape of a launch of `nrows` weight rows and mt token rows. Every work-group stages X
// (2 k mt bytes) next to its rows' packed bytes (k / 2 per row), and fewer loads per thread
// mean more, lighter work-groups in flight. Among the load counts whose rows fill at least 75%
// of the loads: the fewest with at least 4 mt rows (X traffic at most the weight's), unless that
// leaves fewer than 1024 work-groups -- then the fewest of all, for parallelism. Graph-replayed
// on MI355X at one token (us, against the previous 4-8-load rule): 7B gate 17.0 -> 15.3, k/v
// 5.5 -> 3.7, q/o 7.6 -> 6.3; Qwen2.5-1.5B gate 8.4 -> 6.7, down 8.9 -> 7.1, q/o 6.4 -> 4.3,
// k/v 6.0 -> 3.7. The row sums keep their order whatever the shape: the same bits.
static GemvShape gemv_shape(int k, int64_t nrows, int mt, int tgroups) {
    const int cpr = k >> 5;
    GemvShape fewest{0, 0}, most{0, 0};
    double most_fill = -1.0;
    for (int cpt = 1; cpt <= kGemvMaxChunks; ++cpt) {
        const int rows = kGemvThreads * cpt / cpr;
        if (rows < 1) continue;
        const double fill = (double)rows * cpr / (kGemvThreads * cpt);
        if (fill < 0.75) continue;
        if (fewest.cpt == 0) fewest = GemvShape{cpt, rows};
        if (rows >= 4 * mt) {
            most = GemvShape{cpt, rows};
            break;
        }
        if (rows > most.rows || (rows == most.rows && fill > most_fill + 1e-9)) {
            most = GemvShape{cpt, rows};
            most_fill = fill;
        }
    }
    if (most.cpt == 0) return gemv_shape_bound(k);
    GemvShape pick = (nrows + most.rows - 1) / most.rows >= 1024 ? most : fewest;
    if (gemv_smem_bytes(mt, k, pick.rows * cpr) > 158 * 1024) return gemv_shape_bound(k);
    if (mt >= 4) {
        // Four token rows: every work-group stages X of four rows (8 k bytes), so the LDS bounds
        // how many a CU holds; from the pick up, the fewest loads per thread whose work-groups
        // run in one round. Graph-replayed at 4 rows: 7B q/o 12.4 -> 9.3 us (4 rows a
        // work-group instead of 2: 896 work-groups of 39 KB instead of 1792 of 35 KB).
        const int cus = device_cus();
        for (int cpt = pick.cpt; cpt <= kGemvMaxChunks; ++cpt) {
            const int rows = kGemvThreads * cpt / cpr;
            if (rows < 1 || (double)rows * cpr < 0.75 * kGemvThreads * cpt) continue;
            const size_t lds = gemv_smem_bytes(mt, k, rows * cpr) + 256 * sizeof(float2_t);  // + code book
            if (lds > 158 * 1024) break;
            const int64_t per_cu = std::min<int64_t>(32 / (kGemvThreads / 64), (int64_t)(160 * 1024 / lds));
            if ((nrows + rows - 1) / rows * tgroups <= per_cu * cus) {
                pick = GemvShape{cpt, rows};
                break;
            }
        }
    }
    if (gemv_smem_bytes(mt, k, pick.rows * cpr) > kGemvWideLds) {
        // X of long rows limits the work-groups a CU holds (three four-wave work-groups, 12 waves,
        // from 40 KB): eight-wave work-groups with at least 4 loads per thread and 85% fill double
        // the waves per CU for the same LDS. Graph-replayed at one token: 7B down ([3584, 18944])
        // 19.3-21.2 -> 17.5-18.1 us; the shorter-row shapes gained nothing (their work-groups
        // already fill the CU's waves).
        for (int cpt = 4; cpt <= kGemvMaxChunks; ++cpt) {
            const int rows = 2 * kGemvThreads * cpt / cpr;
            if (rows < 1 || (double)rows * cpr < 0.85 * 2 * kGemvThreads * cpt) continue;
            if (gemv_smem_bytes(mt, k, rows * cpr) <= 158 * 1024) return GemvShape{cpt, rows, 2 * kGemvThreads};
            break;
        }
    }
    return pick;
}

template <int MT, bool NESTED, int CPT, int TH>
static hipError_t launch_gemv_th(const FwdArgs& a, int rows, int grid, int tg_shift, hipStream_t s) {
    const size_t lds = gemv_smem_bytes(MT, a.k, rows * (a.k >> 5));
    const hipError_t e = allow_dynamic_lds((const void*)nf4_gemv_kernel<MT, NESTED, CPT, TH>, lds);
    if (e != hipSuccess) return e;
    const uint32_t cpr = (uint32_t)(a.k >> 5), cpr_inv = ((1u << 20) + cpr - 1) / cpr;
    hipLaunchKernelGGL((nf4_gemv_kernel<MT, NESTED, CPT, TH>), dim3(grid << tg_shift), dim3(TH), lds, s, a, rows, cpr_inv,
                       tg_shift);
    return hipGetLastError();
}

template <int MT, bool NESTED, int CPT>
static hipError_t launch_gemv_t(const FwdArgs& a, const GemvShape& sh, int grid, int tg_shift, hipStream_t s) {
    if constexpr (CPT >= 4)  // eight-wave shapes take at least 4 loads per thread
        if (sh.threads == 2 * kGemvThreads) return launch_gemv_th<MT, NESTED, CPT, 2 * kGemvThreads>(a, sh.rows, grid, tg_shift, s);
    if (sh.threads != kGemvThreads) return hipErrorInvalidValue;
    return launch_gemv_th<MT, NESTED, CPT, kGemvThreads>(a, sh.rows, grid, tg_shift, s);
}

template <int MT, bool NESTED>
static hipError_t launch_gemv_cpt(const FwdArgs& a, const GemvShape& sh, int grid, int tg_shift, hipStream_t s) {
    switch (sh.cpt) {
        case 1: return launch_gemv_t<MT, NESTED, 1>(a, sh, grid, tg_shift, s);
        case 2: return launch_gemv_t<MT, NESTED, 2>(a, sh, grid, tg_shift, s);
        case 3: return launch_gemv_t<MT, NESTED, 3>(a, sh, grid, tg_shift, s);
        case 4: return launch_gemv_t<MT, NESTED, 4>(a, sh, grid, tg_shift, s);
        case 5: return launch_gemv_t<MT, NESTED, 5>(a, sh, grid, tg_shift, s);
        case 6: return launch_gemv_t<MT, NESTED, 6>(a, sh, grid, tg_shift, s);
        case 7: return launch_gemv_t<MT, NESTED, 7>(a, sh, grid, tg_shift, s);
        case 8: return launch_gemv_t<MT, NESTED, 8>(a, sh, grid, tg_shift, s);
        default: return hipErrorInvalidValue;
    }
}

int gemv_waves(int64_t m, int64_t k, int64_t nrows) {
    return gemv_shape((int)k, nrows, gemv_mt(m), m > 4 ? 2 : 1).threads / 64;
}

// a: the groups' tile_begin fields are overwritten with their first work-group
hipError_t launch_gemv(FwdArgs& a, hipStream_t s) {
    if (a.glu || !gemv_fits(a.m, a.k)) return hipErrorInvalidValue;
    for (int g = 0; g < a.ngroups; ++g)
        if (a.g[g].lora_u != nullptr) return hipErrorInvalidValue;
    int64_t nrows = 0;
    for (int g = 0; g < a.ngroups; ++g) nrows += a.g[g].w.n;
    const int mt = gemv_mt(a.m);
    const GemvShape sh = gemv_shape(a.k, nrows, mt, a.m > 4 ? 2 : 1);
    int grid = 0;
    for (int g = 0; g < a.ngroups; ++g) {
        a.g[g].tile_begin = grid;
        grid += (int)((a.g[g].w.n + sh.rows - 1) / sh.rows);
    }
    const int tg_shift = a.m > 4 ? 1 : 0;
    switch (mt) {
        case 1: return a.nested ? launch_gemv_cpt<1, true>(a, sh, grid, 0, s) : launch_gemv_cpt<1, false>(a, sh, grid, 0, s);
        case 2: return a.nested ? launch_gemv_cpt<2, true>(a, sh, grid, 0, s) : launch_gemv_cpt<2, false>(a, sh, grid, 0, s);
        default: return a.nested ? launch_gemv_cpt<4, true>(a, sh, grid, tg_shift, s) : launch_gemv_cpt<4, false>(a, sh, grid, tg_shift, s);
    }
}

}  // namespace dk
