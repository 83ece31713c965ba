// Fused NF4 dequant x fp16 GEMM, input gradient (replaces dequantize_nf4 + matmul,
// solution/nf4.py:99-104, and the summed input gradients of solution/mlp.py:106-109):
//
//     dX[m, k] = sum_g sum_n dY_g[m, n] W_g[n, k]  (+ sum_g GU_g[m, t] A_g[t, k] for LoRA)
//
// MFMA v_mfma_f32_32x32x16_f16, fp32 accumulation. The contraction runs over weight rows n, so
// A = W^T (32 output columns x 16 weight rows) and B = dY^T (16 weight rows x 32 tokens), and
// D = (dY.W)^T. Work-group = 8 waves (two per SIMD); tile = 32*MB tokens x 512 output columns,
// 64 columns per wave; main-loop step = 64 weight rows.
//
// A operands straight from the packed bytes: lane l (l32 = l % 32, g = l / 32) serves A row
// l32 of two MFMA column blocks cb = 0, 1, mapped to output column 2 beta + cb of the wave's
// 64, beta = arow_to_n(l32) -- the high and low nibble of packed byte beta of a row. Its eight
// contraction slots of slice j are the eight weight rows 32 g + 8 j + e (the permutation
// freedom of the MFMA sum; dY's B operand uses the same order). With this column order each
// lane ends with 32 consecutive output columns of one token row.
//
// Each wave stages its own packed bytes in LDS as 8-row groups of 4-row quads per dword-column
// (a dword = 4 bytes of one row): the global loads stay contiguous along rows (8 rows x 32
// bytes per instruction) and a lane reads its eight rows of one dword-column with two 16-byte
// loads. Row scales
// (one per row and 32-column half: blocks are 32-aligned in the flat index) are computed one
// step ahead, one row per lane, and published in a per-wave LDS table. dY tiles (32*MB x 64
// fp16) are shared by the work-group. All global loads go straight into LDS rings
// (buffer_load ... lds) issued up to three steps ahead; each step ends with one wait and one
// barrier. Split-K: fp32 partial slabs reduced by splitk_reduce_kernel.
#include "gemm_common.h"

namespace dk {

constexpr int kBwdTableBytes = 256 * 4;                   // per group: code2 table
constexpr int kBwdHeader = kMaxGroups * kBwdTableBytes;    // 4096 (code books: static LDS)
constexpr int kBwdPkStride = 72;                           // dwords per 8-row group (64 + pad)
constexpr int kBwdPkBytes = 8 * kBwdPkStride * 4;          // 2304: packed bytes of 64 rows
constexpr int kBwdStatBytes = 1024;                        // codes / absmax: 2 x 256, absmax2: 2 x 256
constexpr int kBwdWSlot = kBwdPkBytes + kBwdStatBytes;     // 3328
constexpr int kBwdScaleBytes = 2 * 2 * 64 * 4;             // [parity][half][row] fp32

__host__ __device__ constexpr size_t bwd_smem_bytes(int mb, int waves) {
    return kBwdHeader + 3 * (size_t)(32 * mb * 128) + waves * (3 * (size_t)kBwdWSlot + kBwdScaleBytes);
}

// WAVES = 8: one work-group per CU, 512 output columns; WAVES = 4: two per CU, 256 columns (more
// work-groups for launches with few output tiles).
template <int MB, int WAVES, bool NESTED>
__global__ __launch_bounds__(64 * WAVES, 8 / WAVES) void nf4_bwd_kernel(const BwdArgs a) {
    constexpr int NT = 64 * WAVES;                   // threads
    constexpr int BN = 64 * WAVES;                   // output columns per tile
    constexpr int BM = 32 * MB;
    constexpr int DBUF = BM * 128;                   // bytes of one dY ring buffer
    constexpr int DPT = BM * 8 / NT;                 // 16-byte dY loads per thread and step
    static_assert(DPT * NT == BM * 8, "dY tile loader: whole loads per thread");
    constexpr int NL = DPT + 8 + (NESTED ? 2 : 1);   // loads per thread and step (narrow; the
                                                     // wide layout has more: waits stay safe)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* dring = smem + kBwdHeader;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
    const int l32 = lane & 31, g = lane >> 5;
    const int beta = arow_to_n(l32);      // this lane's packed byte within the wave's 32
    const int half = beta >> 4;           // ... and its 32-column half (scale)
    const int xsw = (l32 >> 1) & 7;       // LDS swizzle of this lane's dY rows
    // Narrow statistics (every blocksize >= 64 and k % 64 == 0): a row's 64 wave columns lie in
    // one block, one scale per row. Wide: one scale per row and 32-column half.
    const bool wide = a.wide_stats != 0;

    const int L = xcd_logical_id();
    if (L >= a.m_tiles * a.k_tiles * a.splits) return;
    const int m_tile = L % a.m_tiles;
    const int rest = L / a.m_tiles;
    const int k_tile = rest % a.k_tiles;
    const int split = rest / a.k_tiles;
    const int M = sgpr(a.m), K = sgpr(a.k);
    const int m0 = m_tile * BM;
    const int kw0 = k_tile * BN + 64 * wave;  // wave's first output column
    const int cs0 = split * a.csteps_per_split;
    const int cs1 = min(a.csteps, cs0 + a.csteps_per_split);

    // every group's code book (static LDS, group g at byte 64 g) and code2 table
    __shared__ float luts[16 * kMaxGroups];
    for (int gg = 0; gg < a.ngroups; ++gg) {
        if (tid < 16) luts[16 * gg + tid] = a.g[gg].w.code[tid];
        if (NESTED && tid < 256) ((float*)(smem + gg * kBwdTableBytes))[tid] = a.g[gg].w.code2[tid];
    }
    // v_perm selector that gathers byte (beta & 3) of two dwords into the low two bytes
    const uint32_t bsel = (uint32_t)(beta & 3) | ((uint32_t)((beta & 3) + 4) << 8) | 0x0C0C0000u;

    uint8_t* wring = dring + 3 * DBUF + wave * (3 * kBwdWSlot);
    float* scales = (float*)(dring + 3 * DBUF + WAVES * 3 * kBwdWSlot + wave * kBwdScaleBytes);

    float16_t acc[MB * 2];  // [token block i][column block cb] at i * 2 + cb
#pragma unroll
    for (int t = 0; t < MB * 2; ++t) acc[t] = float16_t{};

    // LoRA input-gradient terms GU_g . A_g first (split 0 only; trip count 0 without LoRA).
    {
        const int R = split == 0 ? sgpr(a.lora_rank) : 0;
        for (int gg = 0; gg < a.ngroups; ++gg) {
            const BwdGroupDev& G = a.g[gg];
            if (G.lora_gu == nullptr || G.lora_keep != nullptr || R == 0) continue;  // dropout: epilogue
            const rsrc_t ars = make_rsrc(G.lora_a, (uint32_t)R * (uint32_t)K * 2u);
            const rsrc_t grs = make_rsrc(G.lora_gu, (uint32_t)M * (uint32_t)R * 2u);
            for (int t0 = 0; t0 < R; t0 += 16) {
                half8_t al[2];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int tr = t0 + 8 * g + e;
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        const int col = kw0 + 2 * beta + cb;
                        al[cb][e] = __builtin_bit_cast(
                            _Float16, (uint16_t)bload16(ars, off_if(col < K, (uint32_t)(tr * K + col) * 2u)));
                    }
                }
#pragma unroll
                for (int i = 0; i < MB; ++i) {
                    const int m = m0 + 32 * i + l32;
                    const half8_t gu = __builtin_bit_cast(
                        half8_t, bload128(grs, off_if(m < M, (uint32_t)(m * R + t0 + 8 * g) * 2u)));
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) acc[i * 2 + cb] = mfma32x32x16(al[cb], gu, acc[i * 2 + cb]);
                }
            }
        }
    }

    // Software pipeline over 16-row slices, as in the forward kernel: while the 2*MB MFMAs of
    // slice j run, the wave prepares slice j + 1 in stages placed between them (sched_barrier
    // keeps each stage next to its MFMA): A = reads of its packed dwords, row scales and dY
    // fragments; B = byte gather, code-book addresses and code-book reads; C = scaling and fp16
    // packing. Step t+1's row scales are made during slice 2 (its statistics are this wave's own
    // loads); the barrier before step t+1's dY fragments sits between slice 3's MFMAs.
    constexpr int nm = 2 * MB;  // MFMAs per slice
    constexpr int qB = nm >= 8 ? 1 : (nm >= 4 ? 1 : 0);
    constexpr int qC0 = nm >= 8 ? nm / 2 + 1 : (nm >= 4 ? 2 : 1);
    constexpr int qC1 = qC0 + (nm >= 4 ? 1 : 0);
    constexpr int qBar = nm >= 8 ? 2 : (nm >= 4 ? qC0 : 0);

    // One weight group at a time: the group's operands (pointers, sizes, block-size shifts, the
    // nested offset) are read once before its steps, so the per-step code issues no scalar
    // memory loads -- their out-of-order returns would make every later wait drain all
    // outstanding LDS reads. The pipeline drains between groups.
    for (int gi = 0; gi < a.ngroups; ++gi) {
        const BwdGroupDev& G = a.g[gi];
        const int sb = sgpr(G.step_begin);
        const int t0 = max(cs0, sb), t1 = min(cs1, sb + sgpr(G.nsteps));
        if (t0 >= t1) continue;
        const int N = sgpr((int)G.w.n);
        const int lddy = sgpr(G.lddy);
        // the group's buffers, held in scalar registers for the whole segment
        const _Float16* const gdy = sgpr(G.dy);
        const uint32_t dy_bytes = sgpr(G.dy_bytes);
        const uint8_t* const gpk = sgpr(G.w.packed);
        const uint32_t pk_bytes = sgpr(G.w.packed_bytes);
        const uint8_t* const gam8 = NESTED ? sgpr(G.w.absmax8) : nullptr;
        const float* const gamf = NESTED ? nullptr : sgpr(G.w.absmaxf);
        const uint32_t am_bytes = sgpr(G.w.absmax_bytes);
        const float* const gam2 = NESTED ? sgpr(G.w.absmax2) : nullptr;
        const uint32_t am2_bytes = NESTED ? sgpr(G.w.absmax2_bytes) : 0u;
        const uint32_t bs_shift = sgpr((uint32_t)G.w.bs_shift), bs2_shift = sgpr((uint32_t)G.w.bs2_shift);
        const float offset = NESTED ? *G.w.offset : 0.0f;
        const float* c2 = (const float*)(smem + gi * kBwdTableBytes);
        const uint32_t gbase4 = (uint32_t)(64 * gi) * 0x01010101u;  // this group's code book

        // Loads use per-lane offsets fixed for the group (bit 31 set where the lane's data lies
        // outside the tile or the weight: it reads zeros) against buffer descriptors whose base
        // advances by whole steps, so a step costs scalar additions. Only a group's last step,
        // when its row count is not a multiple of 64, also checks rows per lane. A step past the
        // segment's end loads from descriptors of size 0 (zeros), keeping the load count uniform.
        uint32_t dyo[DPT];  // dY chunk h of this thread: token row (tid + NT h) / 8 of the tile
        int dyc[DPT];       // ... its first column within the step
#pragma unroll
        for (int h = 0; h < DPT; ++h) {
            const int q = tid + NT * h;
            const int row = q >> 3, pc = q & 7;
            const int c = pc ^ ((row >> 1) & 7);
            const int gm = m0 + row;
            dyc[h] = 8 * c;
            dyo[h] = off_if(gm < M, (uint32_t)(gm * lddy + 8 * c) * 2u);
        }
        // packed bytes: instruction d fetches rows 8 d .. 8 d + 7, all 8 dwords (32 contiguous
        // bytes) of each; lane -> (row quad, dword-column, row) lands at dword
        // 72 d + 32 rq + 4 cg + rho
        const int rq = lane >> 5, cg = (lane >> 2) & 7, rho = lane & 3;
        const uint32_t po = off_if(kw0 + 8 * cg < K, (uint32_t)(4 * rq + rho) * (uint32_t)(K >> 1) + (uint32_t)((kw0 + 8 * cg) >> 1));
        const uint32_t prow8 = 8u * (uint32_t)(K >> 1);  // bytes of 8 weight rows
        // statistics: lane = weight row of the step, one block per 32-column half
        uint32_t blk0[2], so[2];
        bool cok[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            cok[hh] = kw0 + 32 * hh < K;
            blk0[hh] = ((uint32_t)lane * (uint32_t)K + (uint32_t)(kw0 + 32 * hh)) >> bs_shift;
            so[hh] = off_if(cok[hh], NESTED ? blk0[hh] : blk0[hh] * 4u);
        }

        auto load_step = [&](int t, int rd, int rw, bool live) __attribute__((always_inline)) {
            const int n0 = (t - sb) * kBwdBC;
            const bool tail = n0 + kBwdBC > N;  // uniform
            const rsrc_t drs = make_rsrc(gdy + n0, live ? dy_bytes - 2u * (uint32_t)n0 : 0u);
            uint8_t* slot = wring + rw;
            const uint32_t pskip = (uint32_t)n0 * (uint32_t)(K >> 1);
            const rsrc_t wrs = make_rsrc(gpk + pskip, live ? pk_bytes - pskip : 0u);
            if (!tail) {
#pragma unroll
                for (int h = 0; h < DPT; ++h) bload128_lds(drs, dring + rd + (NT * h + 64 * wave) * 16, dyo[h]);
#pragma unroll
                for (int d = 0; d < 8; ++d) bload32_lds(wrs, slot + d * kBwdPkStride * 4, po + (uint32_t)d * prow8);
            } else {
                // the group's last step with fewer than 64 rows left: rows and dY columns past N
                // read zeros
#pragma unroll
                for (int h = 0; h < DPT; ++h)
                    bload128_lds(drs, dring + rd + (NT * h + 64 * wave) * 16, off_if(n0 + dyc[h] < N, dyo[h]));
#pragma unroll
                for (int d = 0; d < 8; ++d)
                    bload32_lds(wrs, slot + d * kBwdPkStride * 4,
                                off_if(n0 + 8 * d + 4 * rq + rho < N, po + (uint32_t)d * prow8));
            }
            const uint32_t kb = ((uint32_t)n0 * (uint32_t)K) >> bs_shift;  // blocks before this step
            const bool rok = !tail || n0 + lane < N;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                if (hh == 1 && !wide) break;
                if constexpr (NESTED) {
                    const rsrc_t ars = make_rsrc(gam8 + kb, live ? am_bytes - kb : 0u);
                    const rsrc_t a2rs = make_rsrc(gam2, live ? am2_bytes : 0u);
                    bload8_lds(ars, slot + kBwdPkBytes + 256 * hh, off_if(rok, so[hh]));
                    bload32_lds(a2rs, slot + kBwdPkBytes + 512 + 256 * hh,
                                off_if(rok && cok[hh], ((blk0[hh] + kb) >> bs2_shift) * 4u));
                } else {
                    const rsrc_t ars = make_rsrc(gamf + kb, live ? am_bytes - 4u * kb : 0u);
                    bload32_lds(ars, slot + kBwdPkBytes + 256 * hh, off_if(rok, so[hh]));
                }
            }
        };
        // Row scales of step t (this lane's row, both halves) from slot rw into scale table sidx.
        // The statistics were fetched by this same wave, so its own wait suffices (no barrier).
        auto make_scales = [&](int t, int rw, int sidx) __attribute__((always_inline)) {
            const int row = (t - sb) * kBwdBC + lane;
            const uint8_t* slot = wring + rw;
            float* dst = scales + sidx * 128;
            for (int hh = 0; hh < (wide ? 2 : 1); ++hh) {
                const bool ok = row < N && cok[hh];
                float sc;
                if constexpr (NESTED) {
                    const uint32_t q = slot[kBwdPkBytes + 256 * hh + 4 * lane];
                    const float a2 = *(const float*)(slot + kBwdPkBytes + 512 + 256 * hh + 4 * lane);
                    sc = c2[q] * a2 + offset;
                } else {
                    sc = *(const float*)(slot + kBwdPkBytes + 256 * hh + 4 * lane);
                }
                dst[64 * hh + lane] = ok ? sc : 0.0f;
            }
        };

        // Ring buffers: step t uses dY buffer rd0 (byte offset in the dY ring), weight slot rw0
        // and scale table si0; step t + 1 uses rd1 / rw1 / 1 - si0; step t + 3 reuses step t's.
        int rd0 = 0, rw0 = 0, rd1 = DBUF, rw1 = kBwdWSlot, si0 = 0;
        // Prologue: three steps in flight; wait for the first.
        load_step(t0, 0, 0, true);
        load_step(t0 + 1, DBUF, kBwdWSlot, t0 + 1 < t1);
        load_step(t0 + 2, 2 * DBUF, 2 * kBwdWSlot, t0 + 2 < t1);
        wait_vmcnt<2 * NL>();
        lds_barrier();  // dY(t0) from every wave, code tables
        make_scales(t0, 0, 0);

        half8_t xf[MB], w0, w1;      // operands of the current slice
        half8_t xn[MB], wn0, wn1;    // ... of the next slice
        u32x4_t d0, d1;              // next slice: packed dwords of rows r0 .. r0 + 3, r0 + 4 .. r0 + 7
        float4_t s0, s1;             // ... and their row scales
        float vh[8], vl[8];          // ... code-book values of the high and low nibbles
        auto stage_A = [&](int rw, int sidx, int j) __attribute__((always_inline)) {
            const uint32_t* pk = (const uint32_t*)(wring + rw) + 4 * (beta >> 2);
            const float* sc = scales + sidx * 128 + (wide ? 64 * half : 0);
            const int r0 = 32 * g + 8 * j, dg = 4 * g + j;
            d0 = *(const u32x4_t*)(pk + kBwdPkStride * dg);
            d1 = *(const u32x4_t*)(pk + kBwdPkStride * dg + 32);
            s0 = *(const float4_t*)(sc + r0);
            s1 = *(const float4_t*)(sc + r0 + 4);
        };
        auto stage_X = [&](int rd, int j) __attribute__((always_inline)) {
            const uint8_t* db = dring + rd;
#pragma unroll
            for (int i = 0; i < MB; ++i)
                xn[i] = *(const half8_t*)(db + (32 * i + l32) * 128 + (((4 * g + j) ^ xsw) << 4));
        };
        auto stage_B = [&]() __attribute__((always_inline)) {
            // this lane's byte of rows r0 .. r0 + 3 and r0 + 4 .. r0 + 7, gathered into two dwords
            const uint32_t rb0 = __builtin_amdgcn_perm(d0[1], d0[0], bsel) | (__builtin_amdgcn_perm(d0[3], d0[2], bsel) << 16);
            const uint32_t rb1 = __builtin_amdgcn_perm(d1[1], d1[0], bsel) | (__builtin_amdgcn_perm(d1[3], d1[2], bsel) << 16);
            uint32_t ah0, al0, ah1, al1;
            nib_addrs(rb0, gbase4, ah0, al0);
            nib_addrs(rb1, gbase4, ah1, al1);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vh[e] = lut_at(luts, ah0, e);
                vl[e] = lut_at(luts, al0, e);
                vh[e + 4] = lut_at(luts, ah1, e);
                vl[e + 4] = lut_at(luts, al1, e);
            }
        };
        auto stage_C = [&](const float* v) __attribute__((always_inline)) -> half8_t {
            u32x4_t o;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                o[q] = pack_half2(v[2 * q] * s0[2 * q], v[2 * q + 1] * s0[2 * q + 1]);
                o[q + 2] = pack_half2(v[2 * q + 4] * s1[2 * q], v[2 * q + 5] * s1[2 * q + 1]);
            }
            return __builtin_bit_cast(half8_t, o);
        };
        auto mfma_q = [&](int q) __attribute__((always_inline)) {
            const int i = q >> 1;
            if (q & 1)
                acc[i * 2 + 1] = mfma32x32x16(w1, xf[i], acc[i * 2 + 1]);
            else
                acc[i * 2 + 0] = mfma32x32x16(w0, xf[i], acc[i * 2 + 0]);
        };

        // slice 0 of the first step
        stage_A(rw0, si0, 0);
        stage_X(rd0, 0);
        stage_B();
        w0 = stage_C(vh);
        w1 = stage_C(vl);
#pragma unroll
        for (int i = 0; i < MB; ++i) xf[i] = xn[i];

        for (int t = t0; t < t1; ++t) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int q = 0; q < nm; ++q) {
                    mfma_q(q);
                    if (j < 3) {
                        if (q == 0) {
                            if (j == 2) {
                                // step t+1's loads have landed (only step t+2's may be in
                                // flight): its row scales from its statistics (this wave's own
                                // loads)
                                wait_vmcnt<NL>();
                                make_scales(t + 1, rw1, 1 - si0);
                            }
                            stage_A(rw0, si0, j + 1);
                            stage_X(rd0, j + 1);
                        }
                        if (q == qB) stage_B();
                    } else {
                        if (q == 0) stage_A(rw1, 1 - si0, 0);
                        if (q == qB) stage_B();
                        if (q == qBar) {
                            // every wave is past step t's slots: refill them with step t+3
                            // (zeros past the segment's end). Past the last step the reads of
                            // this slice see stale slots and their values go unused.
                            lds_barrier();
                            load_step(t + 3, rd0, rw0, t + 3 < t1);
                            stage_X(rd1, 0);
                        }
                    }
                    if (q == qC0) wn0 = stage_C(vh);
                    if (q == qC1) wn1 = stage_C(vl);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int i = 0; i < MB; ++i) xf[i] = xn[i];
                w0 = wn0;
                w1 = wn1;
            }
            // rotate the rings: step t + 1's buffers become the current ones
            rd0 = rd1;
            rw0 = rw1;
            rd1 = rd1 == 2 * DBUF ? 0 : rd1 + DBUF;
            rw1 = rw1 == 2 * kBwdWSlot ? 0 : rw1 + kBwdWSlot;
            si0 = 1 - si0;
        }
        // every load has landed and every wave is done with the rings before the next group's
        // prologue refills them
        wait_vmcnt<0>();
        lds_barrier();
    }

    // ---- epilogue: lane (l32, g) holds columns kw0 + 32 g + c, c = 2 r + cb, of token rows
    // m0 + 32 i + l32 (acc[i * 2 + cb][r]).
    // LoRA input-gradient terms of branches whose input went through dropout (split 0): per token
    // block, P = GU_g . A_g on its own, rounded to fp16, times keep and the keep scale in fp32,
    // then added. Lane value (cb, r) of token block i is column kw0 + 32 g + 2 r + cb: bit 2 r + cb
    // of the four keep bytes at column (kw0 + 32 g) / 8 of the token's row.
    if (split == 0) {
        const int R = sgpr(a.lora_rank);
        const bool kok = kw0 + 32 * g < K;  // k % 32 == 0: the lane's 32 columns all in or out
        for (int gg = 0; gg < a.ngroups; ++gg) {
            const BwdGroupDev& G = a.g[gg];
            if (G.lora_keep == nullptr || G.lora_gu == nullptr || R == 0) continue;
            const rsrc_t ars = make_rsrc(G.lora_a, (uint32_t)R * (uint32_t)K * 2u);
            const rsrc_t grs = make_rsrc(G.lora_gu, (uint32_t)M * (uint32_t)R * 2u);
            const rsrc_t krs = make_rsrc(G.lora_keep, (uint32_t)M * (uint32_t)(K >> 3));
            const float ks = G.lora_keep_scale;
            half8_t al[2][2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 8; ++e)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        const int col = kw0 + 2 * beta + cb;
                        al[h][cb][e] = __builtin_bit_cast(
                            _Float16, (uint16_t)bload16(ars, off_if(col < K && 16 * h < R,
                                                                    (uint32_t)((16 * h + 8 * g + e) * K + col) * 2u)));
                    }
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int m = m0 + 32 * i + l32;
                float16_t p[2] = {};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8_t gu = __builtin_bit_cast(
                        half8_t, bload128(grs, off_if(m < M && 16 * h < R, (uint32_t)(m * R + 16 * h + 8 * g) * 2u)));
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) p[cb] = mfma32x32x16(al[h][cb], gu, p[cb]);  // zeros past the rank
                }
                const uint32_t bits = __builtin_bit_cast(
                    uint32_t, bloadf(krs, off_if(m < M && kok, (uint32_t)m * (uint32_t)(K >> 3) +
                                                                 (uint32_t)((kw0 + 32 * g) >> 3))));
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[i * 2 + cb][r] = acc[i * 2 + cb][r] +
                                             ((float)(_Float16)p[cb][r] * (float)((bits >> (2 * r + cb)) & 1u)) * ks;
            }
        }
    }
    const int kc = kw0 + 32 * g;
    if (a.splits > 1) {
        float* slab = a.partials + (int64_t)split * M * K;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int m = m0 + 32 * i + l32;
            if (m >= M) continue;
            float* dst = slab + (int64_t)m * K + kc;
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (kc + 4 * q < K)  // k % 32 == 0: this lane's 32 columns are all in or all out
                    *(float4_t*)(dst + 4 * q) = float4_t{acc[i * 2][2 * q], acc[i * 2 + 1][2 * q],
                                                         acc[i * 2][2 * q + 1], acc[i * 2 + 1][2 * q + 1]};
        }
        return;
    }
    // Output tiles go through LDS so that every global access instruction covers whole row
    // segments (a lane's own fragment is 32 columns of one token row; accessed directly, each
    // instruction would touch 16-byte pieces of 32 rows). Staging area: this wave's own weight ring
    // (its loads have all landed; LDS operations of one wave complete in order, so no barrier).
    // A 32-row tile of 64 columns has rows 64 * esize + 16 bytes apart.
    uint8_t* stage = wring;
    constexpr int kRow16 = 64 * 2 + 16, kRow32 = 64 * 4 + 16;
    // 32 rows of 64 columns (kw0 .. kw0 + 63) between LDS tile `t` (fp16) and global memory
    auto tile_io = [&](bool to_global, int t, _Float16* gp, int64_t ld, int m_first) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = q * 64 + lane, row = c >> 3, cc = c & 7;
            uint8_t* lp = stage + t * 32 * kRow16 + row * kRow16 + cc * 16;
            const int m = m_first + row, col = kw0 + 8 * cc;
            const bool ok = m < M && col < K;  // k % 32 == 0: chunks are wholly in or out
            if (to_global) {
                if (ok) *(u32x4_t*)(gp + (int64_t)m * ld + col) = *(const u32x4_t*)lp;
            } else {
                *(u32x4_t*)lp = ok ? *(const u32x4_t*)(gp + (int64_t)m * ld + col) : u32x4_t{0u, 0u, 0u, 0u};
            }
        }
    };
    // this lane's 32 columns (32 g .. 32 g + 31 of the tile) of token row l32, fp16 pairs
    auto frag_put = [&](int t, const uint32_t* o) __attribute__((always_inline)) {
        uint8_t* lp = stage + t * 32 * kRow16 + l32 * kRow16 + 64 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) *(u32x4_t*)(lp + 16 * q) = u32x4_t{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
    };
    auto frag_get = [&](int t, uint32_t* o) __attribute__((always_inline)) {
        const uint8_t* lp = stage + t * 32 * kRow16 + l32 * kRow16 + 64 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4_t v = *(const u32x4_t*)(lp + 16 * q);
            o[4 * q] = v[0];
            o[4 * q + 1] = v[1];
            o[4 * q + 2] = v[2];
            o[4 * q + 3] = v[3];
        }
    };
    // column kc + 2 p + cb of this lane is acc[i * 2 + cb][p]; fp16 pair j = columns 2 j, 2 j + 1
    auto pack_row = [&](int i, uint32_t* o) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) o[j] = pack_half2(acc[i * 2][j], acc[i * 2 + 1][j]);
    };
    if (a.swiglu) {
        // G = fp16(dY.W) (the rounding of the matmul output), then dgate / dup of SwiGLU from the
        // lane's 32 columns of gate and up (the tiles are read before any output is written: the
        // outputs may alias gate and up)
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int mf = m0 + 32 * i;
            tile_io(false, 0, const_cast<_Float16*>(a.gate), a.ldgu, mf);
            tile_io(false, 1, const_cast<_Float16*>(a.up), a.ldgu, mf);
            uint32_t gw[16], uw[16], Gw[16], dg[16], du[16];
            frag_get(0, gw);
            frag_get(1, uw);
            pack_row(i, Gw);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const half2_t G2 = __builtin_bit_cast(half2_t, Gw[j]);
                const half2_t g2 = __builtin_bit_cast(half2_t, gw[j]), u2 = __builtin_bit_cast(half2_t, uw[j]);
                float d0, d1, e0, e1;
                swiglu_bwd1((float)G2.x, (float)g2.x, (float)u2.x, d0, e0);
                swiglu_bwd1((float)G2.y, (float)g2.y, (float)u2.y, d1, e1);
                dg[j] = pack_half2(d0, d1);
                du[j] = pack_half2(e0, e1);
            }
            frag_put(0, dg);
            frag_put(1, du);
            tile_io(true, 0, a.dgate, a.ldd, mf);
            tile_io(true, 1, a.dup, a.ldd, mf);
        }
        return;
    }
    if (a.dx_fp32) {
        // fp32: each lane's 32 columns straight from the accumulators (128 bytes per row and lane)
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int m = m0 + 32 * i + l32;
            if (m >= M || kc >= K) continue;
            float* dst = (float*)a.dx + (int64_t)m * a.lddx + kc;
#pragma unroll
            for (int q = 0; q < 8; ++q)
                *(float4_t*)(dst + 4 * q) = float4_t{acc[i * 2][2 * q], acc[i * 2 + 1][2 * q],
                                                     acc[i * 2][2 * q + 1], acc[i * 2 + 1][2 * q + 1]};
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        uint32_t o[16];
        pack_row(i, o);
        frag_put(0, o);
        tile_io(true, 0, (_Float16*)a.dx, a.lddx, m0 + 32 * i);
    }
    (void)kRow32;
}

template <int MB, int WAVES, bool NESTED>
static hipError_t launch_bwd_t(const BwdArgs& a, int grid, hipStream_t s) {
    const size_t sm = bwd_smem_bytes(MB, WAVES);
    const hipError_t e = allow_dynamic_lds((const void*)nf4_bwd_kernel<MB, WAVES, NESTED>, sm);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((nf4_bwd_kernel<MB, WAVES, NESTED>), dim3(grid), dim3(64 * WAVES), sm, s, a);
    return hipGetLastError();
}

// variant: (token row blocks, waves) -- see kBwdVariants in capi.hip
hipError_t launch_bwd(const BwdArgs& a, int mb, int waves, int grid, hipStream_t s) {
#define X(T, W)                                                                                  \
    if (mb == T && waves == W)                                                                   \
        return a.nested ? launch_bwd_t<T, W, true>(a, grid, s) : launch_bwd_t<T, W, false>(a, grid, s);
    X(2, 4) X(2, 8) X(4, 8)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
