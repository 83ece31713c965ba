// Fused NF4 dequant x fp16 GEMM, input gradient: the same product as nf4_bwd_kernel
// (dX = sum_g dY_g . W_g + sum_g GU_g . A_g, solution/nf4.py:99-104, summed over several weights
// as the gate and up projections of solution/mlp.py:106-109), including the SwiGLU epilogue of
// dk_nf4_linear_bwd_swiglu (solution/mlp.py:97-105: dgate / dup from fp16(dY . W_down)).
//
// Why a second kernel: nf4_bwd_kernel's waves own 64 output columns (two A operands, both
// nibbles of a byte per lane) and at most 4 token blocks, so each dequantized weight feeds at
// most four MFMAs and the dequant costs far more issue slots than the matrix pipe leaves free.
// Here a work-group is 8 waves (two per SIMD, one work-group per CU) on a tile of 32*MB tokens
// (MB = 4, 7 or 8) x 256 output columns; each wave owns 32 columns -- one A operand, one nibble
// per lane and weight row -- and all 32*MB tokens, so each dequantized weight feeds MB MFMAs.
// MB = 2 (64 tokens) serves launches with few token rows, which on 128-token tiles would spend
// half their MFMAs on padding (7B gate/up input gradient at 64 tokens: 45 -> 40 us).
//
// A operand (A = W^T): lane l (l32 = l % 32, g = l / 32) serves A row l32 = output column
// c = l32 ^ 1 of the wave's 32. Its eight contraction slots of slice j are the weight rows
// 32 g + 8 j + e of the 64-row step; dY's B operand uses the same order.
//
// Per wave and step: the wave's 16 packed bytes of each of the 64 rows (one 16-byte DMA load per
// lane, stored as rows of 16 bytes) and one block statistic per row (32 aligned columns of a row
// always lie in one block: k % 32 == 0 and blocks are powers of two >= 32). The weights reach the
// MFMA layout through the LDS transpose read ds_read_b64_tr_b4: in each group of 16 lanes, lane r
// reads 8 bytes (16 columns) of row 32 g + 8 j + r and lane i gets back nibble i of the 16 rows,
// i.e. column i ^ 1 (bitsandbytes keeps the first of two columns in the high nibble) for slices j
// and j + 1, one nibble per row in row order. A byte of that dword holds two rows of the lane's
// column, so one byte-pair code-book entry (one 8-byte LDS read, its address one SDWA shift)
// gives both codes; each is scaled by its own row's scale. The dY tile (32*MB x 64 fp16) is
// shared by the work-group through a ring three steps deep, as in nf4_bwd_kernel. Row scales of
// step t + 1 are computed during slice 2 of step t, one row per lane, and read back through a
// per-wave LDS table. The loop is software-pipelined one slice ahead, as in the forward kernels:
// stage A (transposed read every other slice, row scales of the next slice) after the slice's
// first MFMA, stage B (code-book addresses and reads) after the third, stage C (scaling and fp16
// packing) after the last but one, and each dY fragment refilled right after its MFMA read it.
//
// Epilogue: each token block's 32 x 256 tile goes through LDS (the rings, after a barrier) and
// leaves as whole rows: split-K partial slabs (reduced by splitk_reduce_kernel), dX in fp32 or
// fp16, or (SwiGLU mode, MB <= 4) dgate / dup from the tile rounded to fp16 and the matching gate
// and up tiles, which every thread fetches for all its token blocks as the kernel starts.
#include "gemm_common.h"

namespace dk {

// LDS transpose read (gfx950 ds_read_b64_tr_b4): the 16 lanes of each lane group read 8 bytes each
// (row r = lane r's 16 nibbles, low nibble first); lane i of the group receives nibble i of rows
// 0..15, in order (row e at bits 4 e of the 64-bit result).
__device__ __forceinline__ u32x2_t lds_tr4(const uint8_t* p) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i r = __builtin_amdgcn_ds_read_tr4_b64_v2i32((__attribute__((address_space(3))) v2i*)p);
    return u32x2_t{(uint32_t)r[0], (uint32_t)r[1]};
}

constexpr int kB8Waves = 8;
constexpr int kB8Threads = 64 * kB8Waves;
constexpr int kB8BN = 32 * kB8Waves;          // output columns per tile
constexpr int kB8Tables = kMaxGroups * 1024;  // code2 tables (nested statistics), 1 KB per group
constexpr int kB8Dummy = 1024;                // target of the dY loads of waves past the tile
// Per-wave ring slot of one step: 1 KB packed bytes (64 rows of 16 bytes), then one
// statistics dword slot per row (codes or fp32 absmax at +1024, absmax2 at +1280).
constexpr int kB8WSlot = 1536;
constexpr int kB8ScaleBytes = 2 * 64 * 4;  // per wave: row-scale tables of two steps

// Epilogue staging: two 32-token blocks of fp32 tiles (rows 1040 bytes apart), in the dY ring
// and the weight rings and scale tables behind it; the dY ring region is sized so that it fits.
constexpr int kB8Stage = 2 * 32 * (kB8BN * 4 + 16);
__host__ __device__ constexpr int bwd8_dring_bytes(int mb) {
    return 3 * 32 * mb * 128 + kB8Waves * (3 * kB8WSlot + kB8ScaleBytes) >= kB8Stage
               ? 3 * 32 * mb * 128
               : kB8Stage - kB8Waves * (3 * kB8WSlot + kB8ScaleBytes);
}

__host__ __device__ constexpr size_t bwd8_smem_bytes(int mb) {
    return kB8Tables + kB8Dummy + (size_t)bwd8_dring_bytes(mb) +
           kB8Waves * (3 * (size_t)kB8WSlot + kB8ScaleBytes);
}

template <int MB, bool NESTED>
__global__ __launch_bounds__(kB8Threads, 1) void nf4_bwd8_kernel(const BwdArgs a) {
    constexpr int BM = 32 * MB;
    constexpr int DBUF = BM * 128;                             // bytes of one dY ring buffer
    constexpr int DCH = BM * 8;                                // its 16-byte chunks
    constexpr int DPT = (DCH + kB8Threads - 1) / kB8Threads;   // dY loads per thread and step
    constexpr int NL = DPT + 1 + (NESTED ? 2 : 1);             // loads per thread and step
    static_assert(DCH % 64 == 0, "a wave's dY load is wholly inside or past the tile");
    // epilogue staging area: the dY ring, the weight rings and the scale tables (contiguous)
    constexpr int DRING = bwd8_dring_bytes(MB);                // bytes of the dY ring region
    constexpr int STAGE = DRING + kB8Waves * (3 * kB8WSlot + kB8ScaleBytes);
    static_assert(2 * 32 * (kB8BN * 4 + 16) <= STAGE, "epilogue staging fits the rings");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // byte-pair code book of the current group: entry x = (code[x & 15], code[x >> 4]), the
    // weights of the two rows whose nibbles share byte x of a transposed dword
    __shared__ float2_t lutT[256];
    uint8_t* dummy = smem + kB8Tables;
    uint8_t* dring = dummy + kB8Dummy;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
    const int l32 = lane & 31, g = lane >> 5;
    const int c = l32 ^ 1;             // this lane's output column within the wave's 32
    const int xsw = (l32 >> 1) & 7;    // LDS swizzle of this lane's dY rows

    const int L = xcd_logical_id();
    if (L >= a.m_tiles * a.k_tiles * a.splits) return;
    // consecutive logical ids share an XCD's L2: token tiles fastest share the weight columns,
    // column tiles fastest share the dY rows (chosen by the host for large token counts)
    const int mk = L % (a.m_tiles * a.k_tiles);
    const int split = L / (a.m_tiles * a.k_tiles);
    const int m_tile = a.cols_first ? mk / a.k_tiles : mk % a.m_tiles;
    const int k_tile = a.cols_first ? mk % a.k_tiles : mk / a.m_tiles;
    const int M = sgpr(a.m), K = sgpr(a.k);
    const int m0 = m_tile * BM;
    const int tile_k0 = (a.k_tile0 + k_tile) * kB8BN;
    const int kw0 = tile_k0 + 32 * wave;  // the wave's first output column
    const bool cok = kw0 < K;             // k % 32 == 0: the wave's columns are all in or all out
    const int cs0 = split * a.csteps_per_split;
    const int cs1 = min(a.csteps, cs0 + a.csteps_per_split);

    // nested statistics: this thread's entry of every group's code2 table, written to LDS with the
    // first group's code book, once that group's first loads are issued (one memory round trip
    // for both; buffer loads of uniform pointers, which indexed loads would fetch and wait for)
    float c2v[kMaxGroups] = {};
    if constexpr (NESTED) {
#pragma unroll
        for (int gg = 0; gg < kMaxGroups; ++gg)
            if (gg < a.ngroups && tid < 256) c2v[gg] = bloadf(make_rsrc(sgpr(a.g[gg].w.code2), 1024u), 4u * tid);
    }
    bool tables_written = false;
    uint8_t* wring = dring + DRING + wave * (3 * kB8WSlot);
    float* stab = (float*)(dring + DRING + kB8Waves * 3 * kB8WSlot + wave * kB8ScaleBytes);
    // this lane's transposed reads (slices j, j + 1 for even j): row 32 g + 8 j + (lane % 16) of
    // the step, bytes 8 (l32 / 16) .. of the wave's 16
    const int pkl = 16 * (32 * g + (lane & 15)) + 8 * ((lane >> 4) & 1);

    float16_t acc[MB];  // token block i
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = float16_t{};

    // stage positions (MFMA index after which a stage runs). With few MFMAs per slice (P2) the
    // packed dwords and row scales are read two slices ahead (LA = 2), so the next step's row
    // scales are made in slice 1 (JW) instead of slice 2. With two MFMAs a slice (MB = 2) the
    // code-book reads follow stage A in the first gap and the scaling takes the second; the row
    // scales take both gaps of slice 1.
    constexpr bool P2 = MB <= 4;
    constexpr int LA = P2 ? 2 : 1, JW = P2 ? 1 : 2;
    constexpr int qB = MB >= 7 ? 2 : (MB >= 4 ? 1 : 0), qC = MB >= 7 ? MB - 2 : MB - 1;
    // next step's row scales
    constexpr int qS1 = MB >= 4 ? 1 : 0, qS2 = MB >= 7 ? 3 : (MB >= 4 ? 2 : 1), qS3 = MB >= 7 ? 5 : (MB >= 4 ? 3 : 1);
    static_assert(qS3 < MB && qB < qC, "stages inside the slice");
    static_assert(MB <= 4 || DPT + 1 < MB, "a step's load parts fit one slice's MFMA gaps");

    // SwiGLU mode: this thread's two 16-byte chunks (row ch / 32, columns 8 (ch % 32) ..) of
    // every token block's gate and up tiles, requested as the kernel starts so that their reads
    // overlap the main loop (the tiles are read before any output is written: dgate / dup may
    // alias gate / up). The main loop's waits count its own loads only; these are older, so they
    // only make the first wait stricter.
    constexpr int SWB = MB <= 4 ? MB : 1;
    u32x4_t gv[SWB][2], uv[SWB][2];
    if constexpr (MB <= 4) {
        if (a.swiglu) {
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int ch = tid + kB8Threads * h, row = ch >> 5, cc = ch & 31;
                    const int m = m0 + 32 * i + row, col = tile_k0 + 8 * cc;
                    gv[i][h] = uv[i][h] = u32x4_t{0u, 0u, 0u, 0u};
                    if (m < M && col < K) {
                        gv[i][h] = *(const u32x4_t*)(a.gate + (int64_t)m * a.ldgu + col);
                        uv[i][h] = *(const u32x4_t*)(a.up + (int64_t)m * a.ldgu + col);
                    }
                }
        }
    }

    // LoRA input-gradient terms GU_g . A_g first (split 0 only; trip count 0 without LoRA): A row
    // l32 (output column kw0 + c) of rank slots t0 + 8 g + e, B = GU^T.
    {
        const int R = split == 0 ? sgpr(a.lora_rank) : 0;
        for (int gg = 0; gg < a.ngroups; ++gg) {
            const BwdGroupDev& G = a.g[gg];
            if (G.lora_gu == nullptr || G.lora_keep != nullptr || R == 0) continue;  // dropout: epilogue
            const rsrc_t ars = make_rsrc(G.lora_a, (uint32_t)R * (uint32_t)K * 2u);
            const rsrc_t grs = make_rsrc(G.lora_gu, (uint32_t)M * (uint32_t)R * 2u);
            for (int t0 = 0; t0 < R; t0 += 16) {
                half8_t al;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    al[e] = __builtin_bit_cast(
                        _Float16, (uint16_t)bload16(ars, off_if(cok, (uint32_t)((t0 + 8 * g + e) * K + kw0 + c) * 2u)));
#pragma unroll
                for (int i = 0; i < MB; ++i) {
                    const int m = m0 + 32 * i + l32;
                    const half8_t gu = __builtin_bit_cast(
                        half8_t, bload128(grs, off_if(m < M, (uint32_t)(m * R + t0 + 8 * g) * 2u)));
                    acc[i] = mfma32x32x16(al, gu, acc[i]);
                }
            }
        }
    }

    // One weight group at a time, as in nf4_bwd_kernel: the group's operands are pinned in
    // scalar registers for its steps and the pipeline drains between groups.
    for (int gi = 0; gi < a.ngroups; ++gi) {
        const BwdGroupDev& G = a.g[gi];
        const int sb = sgpr(G.step_begin);
        const int t0 = max(cs0, sb), t1 = min(cs1, sb + sgpr(G.nsteps));
        if (t0 >= t1) continue;
        const int N = sgpr((int)G.w.n);
        const int lddy = sgpr(G.lddy);
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
        const float* c2 = (const float*)smem + 256 * gi;
        // this group's code book: loaded here, written to LDS once the group's first steps are in
        // flight (the previous group's readers are past the barrier that ended its loop; this
        // group's prologue barrier publishes the new book)
        const rsrc_t bkr = make_rsrc(sgpr(G.w.code), 64u);
        const float book_lo = bloadf(bkr, 4u * (tid & 15)), book_hi = bloadf(bkr, 4u * ((tid >> 4) & 15));

        // Loads use per-lane offsets fixed for the group (bit 31 set where the lane's data lies
        // outside the tile or the weight: it reads zeros) against buffer descriptors whose base
        // advances by whole steps. Only a group's last step, when its row count is not a
        // multiple of 64, also checks rows and dY columns per lane. A step past the segment's
        // end loads from descriptors of size 0 (zeros), keeping the load count uniform.
        // dY chunk h of this thread: token row (tid + 512 h) / 8 of the tile, 16-byte column
        // dy_col(h) of the step (the LDS swizzle applied to the thread's position in the row)
        auto dy_col = [&](int h) __attribute__((always_inline)) -> int {
            const int q = tid + kB8Threads * h;
            return (q & 7) ^ ((q >> 4) & 7);
        };
        uint32_t dyo[DPT];
#pragma unroll
        for (int h = 0; h < DPT; ++h) {
            const int q = tid + kB8Threads * h;
            const int gm = m0 + (q >> 3);
            dyo[h] = off_if(q < DCH && gm < M, (uint32_t)(gm * lddy + 8 * dy_col(h)) * 2u);
        }
        // the LDS destination of a wave's dY load h within ring buffer rd (waves past the tile:
        // the dummy area)
        auto dy_dst = [&](int rd, int h) __attribute__((always_inline)) -> uint8_t* {
            const int wq0 = kB8Threads * h + 64 * wave;  // the wave's first chunk (uniform)
            // loads h < DPT - 1 never pass the tile (folded at compile time: no scalar select)
            return ((h + 1) * kB8Threads <= DCH || wq0 < DCH) ? dring + rd + wq0 * 16 : dummy;
        };
        // packed bytes: lane l fetches the wave's 16 bytes of row l of the step, landing at
        // byte 16 l of the slot (rows of 16 bytes, the layout the transposed reads take)
        const uint32_t po = off_if(cok, (uint32_t)lane * (uint32_t)(K >> 1) + (uint32_t)(kw0 >> 1));
        // statistics: lane = weight row of the step
        const uint32_t blk0 = ((uint32_t)lane * (uint32_t)K + (uint32_t)kw0) >> bs_shift;
        const uint32_t so = off_if(cok, NESTED ? blk0 : blk0 * 4u);

        // Part p of load_step (p < DPT: dY chunk p; DPT: the packed weights; DPT + 1: their
        // statistics), so that the main loop issues a step's loads one per MFMA gap: issued in one
        // burst after the barrier they held up the matrix pipe (7.7% of the 7B q/o input gradient
        // at M = 8192).
        auto load_part = [&](int p, int t, int rd, int rw, bool live) __attribute__((always_inline)) {
            const int n0 = (t - sb) * kBwdBC;
            const bool tail = n0 + kBwdBC > N;  // uniform
            if (p < DPT) {
                const rsrc_t drs = make_rsrc(gdy + n0, live ? dy_bytes - 2u * (uint32_t)n0 : 0u);
                if (!tail) {
                    bload128_lds(drs, dy_dst(rd, p), dyo[p]);
                } else {
                    // rows and dY columns past N read zeros. The empty volatile asm keeps this a
                    // branch taken only on a group's last, partial step: merged with the plain
                    // loads, the per-lane checks became selects on every step (~8% of the loop).
                    asm volatile("");
                    bload128_lds(drs, dy_dst(rd, p), off_if(n0 + 8 * dy_col(p) < N, dyo[p]));
                }
                return;
            }
            uint8_t* slot = wring + rw;
            if (p == DPT) {
                const uint32_t pskip = (uint32_t)n0 * (uint32_t)(K >> 1);
                const rsrc_t wrs = make_rsrc(gpk + pskip, live ? pk_bytes - pskip : 0u);
                if (!tail) {
                    bload128_lds(wrs, slot, po);
                } else {
                    asm volatile("");
                    bload128_lds(wrs, slot, off_if(n0 + lane < N, po));
                }
                return;
            }
            const uint32_t kb = ((uint32_t)n0 * (uint32_t)K) >> bs_shift;  // blocks before this step
            const bool rok = !tail || n0 + lane < N;
            if constexpr (NESTED) {
                const rsrc_t ars = make_rsrc(gam8 + kb, live ? am_bytes - kb : 0u);
                const rsrc_t a2rs = make_rsrc(gam2, live ? am2_bytes : 0u);
                bload8_lds(ars, slot + 1024, off_if(rok, so));
                bload32_lds(a2rs, slot + 1280, off_if(rok && cok, ((blk0 + kb) >> bs2_shift) * 4u));
            } else {
                const rsrc_t ars = make_rsrc(gamf + kb, live ? am_bytes - 4u * kb : 0u);
                bload32_lds(ars, slot + 1024, off_if(rok, so));
            }
        };
        // every load of step t (the prologue)
        auto load_step = [&](int t, int rd, int rw, bool live) __attribute__((always_inline)) {
#pragma unroll
            for (int p = 0; p < DPT + 2; ++p) load_part(p, t, rd, rw, live);
        };

        // Row scale of step t (lane = row) from this wave's statistics in slot rw, into table
        // sidx, in three parts spread over slice 2's MFMAs (the loads were this wave's own, so its
        // own wait suffices: no barrier).
        uint32_t sq = 0;
        float sa = 0.0f;
        auto scales_1 = [&](int rw) __attribute__((always_inline)) {
            const uint8_t* slot = wring + rw;
            if constexpr (NESTED) {
                sq = slot[1024 + 4 * lane];
                sa = *(const float*)(slot + 1280 + 4 * lane);
            } else {
                sa = *(const float*)(slot + 1024 + 4 * lane);
            }
        };
        auto scales_2 = [&]() __attribute__((always_inline)) {
            if constexpr (NESTED) sa = c2[sq] * sa;
        };
        auto scales_3 = [&](int t, int sidx) __attribute__((always_inline)) {
            const int row = (t - sb) * kBwdBC + lane;
            const float sc = NESTED ? sa + offset : sa;
            stab[64 * sidx + lane] = (row < N && cok) ? sc : 0.0f;
        };

        // Ring buffers: step t uses dY buffer rd0 (byte offset in the dY ring), weight slot rw0
        // and scale table si0; step t + 1 uses rd1 / rw1 / 1 - si0; step t + 3 reuses step t's.
        int rd0 = 0, rw0 = 0, rd1 = DBUF, rw1 = kB8WSlot, si0 = 0;
        // Prologue: three steps in flight; wait for the first.
        load_step(t0, 0, 0, true);
        load_step(t0 + 1, DBUF, kB8WSlot, t0 + 1 < t1);
        load_step(t0 + 2, 2 * DBUF, 2 * kB8WSlot, t0 + 2 < t1);
        if (tid < 256) lutT[tid] = float2_t{book_lo, book_hi};
        if constexpr (NESTED) {
            if (!tables_written) {
#pragma unroll
                for (int gg = 0; gg < kMaxGroups; ++gg)
                    if (gg < a.ngroups && tid < 256) ((float*)smem)[256 * gg + tid] = c2v[gg];
                tables_written = true;
            }
        }
        wait_vmcnt<2 * NL>();
        lds_barrier();  // dY(t0) from every wave, code tables
        scales_1(0);
        scales_2();
        scales_3(t0, 0);

        half8_t xf[MB], w, wn;
        u32x2_t tr;      // the last transposed read: this lane's nibbles of two slices
        uint32_t d0;     // next slice: this lane's nibbles of its 8 rows (row e at bits 4 e)
        float4_t s0, s1; // ... their row scales
        float v[8];      // ... their code-book values
        uint32_t e0;     // two-slice pipeline: the nibbles and scales of the slice after
        float4_t t0s, t1s;
        auto stage_A = [&](int rw, int sidx, int j) __attribute__((always_inline)) {
            if ((j & 1) == 0) tr = lds_tr4(wring + rw + pkl + 128 * j);
            const uint32_t dj = (j & 1) ? tr[1] : tr[0];
            const float* sc = stab + 64 * sidx + 32 * g + 8 * j;
            if constexpr (P2) {
                e0 = dj;
                t0s = *(const float4_t*)sc;
                t1s = *(const float4_t*)(sc + 4);
            } else {
                d0 = dj;
                s0 = *(const float4_t*)sc;
                s1 = *(const float4_t*)(sc + 4);
            }
        };
        // two-slice pipeline: the slice after next becomes the next one
        auto advance = [&]() __attribute__((always_inline)) {
            if constexpr (P2) {
                d0 = e0;
                s0 = t0s;
                s1 = t1s;
            }
        };
        auto stage_B = [&]() __attribute__((always_inline)) {
            // byte b of d0 holds rows 2 b (low nibble) and 2 b + 1: one code-book pair each
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float2_t cv = *(const float2_t*)((const char*)lutT + byte_x8(d0, b));
                v[2 * b] = cv.x;
                v[2 * b + 1] = cv.y;
            }
        };
        auto stage_C = [&]() __attribute__((always_inline)) -> half8_t {
            u32x4_t o;
            o[0] = pack_half2(v[0] * s0[0], v[1] * s0[1]);
            o[1] = pack_half2(v[2] * s0[2], v[3] * s0[3]);
            o[2] = pack_half2(v[4] * s1[0], v[5] * s1[1]);
            o[3] = pack_half2(v[6] * s1[2], v[7] * s1[3]);
            return __builtin_bit_cast(half8_t, o);
        };
        auto xfrag = [&](int rd, int i, int j) __attribute__((always_inline)) -> half8_t {
            return *(const half8_t*)(dring + rd + (32 * i + l32) * 128 + (((4 * g + j) ^ xsw) << 4));
        };

        // slice 0 of the first step (and, two slices deep, slice 1's packed dwords and scales)
        stage_A(rw0, si0, 0);
        advance();
#pragma unroll
        for (int i = 0; i < MB; ++i) xf[i] = xfrag(rd0, i, 0);
        stage_B();
        w = stage_C();
        if constexpr (P2) {
            stage_A(rw0, si0, 1);
            advance();
        }

        for (int t = t0; t < t1; ++t) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int jn = (j + 1) & 3;
#pragma unroll
                for (int q = 0; q < MB; ++q) {
                    acc[q] = mfma32x32x16(w, xf[q], acc[q]);
                    if (j == 3 && q == 0) {
                        // every wave's loads of step t+1 have landed (each waited in slice 1 or 2)
                        // and every wave is past step t's slots: refill them with step t+3
                        // (zeros past the segment's end), one part after each of this slice's
                        // MFMAs. Past the last step the reads below see stale slots and their
                        // values go unused.
                        lds_barrier();
                    }
                    if constexpr (MB > 4) {
                        if (j == 3 && q <= DPT + 1) load_part(q, t + 3, rd0, rw0, t + 3 < t1);
                    } else if (j == 3 && q == 0) {
                        // four MFMAs a slice leave no room to spread them (measured: the burst is
                        // 1.3% faster for the down-projection input gradient at MB = 4)
                        load_step(t + 3, rd0, rw0, t + 3 < t1);
                    }
                    // refill the dY fragment the MFMA above has read (slice j + 1)
                    xf[q] = xfrag(j < 3 ? rd0 : rd1, q, jn);
                    if (q == 0) {
                        // step t+1's loads (this wave's) landed; its row scales follow in this
                        // slice, before any stage A reads them
                        if (j == JW) wait_vmcnt<NL>();
                        const int ja = j + LA;  // the slice stage A prepares
                        if (ja < 4) stage_A(rw0, si0, ja);
                        else stage_A(rw1, 1 - si0, ja - 4);
                    }
                    if (j == JW) {
                        if (q == qS1) scales_1(rw1);
                        if (q == qS2) scales_2();
                        if (q == qS3) scales_3(t + 1, 1 - si0);
                    }
                    if (q == qB) stage_B();
                    if (q == qC) wn = stage_C();
                    __builtin_amdgcn_sched_barrier(0);
                }
                w = wn;
                advance();
            }
            // rotate the rings: step t + 1's buffers become the current ones
            rd0 = rd1;
            rw0 = rw1;
            rd1 = rd1 == 2 * DBUF ? 0 : rd1 + DBUF;
            rw1 = rw1 == 2 * kB8WSlot ? 0 : rw1 + kB8WSlot;
            si0 = 1 - si0;
        }
        // every load has landed and every wave is done with the rings before the next group's
        // prologue refills them
        wait_vmcnt<0>();
        lds_barrier();
    }
    lds_barrier();  // the rings become the staging area (also when no group had steps here)

    // ---- epilogue. Lane (l32, g) holds, for token block i, token row m0 + 32 i + l32 and, in
    // acc[i][4 a + b], column colw + 8 a + (b ^ 1) of the tile (D row 8 a + 4 g + b is A row, i.e.
    // output column, (8 a + 4 g + b) ^ 1): four runs of 4 columns, 8 apart, pairs swapped.
    const int colw = 32 * wave + 4 * g;
    // stage a lane's 16 values of one token block as fp16 / fp32 at their columns of an LDS row
    auto stage_half = [&](uint8_t* lp, const float16_t& v) __attribute__((always_inline)) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)
            *(u32x2_t*)(lp + 16 * a4) = u32x2_t{pack_half2(v[4 * a4 + 1], v[4 * a4]), pack_half2(v[4 * a4 + 3], v[4 * a4 + 2])};
    };
    auto stage_float = [&](uint8_t* lp, const float16_t& v) __attribute__((always_inline)) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)
            *(float4_t*)(lp + 32 * a4) = float4_t{v[4 * a4 + 1], v[4 * a4], v[4 * a4 + 3], v[4 * a4 + 2]};
    };
    if constexpr (MB <= 4) {
        if (a.swiglu) {
            // dgate / dup from G = fp16(dY . W) and the gate / up chunks fetched at the start
            constexpr int RB = kB8BN * 2 + 16;
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                // G = fp16(dY . W) through LDS as 32 x 256 fp16 rows
                uint8_t* buf = dring + (i & 1) * 32 * RB;
                uint8_t* lp = buf + l32 * RB + colw * 2;
                stage_half(lp, acc[i]);
                lds_barrier();
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int ch = tid + kB8Threads * h, row = ch >> 5, cc = ch & 31;
                    const u32x4_t Gv = *(const u32x4_t*)(buf + row * RB + cc * 16);
                    const int m = m0 + 32 * i + row, col = tile_k0 + 8 * cc;
                    u32x4_t dg, du;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        // elements copied to scalars first: hipcc compiles __builtin_bit_cast of
                        // a vector element (vec[q]) as element 0 whatever q is
                        const uint32_t Gq = Gv[q], gq = gv[i][h][q], uq = uv[i][h][q];
                        const half2_t G2 = __builtin_bit_cast(half2_t, Gq);
                        const half2_t g2 = __builtin_bit_cast(half2_t, gq);
                        const half2_t u2 = __builtin_bit_cast(half2_t, uq);
                        float d0, d1, e0, e1;
                        swiglu_bwd1((float)G2.x, (float)g2.x, (float)u2.x, d0, e0);
                        swiglu_bwd1((float)G2.y, (float)g2.y, (float)u2.y, d1, e1);
                        dg[q] = pack_half2(d0, d1);
                        du[q] = pack_half2(e0, e1);
                    }
                    if (m < M && col < K) {
                        *(u32x4_t*)(a.dgate + (int64_t)m * a.ldd + col) = dg;
                        *(u32x4_t*)(a.dup + (int64_t)m * a.ldd + col) = du;
                    }
                }
            }
            return;
        }
    }
    // LoRA input-gradient terms of branches whose input went through dropout (split 0): per token
    // block, P = GU_g . A_g on its own, rounded to fp16 (the branch's fp16 input gradient), times
    // keep and the keep scale in fp32, then added to the block's dX. Lane value r of token block i
    // is column kw0 + 16 g + r: bit r of the two keep bytes at column (kw0 + 16 g) / 8 of the row.
    if (split == 0) {
        const int R = sgpr(a.lora_rank);
        for (int gg = 0; gg < a.ngroups; ++gg) {
            const BwdGroupDev& G = a.g[gg];
            if (G.lora_keep == nullptr || G.lora_gu == nullptr || R == 0) continue;
            const rsrc_t ars = make_rsrc(G.lora_a, (uint32_t)R * (uint32_t)K * 2u);
            const rsrc_t grs = make_rsrc(G.lora_gu, (uint32_t)M * (uint32_t)R * 2u);
            const rsrc_t krs = make_rsrc(G.lora_keep, (uint32_t)M * (uint32_t)(K >> 3));
            const float ks = G.lora_keep_scale;
            half8_t al[2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    al[h][e] = __builtin_bit_cast(
                        _Float16, (uint16_t)bload16(ars, off_if(cok && 16 * h < R,
                                                                (uint32_t)((16 * h + 8 * g + e) * K + kw0 + c) * 2u)));
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int m = m0 + 32 * i + l32;
                float16_t p{};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8_t gu = __builtin_bit_cast(
                        half8_t, bload128(grs, off_if(m < M && 16 * h < R, (uint32_t)(m * R + 16 * h + 8 * g) * 2u)));
                    p = mfma32x32x16(al[h], gu, p);  // zeros past the rank
                }
                // the wave's 32 keep bits of the row (k % 32 == 0: 4-byte aligned)
                const uint32_t bits = __builtin_bit_cast(
                    uint32_t, bloadf(krs, off_if(m < M && cok, (uint32_t)m * (uint32_t)(K >> 3) + (uint32_t)(kw0 >> 3))));
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int col = 8 * (r >> 2) + 4 * g + ((r & 3) ^ 1);  // of the wave's 32
                    acc[i][r] = acc[i][r] + ((float)(_Float16)p[r] * (float)((bits >> col) & 1u)) * ks;
                }
            }
        }
    }
    const bool out32 = a.splits > 1 || a.dx_fp32;
    if (out32) {
        // 32 x 256 fp32 tiles (rows 1040 bytes apart) -> whole 1 KB rows of the split's partial
        // slab or of dX
        // (a slab holds the launch's pcols columns from column c0 = 256 k_tile0 on)
        float* dst = a.splits > 1 ? a.partials + (int64_t)split * M * a.pcols : (float*)a.dx;
        const int64_t ld = a.splits > 1 ? (int64_t)a.pcols : a.lddx;
        const int c0 = a.splits > 1 ? a.k_tile0 * kB8BN : 0;
        constexpr int RB = kB8BN * 4 + 16;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            uint8_t* buf = dring + (i & 1) * 32 * RB;
            uint8_t* lp = buf + l32 * RB + colw * 4;
            stage_float(lp, acc[i]);
            lds_barrier();
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int ch = tid + kB8Threads * h, row = ch >> 6, cc = ch & 63;
                const float4_t val = *(const float4_t*)(buf + row * RB + cc * 16);
                const int m = m0 + 32 * i + row, col = tile_k0 + 4 * cc;
                if (m < M && col < K) *(float4_t*)(dst + (int64_t)m * ld + (col - c0)) = val;
            }
        }
        return;
    }
    {
        // 32 x 256 fp16 tiles (rows 528 bytes apart) -> whole 512-byte rows of dX
        _Float16* dst = (_Float16*)a.dx;
        constexpr int RB = kB8BN * 2 + 16;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            uint8_t* buf = dring + (i & 1) * 32 * RB;
            uint8_t* lp = buf + l32 * RB + colw * 2;
            stage_half(lp, acc[i]);
            lds_barrier();
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int ch = tid + kB8Threads * h, row = ch >> 5, cc = ch & 31;
                const u32x4_t val = *(const u32x4_t*)(buf + row * RB + cc * 16);
                const int m = m0 + 32 * i + row, col = tile_k0 + 8 * cc;
                if (m < M && col < K) *(u32x4_t*)(dst + (int64_t)m * a.lddx + col) = val;
            }
        }
    }
}

template <int MB, bool NESTED>
static hipError_t launch_bwd8_t(const BwdArgs& a, int grid, hipStream_t s) {
    const hipError_t e = allow_dynamic_lds((const void*)nf4_bwd8_kernel<MB, NESTED>, bwd8_smem_bytes(MB));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((nf4_bwd8_kernel<MB, NESTED>), dim3(grid), dim3(kB8Threads),
                       bwd8_smem_bytes(MB), s, a);
    return hipGetLastError();
}

hipError_t launch_bwd8(const BwdArgs& a, int mb, int grid, hipStream_t s) {
    if (a.swiglu && (mb > 4 || a.splits > 1)) return hipErrorInvalidValue;  // SwiGLU: MB <= 4, no split
#define X(T) \
    if (mb == T) return a.nested ? launch_bwd8_t<T, true>(a, grid, s) : launch_bwd8_t<T, false>(a, grid, s);
    X(2) X(4) X(7) X(8)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
