// Fused NF4 dequant x fp16 GEMM, forward (replaces dequantize_nf4 + F.linear,
// solution/nf4.py:93-96; the LoRA term of solution/attn.py:225-228 rides in the epilogue):
//
//     Y[m, n] = sum_k X[m, k] W[n, k] + bias[n] + sum_t U[m, t] fp16(s * B[n, t])
//
// MFMA v_mfma_f32_32x32x16_f16 with fp32 accumulation. The dequantized weight is the A operand
// (32 weight rows per block), X the B operand (32 token rows per block), so D = W.X^T = Y^T.
// Work-group = 4 waves; tile = 32*MB token rows x 256 weight rows, 64 weight rows per wave.
// Each wave unpacks its own weight rows' packed bytes in registers and feeds them straight to
// the MFMA: no fp16 weight is ever written anywhere.
//
// Occupancy: for MB <= 4 a work-group fits in 80 KB of LDS and 256 registers per lane, so two
// work-groups share a CU and each SIMD runs two waves. The SIMD then overlaps one wave's
// unpacking (VALU, code-book reads) with the other's MFMAs; the code below stays a plain
// in-order pipeline.
//
// Data movement: every global load goes straight into LDS rings (buffer_load ... lds), issued
// up to three steps (3 x 64 of k) ahead: the X tile (shared by the work-group) and, per wave,
// the packed weights and block statistics of its rows. Each step ends with one explicit wait
// for the next step's loads and one barrier; then the freed slots are refilled.
//
// Contraction order: an MFMA sums its 16 contraction slots in any order, so lane group
// g = lane / 32 takes k = 32 g + 8 j + e (j = MFMA index within the 64-wide step, e = 0..7):
// its 32 weights of a step are one contiguous 16-byte load. A rows follow arow_to_n, so each
// lane ends with 16 consecutive output columns of one token row (two 16-byte stores).

#include "gemm_common.h"

namespace dk {

constexpr int kFwdSmemHeader = 1024;  // code2 table; X ring follows (the code book is static LDS)

// Per-wave ring slot of one step: 2 x 1 KB packed bytes, then block statistics in dword slots
// (codes or fp32 absmax, then absmax2). Narrow layout (every blocksize >= 64 and k % 64 == 0,
// so a row's 64-wide step lies in one block): 64 slots each, slot l32 + 32 b holding row block
// b's statistics. Wide layout (otherwise): 128 slots each, slot lane + 64 b for the lane's own
// 32-wide k half (32-aligned in the flat index, so inside one block).
__host__ __device__ constexpr int fwd_wslot_bytes(bool wide) { return wide ? 3072 : 2560; }

__host__ __device__ constexpr size_t fwd_smem_bytes(int mb, bool wide) {
    return kFwdSmemHeader + 3 * (size_t)(32 * mb * 128) + 4 * 3 * (size_t)fwd_wslot_bytes(wide);
}

template <int MB, bool NESTED>
__global__ __launch_bounds__(kGemmThreads, MB <= 4 ? 2 : 1) void nf4_fwd_kernel(const FwdArgs a) {
    constexpr int BM = 32 * MB;
    constexpr int XBUF = BM * 128;             // bytes of one X ring buffer
    constexpr int NL = MB + 4;  // loads per step and thread (narrow layout)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // code books of row blocks 0 and 1 (the same book unless GLU); static, so their addresses
    // fold into the lookups
    __shared__ float lut[32];
    float* c2 = (float*)smem;
    uint8_t* xs = smem + kFwdSmemHeader;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
    const int l32 = lane & 31, g = lane >> 5;
    const bool wide = a.wide_stats != 0;
    const bool glu = a.glu != 0;  // (host: plain narrow statistics, two weights of one shape)
    const int wslot_bytes = fwd_wslot_bytes(wide);

    const int L = xcd_logical_id();
    if (L >= a.m_tiles * a.n_tiles * a.splits) return;
    const int m_tile = L % a.m_tiles;
    const int rest = L / a.m_tiles;
    const int n_tile = rest % a.n_tiles;
    const int split = rest / a.n_tiles;

    int gi = 0;  // the weight this tile's columns belong to (wave-uniform)
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && n_tile >= a.g[i].tile_begin) gi = i;
    gi = __builtin_amdgcn_readfirstlane(glu ? 0 : gi);
    const FwdGroupDev& G = a.g[gi];                 // row block 0's weight (and block 1's ...
    const FwdGroupDev& G1 = a.g[glu ? 1 : gi];      // ... unless GLU: block 1 is the up weight)
    const NF4Dev& W = G.w;
    const NF4Dev& W1 = G1.w;
    // Scalars the main loop uses, pinned in SGPRs: left to itself the compiler re-reads them
    // from the kernel arguments inside the loop, and every such scalar load waits for all
    // outstanding LDS reads (they share the lgkm counter).
    const int M = sgpr(a.m), K = sgpr(a.k), N = sgpr((int)W.n), ldx = sgpr((int)a.ldx);
    const uint32_t bs_shift = sgpr((uint32_t)W.bs_shift), bs2_shift = sgpr((uint32_t)W.bs2_shift);
    const int m0 = m_tile * BM;
    // first weight row of the wave: 64 rows (blocks 0, 1) or, GLU, 32 rows of each weight
    const int nw0 = glu ? n_tile * (kFwdBN / 2) + wave * 32 : (n_tile - G.tile_begin) * kFwdBN + wave * 64;
    const int ks0 = split * a.ksteps_per_split;
    const int ks1 = min(a.ksteps, ks0 + a.ksteps_per_split);

    if (tid < 32) lut[tid] = (tid < 16 ? W.code : W1.code)[tid & 15];
    if constexpr (NESTED) c2[tid] = W.code2[tid];
    const float offset = NESTED ? *W.offset : 0.0f;

    const rsrc_t xrs = make_rsrc(a.x, a.x_bytes);
    const rsrc_t wrs = make_rsrc(W.packed, W.packed_bytes);
    const rsrc_t wrs1 = make_rsrc(W1.packed, W1.packed_bytes);
    const rsrc_t ars = make_rsrc(NESTED ? (const void*)W.absmax8 : (const void*)W.absmaxf, W.absmax_bytes);
    const rsrc_t ars1 = make_rsrc(W1.absmaxf, NESTED ? 0u : W1.absmax_bytes);  // GLU (plain) only
    const rsrc_t a2rs = make_rsrc(W.absmax2, W.absmax2_bytes);
    const int wrow0 = nw0 + arow_to_n(l32);   // this lane's A row in block 0 ...
    const int wrow1 = glu ? wrow0 : wrow0 + 32;  // ... and in block 1
    const int xsw = (l32 >> 1) & 7;           // LDS swizzle of this lane's X rows

    uint8_t* wring = xs + 3 * XBUF + wave * (3 * wslot_bytes);
    auto ring = [&](int t) __attribute__((always_inline)) { return (t - ks0) % 3; };
    auto xbuf = [&](int t) -> uint8_t* { return xs + ring(t) * XBUF; };
    auto wslot = [&](int t) -> uint8_t* { return wring + ring(t) * wslot_bytes; };

    // Loads of step t: the X tile, then this wave's packed weights and statistics.
    // `live` false: every load reads zeros (a step past the split's end keeps the ring's load
    // count uniform without a branch).
    auto load_step = [&](int t, bool live) __attribute__((always_inline)) {
        const int k0 = t * kFwdBK;
        uint8_t* xd = xbuf(t);
#pragma unroll
        for (int h = 0; h < MB; ++h) {
            // wave-contiguous LDS destination: chunk q lands at q * 16 = row * 128 + pc * 16
            const int q = tid + kGemmThreads * h;
            const int row = q >> 3, pc = q & 7;
            const int c = pc ^ ((row >> 1) & 7);  // the logical k chunk stored at this position
            const int gm = m0 + row, gk = k0 + 8 * c;
            bload128_lds(xrs, xd + (kGemmThreads * h + 64 * wave) * 16,
                         off_if(live && gm < M && gk < K, (uint32_t)(gm * ldx + gk) * 2u));
        }
        const int krun = k0 + 32 * g;
        uint8_t* slot = wslot(t);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int row = b ? wrow1 : wrow0;
            const bool ok = live && row < N && krun < K;
            bload128_lds(b ? wrs1 : wrs, slot + b * 1024,
                         off_if(ok, ((uint32_t)row * (uint32_t)K + (uint32_t)krun) >> 1));
        }
        if (!wide) {
            // lane (l32, g) fetches row block g's statistics (one block spans the 64-wide step);
            // GLU: lanes g = 0 those of the gate row, lanes g = 1 those of the up row (a second
            // load, into slot + 2304; all-zero without GLU)
            const int row = glu ? wrow0 : wrow0 + 32 * g;
            const bool ok = live && row < N && k0 < K;
            const uint32_t blk = ((uint32_t)row * (uint32_t)K + (uint32_t)k0) >> bs_shift;
            if constexpr (NESTED) {
                bload8_lds(ars, slot + 2048, off_if(ok, blk));
                bload32_lds(a2rs, slot + 2304, off_if(ok, (blk >> bs2_shift) * 4u));
            } else {
                bload32_lds(ars, slot + 2048, off_if(ok && (!glu || g == 0), blk * 4u));
                bload32_lds(ars1, slot + 2304, off_if(ok && glu && g == 1, blk * 4u));
            }
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int row = wrow0 + 32 * b;
                const bool ok = live && row < N && krun < K;
                const uint32_t blk = ((uint32_t)row * (uint32_t)K + (uint32_t)krun) >> bs_shift;
                if constexpr (NESTED) {
                    bload8_lds(ars, slot + 2048 + 256 * b, off_if(ok, blk));
                    bload32_lds(a2rs, slot + 2560 + 256 * b, off_if(ok, (blk >> bs2_shift) * 4u));
                } else {
                    bload32_lds(ars, slot + 2048 + 256 * b, off_if(ok, blk * 4u));
                }
            }
        }
    };
    const bool rowok0 = wrow0 < N, rowok1 = wrow1 < N;
    // fp32 scale of this lane's row block b at step t (0 outside the weight)
    auto scale_of = [&](const uint8_t* slot, int t, int b) __attribute__((always_inline)) -> float {
        const int si = wide ? lane + 64 * b : l32 + 32 * b;
        const int a2o = wide ? 2560 : 2304;
        const bool ok = (b ? rowok1 : rowok0) && t * kFwdBK + 32 * g < K;
        float sc;
        if constexpr (NESTED) {
            const uint32_t q = slot[2048 + 4 * si];
            const float a2 = *(const float*)(slot + a2o + 4 * si);
            sc = c2[q] * a2 + offset;
        } else {
            sc = *(const float*)(slot + 2048 + 4 * si + (b && glu ? 256 : 0));
        }
        return ok ? sc : 0.0f;
    };
    auto xfrag = [&](const uint8_t* xb, int i, int j) __attribute__((always_inline)) -> half8_t {
        return *(const half8_t*)(xb + (32 * i + l32) * 128 + (((4 * g + j) ^ xsw) << 4));
    };
    auto unpack8 = [&](uint32_t word, float s, int b) __attribute__((always_inline)) -> half8_t {
        uint32_t o[4];
        dequant4s(word, s, lut + 16 * b, o);
        return __builtin_bit_cast(half8_t, u32x4_t{o[0], o[1], o[2], o[3]});
    };

    float16_t acc[MB * 2];  // [token block i][weight block b] at i * 2 + b
#pragma unroll
    for (int t = 0; t < MB * 2; ++t) acc[t] = float16_t{};

    // LoRA term s * U.B^T first (split 0 only): rank/16 extra 16-wide contraction slices with
    // A = fp16(s * B) and B = U. Loads are branch-free (rows past the end read zeros) and the
    // trip count is 0 without LoRA.
    {
        const bool has = G.lora_u != nullptr || G1.lora_u != nullptr;
        const int R = (has && split == 0) ? sgpr(a.lora_rank) : 0;
        // a weight without LoRA gets zero-size buffers: its loads read zeros
        const rsrc_t brs0 = make_rsrc(G.lora_b, G.lora_u ? (uint32_t)N * (uint32_t)R * 2u : 0u);
        const rsrc_t urs0 = make_rsrc(G.lora_u, G.lora_u ? (uint32_t)M * (uint32_t)R * 2u : 0u);
        const rsrc_t brs1 = make_rsrc(G1.lora_b, G1.lora_u ? (uint32_t)N * (uint32_t)R * 2u : 0u);
        const rsrc_t urs1 = make_rsrc(G1.lora_u, G1.lora_u ? (uint32_t)M * (uint32_t)R * 2u : 0u);
        for (int t0 = 0; t0 < R; t0 += 16) {
            half8_t bl[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int row = b ? wrow1 : wrow0;
                const float ls = b ? G1.lora_scale : G.lora_scale;
                bl[b] = __builtin_bit_cast(half8_t, bload128(b ? brs1 : brs0, off_if(row < N, (uint32_t)(row * R + t0 + 8 * g) * 2u)));
#pragma unroll
                for (int e = 0; e < 8; ++e) bl[b][e] = (_Float16)((float)bl[b][e] * ls);
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int m = m0 + 32 * i + l32;
                const uint32_t uo = off_if(m < M, (uint32_t)(m * R + t0 + 8 * g) * 2u);
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const half8_t uu = __builtin_bit_cast(half8_t, bload128(b ? urs1 : urs0, uo));
                    acc[i * 2 + b] = mfma32x32x16(bl[b], uu, acc[i * 2 + b]);
                }
            }
        }
    }

    // Prologue: three steps in flight; wait for the first.
    load_step(ks0, true);
    load_step(ks0 + 1, ks0 + 1 < ks1);
    load_step(ks0 + 2, ks0 + 2 < ks1);
    wait_vmcnt<2 * NL>();
    lds_barrier();

    // Software pipeline over 16-wide k slices: while the 2*MB MFMAs of slice j run, the wave
    // prepares slice j + 1 in stages placed between them (sched_barrier keeps each stage next to
    // its MFMA): A = code-book addresses and X fragment reads, B = code-book reads (one per
    // weight), C = scale and fp16 packing. The LDS latency of A and B then hides under the matrix
    // core. Slice 3 holds the step boundary: after its first MFMA the wave fetches step t+1's
    // packed weights and scales from its own ring slot (its own loads, no barrier needed), and
    // the barrier before step t+1's X fragments sits between later MFMAs.
    u32x4_t p0, p1;  // packed weights of the current step (rows of block 0 and 1)
    float s0, s1;
    half8_t xf[MB], w0, w1;
    auto fetch_step = [&](int t) __attribute__((always_inline)) {
        const uint8_t* ws = wslot(t);
        p0 = *(const u32x4_t*)(ws + 16 * lane);
        p1 = *(const u32x4_t*)(ws + 1024 + 16 * lane);
        s0 = scale_of(ws, t, 0);
        s1 = scale_of(ws, t, 1);
    };
    fetch_step(ks0);
#pragma unroll
    for (int i = 0; i < MB; ++i) xf[i] = xfrag(xbuf(ks0), i, 0);
    w0 = unpack8(p0[0], s0, 0);
    w1 = unpack8(p1[0], s1, 1);

    constexpr int nm = 2 * MB;  // MFMAs per slice
    // stage positions: the MFMA index after which a stage is issued
    constexpr int qB0 = nm >= 8 ? 1 : 0;
    constexpr int qB1 = nm >= 8 ? 2 : (nm >= 4 ? 1 : 0);
    constexpr int qC0 = nm >= 8 ? nm / 2 + 1 : (nm >= 4 ? 2 : 1);
    constexpr int qC1 = qC0 + (nm >= 4 ? 1 : 0);
    // ... in slice 3: F = own-slot fetch, then A, B; the barrier, step t+3's loads and X reads
    constexpr int qA3 = nm >= 4 ? 1 : 0;
    constexpr int qB13 = nm >= 8 ? 2 : qA3;
    constexpr int qBar = nm >= 8 ? 3 : (nm >= 4 ? 2 : 0);

    uint32_t h0, l0, h1, l1;  // code-book byte addresses of the next slice (see nib_addrs)
    float v0[8], v1[8];       // its code-book values
    half8_t xn[MB], wn0, wn1;
    auto stage_A = [&](int jn) __attribute__((always_inline)) {
        nib_addrs(p0[jn], 0u, h0, l0);
        nib_addrs(p1[jn], 0u, h1, l1);
    };
    auto stage_X = [&](const uint8_t* xb, int jn) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MB; ++i) xn[i] = xfrag(xb, i, jn);
    };
    auto stage_B = [&](float* v, uint32_t h, uint32_t l, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = lut_at(lut + 16 * b, h, e);
            v[2 * e + 1] = lut_at(lut + 16 * b, l, e);
        }
    };
    auto stage_C = [&](const float* v, float sc) __attribute__((always_inline)) -> half8_t {
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = pack_half2(v[2 * e] * sc, v[2 * e + 1] * sc);
        return __builtin_bit_cast(half8_t, o);
    };
    auto mfma_q = [&](int q) __attribute__((always_inline)) {
        const int i = q >> 1;
        if (q & 1)
            acc[i * 2 + 1] = mfma32x32x16(w1, xf[i], acc[i * 2 + 1]);
        else
            acc[i * 2 + 0] = mfma32x32x16(w0, xf[i], acc[i * 2 + 0]);
    };

    for (int t = ks0; t < ks1; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int q = 0; q < nm; ++q) {
                mfma_q(q);
                if (j < 3) {
                    if (q == 0) {
                        stage_A(j + 1);
                        stage_X(xbuf(t), j + 1);
                    }
                    if (q == qB0) stage_B(v0, h0, l0, 0);
                    if (q == qB1) stage_B(v1, h1, l1, 1);
                } else {
                    if (q == 0) {
                        // step t+1's loads have landed (only step t+2's may be in flight)
                        wait_vmcnt<NL>();
                        fetch_step(t + 1);
                    }
                    if (q == qA3) {
                        stage_A(0);
                        stage_B(v0, h0, l0, 0);
                    }
                    if (q == qB13) stage_B(v1, h1, l1, 1);
                    if (q == qBar) {
                        // every wave is past step t's slots: refill them with step t+3 (zeros
                        // past the split's end). Past the last step the reads above and below
                        // see stale slots and their values go unused.
                        lds_barrier();
                        load_step(t + 3, t + 3 < ks1);
                        stage_X(xbuf(t + 1), 0);
                    }
                }
                if (q == qC0) wn0 = stage_C(v0, s0);
                if (q == qC1) wn1 = stage_C(v1, s1);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) xf[i] = xn[i];
            w0 = wn0;
            w1 = wn1;
        }
    }
    wait_vmcnt<0>();

    // ---- epilogue: bias, one fp16 rounding, stores (or, with split-K, the fp32 partial slab).
    // Both paths end in their own stores, so the accumulators never meet at a control-flow merge
    // (which makes the register allocator copy all of them).
    // Output tiles go through LDS so that every store instruction writes whole row segments
    // (a lane's own fragment is 16 columns of one token row; stored directly, each instruction
    // would scatter 16-byte pieces over 32 rows). The staging area is this wave's own weight ring
    // (its loads have all landed), so no barrier is needed: LDS operations of one wave complete
    // in order. A 32-row tile of `cols` columns has rows `cols * 2 + 16` bytes apart (no bank
    // conflicts on the fragment writes).
    uint8_t* stage = wring;
    auto stage_put = [&](int tile, int cols, int col0, const uint32_t* o) __attribute__((always_inline)) {
        uint8_t* p = stage + tile * 32 * (cols * 2 + 16) + l32 * (cols * 2 + 16) + col0 * 2;
        *(u32x4_t*)p = u32x4_t{o[0], o[1], o[2], o[3]};
        *(u32x4_t*)(p + 16) = u32x4_t{o[4], o[5], o[6], o[7]};
    };
    // rows m_first .. m_first + 31, columns n_first .. n_first + cols - 1 of out (row stride ld)
    auto stage_out = [&](int tile, int cols, _Float16* out, int64_t ld, int m_first, int n_first)
                         __attribute__((always_inline)) {
        const int cpr = cols / 8;  // 16-byte chunks per row
#pragma unroll
        for (int q = 0; q < cols / 16; ++q) {
            const int c = q * 64 + lane, row = c / cpr, cc = c % cpr;
            const u32x4_t v = *(const u32x4_t*)(stage + tile * 32 * (cols * 2 + 16) + row * (cols * 2 + 16) + cc * 16);
            const int m = m_first + row, n = n_first + 8 * cc;
            if (m < M && n < N)  // n % 8 == 0: a chunk is wholly inside or past the end
                *(u32x4_t*)(out + (int64_t)m * ld + n) = v;
        }
    };
    auto load_bias16 = [&](const _Float16* bp, int nb, float* bias) __attribute__((always_inline)) {
        // two 16-byte loads (n % 8 == 0, so each is wholly inside or past the end)
        const rsrc_t brs = make_rsrc(bp, bp != nullptr ? (uint32_t)N * 2u : 0u);
        const half8_t b0 = __builtin_bit_cast(half8_t, bload128(brs, (uint32_t)nb * 2u));
        const half8_t b1 = __builtin_bit_cast(half8_t, bload128(brs, (uint32_t)nb * 2u + 16u));
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            bias[r] = (float)b0[r];
            bias[r + 8] = (float)b1[r];
        }
    };
    auto store = [&]() __attribute__((always_inline)) {
        // lane: columns nw0 + 32 b + 16 g .. + 15 of token row m0 + 32 i + l32; the wave's 32 x 64
        // tile per i
        float bias[2][16];
#pragma unroll
        for (int b = 0; b < 2; ++b) load_bias16(G.bias, nw0 + 32 * b + 16 * g, bias[b]);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                uint32_t o[8];
#pragma unroll
                for (int r = 0; r < 16; r += 2)
                    o[r >> 1] = pack_half2(acc[i * 2 + b][r] + bias[b][r], acc[i * 2 + b][r + 1] + bias[b][r + 1]);
                stage_put(0, 64, 32 * b + 16 * g, o);
            }
            stage_out(0, 64, G.y, G.ldy, m0 + 32 * i, nw0);
        }
    };
    if (glu) {
        // gate = fp16(acc0 + bias0), up = fp16(acc1 + bias1), h = fp16(silu(gate) up): this
        // lane's 16 consecutive columns nw0 + 16 g .. + 15 of each, token rows m0 + 32 i + l32;
        // three 32 x 32 tiles per i
        const int nb = nw0 + 16 * g;
        float bias[2][16];
        load_bias16(G.bias, nb, bias[0]);
        load_bias16(G1.bias, nb, bias[1]);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            uint32_t og[8], ou[8], oh[8];
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                og[r >> 1] = pack_half2(acc[i * 2][r] + bias[0][r], acc[i * 2][r + 1] + bias[0][r + 1]);
                ou[r >> 1] = pack_half2(acc[i * 2 + 1][r] + bias[1][r], acc[i * 2 + 1][r + 1] + bias[1][r + 1]);
                oh[r >> 1] = swiglu_fwd2(og[r >> 1], ou[r >> 1]);
            }
            stage_put(0, 32, 16 * g, og);
            stage_put(1, 32, 16 * g, ou);
            stage_put(2, 32, 16 * g, oh);
            if (G.y != nullptr) stage_out(0, 32, G.y, G.ldy, m0 + 32 * i, nw0);
            if (G1.y != nullptr) stage_out(1, 32, G1.y, G1.ldy, m0 + 32 * i, nw0);
            stage_out(2, 32, a.h, a.ldh, m0 + 32 * i, nw0);
        }
        return;
    }
    if (a.splits > 1) {
        // fp32 partial sums into this split's slab (bias and rounding happen in the reduction)
        float* slab = a.partials + (int64_t)split * a.m * a.ncols;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int nb = nw0 + 32 * b + 16 * g;
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int m = m0 + 32 * i + l32;
                if (m >= M) continue;
                float* dst = slab + (int64_t)m * a.ncols + G.col_begin + nb;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (nb + 4 * q < N)  // n % 8 == 0: whole 16-byte chunks
                        *(float4_t*)(dst + 4 * q) = AccChunks<float16_t>::get(acc[i * 2 + b], q);
            }
        }
        return;
    }
    store();
}

template <int MB, bool NESTED>
static hipError_t launch_fwd_t(const FwdArgs& a, int grid, hipStream_t s) {
    const hipError_t e = allow_dynamic_lds((const void*)nf4_fwd_kernel<MB, NESTED>, fwd_smem_bytes(MB, true));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((nf4_fwd_kernel<MB, NESTED>), dim3(grid), dim3(kGemmThreads),
                       fwd_smem_bytes(MB, a.wide_stats != 0), s, a);
    return hipGetLastError();
}

hipError_t launch_fwd(const FwdArgs& a, int mb, int grid, hipStream_t s) {
#define X(T) \
    if (mb == T) return a.nested ? launch_fwd_t<T, true>(a, grid, s) : launch_fwd_t<T, false>(a, grid, s);
    X(1) X(2) X(4)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
