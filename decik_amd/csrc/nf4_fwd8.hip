// Fused NF4 dequant x fp16 GEMM, forward, for launches with many token rows (the same product as
// nf4_fwd_kernel: Y = X.W^T + bias + LoRA, solution/nf4.py:93-96, and the GLU mode of
// dk_nf4_glu_fwd, solution/mlp.py:69-71).
//
// Why a second kernel: with 128-token tiles every packed weight is dequantized once per 128
// tokens, and the dequant (code-book address, code-book read, fp32 multiply, fp16 pack per
// weight) is ~6 VALU instructions per 32x32x16 MFMA -- more than the SIMD co-issues with the
// matrix pipe (~4). Here a work-group is 8 waves (two per SIMD, one work-group per CU) on a tile
// of 32*MB tokens (MB = 7, 8 or 9: 224, 256 or 288 tokens) x 256 weight rows; each wave owns 32 weight
// rows and all 32*MB tokens, so each dequantized weight feeds MB MFMAs (~3 VALU per MFMA), and
// the X tile, staged once per step for all eight waves, is read by each wave at one 16-byte
// fragment per MFMA. MB = 2 and 4 (64 and 128 tokens) serve launches with few token rows: there
// the four-wave kernel's tiles leave a single wave per SIMD (one work-group per CU), which then
// waits on its own code-book reads; two waves per SIMD on the same tiles hide them (7B gate
// projection at 64 tokens: 40.2 -> 30.8 us per call).
//
// Per wave and 64-wide step: one 16-byte packed load per lane (row arow_to_n(l32), k half
// g = lane / 32) and the row's block statistics, through a per-wave LDS ring three steps deep;
// the X tile through a shared ring three steps deep (buffer_load ... lds). Slice j (16 of k) =
// one unpacked dword of 8 weights (A operand) x MB X fragments (B operands). The loop is
// software-pipelined one slice ahead: between the MFMAs of slice j the wave refills each X
// fragment register right after its MFMA has read it and unpacks slice j + 1 in three stages
// (code-book addresses, code-book reads, scaling and fp16 packing). Slice 3 holds the step
// boundary (own-slot fetch, wait, barrier); the refill of the freed ring slots starts there and
// continues through slices 0-2 of the next step, at most two loads per slice (spread_part), so
// that the eight waves' loads do not queue up in one slice.
//
// Epilogue: each token block's 32 x 256 output tile goes through LDS (the X ring, after a
// barrier) and leaves as whole 512-byte rows; GLU tiles pair the gate wave (0..3) and up wave
// (4..7) of the same columns there, so the SwiGLU needs no register exchange.
#include "gemm_common.h"

namespace dk {

constexpr int kF8Waves = 8;
constexpr int kF8Threads = 64 * kF8Waves;
constexpr int kF8Header = 2048;  // code2 tables (GLU: gate's, then up's)
constexpr int kF8Dummy = 1024;   // target of the X loads of waves past the tile (zeros)

// Per-wave ring slot of one step: 1 KB packed bytes (lane: 16 bytes), then 64 statistics dword
// slots (codes or fp32 absmax at +1024, absmax2 at +1280). Narrow (every blocksize >= 64,
// k % 64 == 0): slot l32 holds row arow(l32)'s block (lanes g = 1 load zeros into slots 32..63);
// wide: slot lane holds the block of the lane's row and k half.
constexpr int kF8WSlot = 1536;

// Epilogue staging: two 32-token blocks of fp32 partial sums (rows 1040 bytes apart), the
// largest of the epilogues; it reuses the X ring, which is sized to hold it.
constexpr int kF8Stage = 2 * 32 * (256 * 4 + 16);

// bytes of the X ring region: three step buffers, or the epilogue staging if that is larger
__host__ __device__ constexpr int fwd8_xring_bytes(int mb) {
    return 3 * 32 * mb * 128 > kF8Stage ? 3 * 32 * mb * 128 : kF8Stage;
}

__host__ __device__ constexpr size_t fwd8_smem_bytes(int mb) {
    return kF8Header + kF8Dummy + (size_t)fwd8_xring_bytes(mb) + kF8Waves * 3 * (size_t)kF8WSlot;
}

template <int MB, bool NESTED>
__global__ __launch_bounds__(kF8Threads, 1) void nf4_fwd8_kernel(const FwdArgs a) {
    constexpr int BM = 32 * MB;
    constexpr int XBUF = BM * 128;                               // bytes of one X ring buffer
    constexpr int XCH = BM * 8;                                  // its 16-byte chunks
    constexpr int XPT = (XCH + kF8Threads - 1) / kF8Threads;     // X loads per thread and step
    constexpr int NL = XPT + 1 + (NESTED ? 2 : 1);               // loads per thread and step
    static_assert(XCH % 64 == 0, "a wave's X load is wholly inside or past the tile");
    static_assert(kF8Stage <= fwd8_xring_bytes(MB), "epilogue staging fits the X ring");
    constexpr int NP = XPT + 2;                                  // load parts per step
    static_assert(NP <= 8 && MB >= 2, "at most two load parts per slice");
    constexpr int L3 = spread_loads(NP, NESTED ? 2 : 1, -1);     // loads issued in slice 3
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // byte-pair code books (gate, up in GLU mode; the same book otherwise): entry 256 b + byte
    // holds (code_b[byte >> 4], code_b[byte & 15]), the two weights of one packed byte
    __shared__ float2_t lut2[512];
    float* c2 = (float*)smem;
    uint8_t* dummy = smem + kF8Header;
    uint8_t* xs = dummy + kF8Dummy;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
    const int l32 = lane & 31, g = lane >> 5;
    const bool wide = a.wide_stats != 0;
    const bool glu = a.glu != 0;
    const int wslot_bytes = kF8WSlot;

    const int L = xcd_logical_id();
    if (L >= a.m_tiles * a.n_tiles * a.splits) return;
    // consecutive logical ids share an XCD's L2: token tiles fastest share the weight columns,
    // column tiles fastest share the token rows (chosen by the host for large token counts)
    const int mn = L % (a.m_tiles * a.n_tiles);
    const int split = L / (a.m_tiles * a.n_tiles);
    const int m_tile = a.cols_first ? mn / a.n_tiles : mn % a.m_tiles;
    const int n_tile = a.cols_first ? mn % a.n_tiles : mn / a.m_tiles;

    int gi = 0;  // the weight of this tile (normal mode)
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && n_tile >= a.g[i].tile_begin) gi = i;
    // this wave's weight: GLU waves 0..3 the gate weight, 4..7 the up weight (wave-uniform index)
    const int wgi = __builtin_amdgcn_readfirstlane(glu ? (wave >> 2) : gi);
    const FwdGroupDev& G = a.g[wgi];
    const NF4Dev& W = G.w;
    const int M = sgpr(a.m), K = sgpr(a.k), N = sgpr((int)W.n), ldx = sgpr((int)a.ldx);
    const uint32_t bs_shift = sgpr((uint32_t)W.bs_shift), bs2_shift = sgpr((uint32_t)W.bs2_shift);
    const int m0 = m_tile * BM;
    // the tile's first weight row and this wave's 32 rows within the tile's columns
    const int tile_n0 = glu ? n_tile * (kFwdBN / 2) : (n_tile - G.tile_begin) * kFwdBN;
    const int wcol = glu ? 32 * (wave & 3) : 32 * wave;  // the wave's first column in the tile
    const int nw0 = tile_n0 + wcol;
    const int ks0 = split * a.ksteps_per_split;
    const int ks1 = min(a.ksteps, ks0 + a.ksteps_per_split);

    // this thread's code-book entry and code2 entry (GLU: threads 256..511 bring the up weight's
    // table; the waves of each weight index their own), written to LDS once the ring's first
    // loads are issued, so that the two memory round trips overlap
    // (the table pointers are picked from uniform ones: indexed by thread, they would be fetched
    // by a vector load and waited for before the tables themselves)
    // (read through buffer descriptors of uniform pointers: indexed by thread, the pointers would
    // be fetched by a vector load and waited for before the tables themselves)
    const bool up_half = glu && tid >= 256;
    const rsrc_t bk0 = make_rsrc(sgpr(glu ? a.g[0].w.code : W.code), 64u);
    const rsrc_t bk1 = make_rsrc(sgpr(a.g[glu ? 1 : 0].w.code), 64u);
    const float book_hi = bloadf(up_half ? bk1 : bk0, 4u * ((tid >> 4) & 15));
    const float book_lo = bloadf(up_half ? bk1 : bk0, 4u * (tid & 15));
    float c2v = 0.0f;
    if constexpr (NESTED) {
        const rsrc_t c0 = make_rsrc(sgpr(glu ? a.g[0].w.code2 : W.code2), 1024u);
        const rsrc_t c1 = make_rsrc(sgpr(a.g[glu ? 1 : 0].w.code2), 1024u);
        if (glu || tid < 256) c2v = bloadf(up_half ? c1 : c0, 4u * (tid & 255));
    }
    const float* const c2w = c2 + (glu ? 256 * (wave >> 2) : 0);  // this wave's weight's table
    const float offset = NESTED ? *W.offset : 0.0f;
    // byte offset of this wave's byte-pair code book in lut2
    const uint32_t book8 = (uint32_t)(glu ? 2048 * (wave >> 2) : 0);
    // LDS byte address of the code-book pair of byte e of a packed dword
    auto pair_addr = [&](uint32_t w, int e) __attribute__((always_inline)) -> uint32_t {
        return (((w >> (8 * e)) & 0xFFu) << 3) + book8;
    };
    auto pair_at = [&](uint32_t addr) __attribute__((always_inline)) -> float2_t {
        return *(const float2_t*)((const char*)lut2 + addr);
    };

    const int wrow = nw0 + arow_to_n(l32);  // this lane's A row
    const bool rowok = wrow < N;
    const int xsw = (l32 >> 1) & 7;          // LDS swizzle of this lane's X rows

    // Loads use loop-invariant per-lane offsets (a lane outside the tile or the weight has bit 31
    // set: it reads zeros) against buffer descriptors whose base advances with the step, so a step
    // costs scalar additions only. This needs k % 64 == 0 and blocks that do not straddle rows
    // (k % blocksize == 0), which the planner checks before choosing this kernel. A step past the
    // split's end loads from descriptors of size 0 (zeros), keeping the ring's load count uniform.
    uint32_t xo[XPT];       // X chunk h of this thread: row (tid + 512 h) / 8 of the tile
    int xdst[XPT];          // ... and its wave's LDS destination within a ring buffer
#pragma unroll
    for (int h = 0; h < XPT; ++h) {
        const int q = tid + kF8Threads * h;
        const int row = q >> 3, pc = q & 7;
        const int c = pc ^ ((row >> 1) & 7);
        const int gm = m0 + row;
        xo[h] = off_if(q < XCH && gm < M, (uint32_t)(gm * ldx + 8 * c) * 2u);
        const int wq0 = kF8Threads * h + 64 * wave;  // the wave's first chunk (uniform)
        xdst[h] = wq0 < XCH ? wq0 * 16 : -1;         // waves past the tile load into the dummy area
    }
    const uint32_t wo = off_if(rowok, ((uint32_t)wrow * (uint32_t)K + 32u * (uint32_t)g) >> 1);
    // statistics: narrow -- lanes g = 0 fetch their row's block (g = 1 lanes load zeros into
    // unused slots); wide (blocksize 32) -- every lane its row's block at its own k half
    const uint32_t blk0 = ((uint32_t)wrow * (uint32_t)K + (wide ? 32u * (uint32_t)g : 0u)) >> bs_shift;
    const bool sok = rowok && (wide || g == 0);
    const uint32_t so = off_if(sok, NESTED ? blk0 : blk0 * 4u);

    // the buffers, held in scalar registers for the whole loop
    const uint8_t* const gx = sgpr((const uint8_t*)a.x);
    const uint32_t x_bytes = sgpr(a.x_bytes);
    const uint8_t* const gpk = sgpr(W.packed);
    const uint32_t pk_bytes = sgpr(W.packed_bytes);
    const uint8_t* const gam8 = NESTED ? sgpr(W.absmax8) : nullptr;
    const float* const gamf = NESTED ? nullptr : sgpr(W.absmaxf);
    const uint32_t am_bytes = sgpr(W.absmax_bytes);
    const float* const gam2 = NESTED ? sgpr(W.absmax2) : nullptr;
    const uint32_t am2_bytes = NESTED ? sgpr(W.absmax2_bytes) : 0u;
    uint8_t* wring = xs + fwd8_xring_bytes(MB) + wave * (3 * wslot_bytes);
    // Part p of step t's loads (p < XPT: X chunk p; XPT: the packed weights; XPT + 1: their
    // statistics), so that the main loop issues a step's loads one per MFMA gap: issued in one
    // burst after the barrier they held up the matrix pipe.
    auto load_part = [&](int p, int t, int rx, int rw, bool live) __attribute__((always_inline)) {
        const uint32_t k0 = (uint32_t)t * kFwdBK;
        if (p < XPT) {
            const rsrc_t xrs = make_rsrc(gx + 2u * k0, live ? x_bytes - 2u * k0 : 0u);
            // loads p < XPT - 1 never pass the tile (folded at compile time: no scalar select)
            bload128_lds(xrs, ((p + 1) * kF8Threads <= XCH || xdst[p] >= 0) ? xs + rx + xdst[p] : dummy, xo[p]);
            return;
        }
        uint8_t* slot = wring + rw;
        if (p == XPT) {
            const rsrc_t wrs = make_rsrc(gpk + k0 / 2u, live ? pk_bytes - k0 / 2u : 0u);
            bload128_lds(wrs, slot, wo);
            return;
        }
        const uint32_t kb = k0 >> bs_shift;  // blocks of a row before this step
        if constexpr (NESTED) {
            const rsrc_t ars = make_rsrc(gam8 + kb, live ? am_bytes - kb : 0u);
            const rsrc_t a2rs = make_rsrc(gam2, live ? am2_bytes : 0u);
            bload8_lds(ars, slot + 1024, so);
            bload32_lds(a2rs, slot + 1280, off_if(sok, ((blk0 + kb) >> bs2_shift) * 4u));
        } else {
            const rsrc_t ars = make_rsrc(gamf + kb, live ? am_bytes - 4u * kb : 0u);
            bload32_lds(ars, slot + 1024, so);
        }
    };
    // every load of step t (the prologue)
    auto load_step = [&](int t, int rx, int rw, bool live) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < XPT + 2; ++p) load_part(p, t, rx, rw, live);
    };
    // fp32 scale of this lane's row at step t (0 outside the weight)
    auto scale_of = [&](const uint8_t* slot) __attribute__((always_inline)) -> float {
        const int si = wide ? lane : l32;
        float sc;
        if constexpr (NESTED) {
            const uint32_t q = slot[1024 + 4 * si];
            const float a2 = *(const float*)(slot + 1280 + 4 * si);
            sc = c2w[q] * a2 + offset;
        } else {
            sc = *(const float*)(slot + 1024 + 4 * si);
        }
        return rowok ? sc : 0.0f;
    };
    auto xfrag = [&](const uint8_t* xb, int i, int j) __attribute__((always_inline)) -> half8_t {
        return *(const half8_t*)(xb + (32 * i + l32) * 128 + (((4 * g + j) ^ xsw) << 4));
    };

    float16_t acc[MB];  // token block i
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = float16_t{};

    // Ring buffers: step t uses X buffer rx0 (byte offset in the X ring) and weight slot rw0;
    // step t + 1 uses rx1 / rw1; step t + 3 reuses step t's.
    int rx0 = 0, rw0 = 0, rx1 = XBUF, rw1 = wslot_bytes, rx2 = 2 * XBUF, rw2 = 2 * wslot_bytes;
    // Prologue: two steps and the slice-3 parts of the third in flight (issued before the LoRA
    // term, whose loads then share their round trip); the wait for the first follows the LoRA term.
    load_step(ks0, 0, 0, true);
    load_step(ks0 + 1, XBUF, wslot_bytes, ks0 + 1 < ks1);
#pragma unroll
    for (int i = 0; i < NP; i += 4) load_part(spread_part(i, XPT), ks0 + 2, rx2, rw2, ks0 + 2 < ks1);

    // LoRA term s * U.B^T first (split 0 only), as in nf4_fwd_kernel, for this wave's weight.
    {
        const int R = (G.lora_u != nullptr && split == 0) ? sgpr(a.lora_rank) : 0;
        const float ls = G.lora_scale;
        const rsrc_t brs = make_rsrc(G.lora_b, (uint32_t)N * (uint32_t)R * 2u);
        const rsrc_t urs = make_rsrc(G.lora_u, (uint32_t)M * (uint32_t)R * 2u);
        for (int t0 = 0; t0 < R; t0 += 16) {
            half8_t bl = __builtin_bit_cast(half8_t, bload128(brs, off_if(rowok, (uint32_t)(wrow * R + t0 + 8 * g) * 2u)));
#pragma unroll
            for (int e = 0; e < 8; ++e) bl[e] = (_Float16)((float)bl[e] * ls);
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int m = m0 + 32 * i + l32;
                const half8_t uu = __builtin_bit_cast(half8_t, bload128(urs, off_if(m < M, (uint32_t)(m * R + t0 + 8 * g) * 2u)));
                acc[i] = mfma32x32x16(bl, uu, acc[i]);
            }
        }
    }

    // the code book and code2 table (their loads have landed: they are older than the ring's)
    lut2[tid] = float2_t{book_hi, book_lo};
    if constexpr (NESTED)
        if (glu || tid < 256) c2[tid] = c2v;
    wait_vmcnt<NL + L3>();
    lds_barrier();

    u32x4_t p;  // packed weights of the current step (slice j: dword j)
    float s;    // their scale
    auto fetch_step = [&](int rw) __attribute__((always_inline)) {
        const uint8_t* ws = wring + rw;
        p = *(const u32x4_t*)(ws + 16 * lane);
        s = scale_of(ws);
    };
    half8_t xf[MB], w, wn;
    uint32_t pa[4];   // code-book pair addresses of the next slice's 4 packed bytes
    float v[8];       // its code-book values
    fetch_step(rw0);
#pragma unroll
    for (int i = 0; i < MB; ++i) xf[i] = xfrag(xs + rx0, i, 0);
    {
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float2_t cv = pair_at(pair_addr(p[0], e));
            o[e] = pack_half2(cv.x * s, cv.y * s);
        }
        w = __builtin_bit_cast(half8_t, o);
    }
    // stage positions (MFMA index after which a stage runs). With seven or more MFMAs a slice the
    // stages take separate gaps, and in slice 3, whose first gap holds the step boundary, the
    // address and code-book stages move one gap later; with fewer (MB = 2, 4) the code-book reads
    // follow the addresses in the first gap of every slice and the scaling takes the last gap
    // that leaves them time to land.
    constexpr bool SMALL = MB < 7;
    constexpr int qA = 0, qB = SMALL ? 0 : 1, qC = SMALL ? (MB > 2 ? MB - 2 : 1) : MB - 3;
    constexpr int q3 = SMALL ? 0 : 1;  // slice 3's shift of stages A and B
    for (int t = ks0; t < ks1; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int jn = (j + 1) & 3;
#pragma unroll
            for (int q = 0; q < MB; ++q) {
                acc[q] = mfma32x32x16(w, xf[q], acc[q]);
                if (j == 3 && q == 0) {
                    // step t+1's loads have landed (only step t+2's may be in flight): fetch this
                    // wave's packed bytes and scale; after the barrier no wave reads step t's
                    // slots again: refill them with step t+3. Past the last step these reads
                    // see stale slots and their values go unused.
                    wait_vmcnt<NL>();
                    fetch_step(rw1);
                    lds_barrier();
                }
                // ring refills: slice 3 starts step t+3 in the slots step t has freed, slices 0-2
                // continue step t+2
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int i = 4 * r + (j == 3 ? 0 : j + 1);
                    if (i < NP && q == r * (MB / 2)) {
                        if (j == 3) load_part(spread_part(i, XPT), t + 3, rx0, rw0, t + 3 < ks1);
                        else load_part(spread_part(i, XPT), t + 2, rx2, rw2, t + 2 < ks1);
                    }
                }
                // refill the X fragment the MFMA above has read (slice j + 1)
                xf[q] = xfrag(xs + (j < 3 ? rx0 : rx1), q, jn);
                if (q == (j < 3 ? qA : qA + q3)) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) pa[e] = pair_addr(p[jn], e);
                }
                if (q == (j < 3 ? qB : qB + q3)) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float2_t cv = pair_at(pa[e]);
                        v[2 * e] = cv.x;
                        v[2 * e + 1] = cv.y;
                    }
                }
                if (q == qC) {
                    u32x4_t o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = pack_half2(v[2 * e] * s, v[2 * e + 1] * s);
                    wn = __builtin_bit_cast(half8_t, o);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            w = wn;
        }
        // rotate the rings: step t + 1's buffers become the current ones
        const int rxo = rx0, rwo = rw0;
        rx0 = rx1;
        rw0 = rw1;
        rx1 = rx2;
        rw1 = rw2;
        rx2 = rxo;
        rw2 = rwo;
    }
    wait_vmcnt<0>();
    lds_barrier();  // every wave is done with the X ring: it becomes the staging area

    // ---- epilogue. Lane (l32, g) holds, for token block i, token row m0 + 32 i + l32 and the 16
    // consecutive columns nw0 + 16 g + r (acc[i][r]).
    const int colw = wcol + 16 * g;  // ... as a column of the tile
    float bias[16];
    {
        const rsrc_t brs = make_rsrc(G.bias, G.bias != nullptr ? (uint32_t)N * 2u : 0u);
        const uint32_t nb = (uint32_t)(nw0 + 16 * g);
        const half8_t b0 = __builtin_bit_cast(half8_t, bload128(brs, nb * 2u));
        const half8_t b1 = __builtin_bit_cast(half8_t, bload128(brs, nb * 2u + 16u));
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            bias[r] = (float)b0[r];
            bias[r + 8] = (float)b1[r];
        }
    }
    if (a.splits > 1) {
        // fp32 partial sums, staged as 32 x 256 fp32 tiles (rows 1040 bytes apart), into this
        // split's slab (bias and rounding happen in the reduction)
        constexpr int RB = 256 * 4 + 16;
        float* slab = a.partials + (int64_t)split * a.m * a.ncols;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            uint8_t* buf = xs + (i & 1) * 32 * RB;
            uint8_t* lp = buf + l32 * RB + colw * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q) *(float4_t*)(lp + 16 * q) = AccChunks<float16_t>::get(acc[i], q);
            lds_barrier();
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int c = tid + kF8Threads * h, row = c >> 6, cc = c & 63;
                const float4_t val = *(const float4_t*)(buf + row * RB + cc * 16);
                const int m = m0 + 32 * i + row, n = tile_n0 + 4 * cc;
                if (m < M && n < N) *(float4_t*)(slab + (int64_t)m * a.ncols + G.col_begin + n) = val;
            }
        }
        return;
    }
    if (glu) {
        // gate (waves 0..3) and up (waves 4..7) tiles of 32 x 128 fp16 side by side in LDS; each
        // thread then owns one 16-byte chunk of both and writes gate, up and h
        constexpr int RB = 128 * 2 + 16;
        const FwdGroupDev& Gg = a.g[0];
        const FwdGroupDev& Gu = a.g[1];
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            uint8_t* buf = xs + (i & 1) * 2 * 32 * RB;
            uint8_t* lp = buf + (wave >> 2) * 32 * RB + l32 * RB + colw * 2;
            uint32_t o[8];
#pragma unroll
            for (int r = 0; r < 16; r += 2) o[r >> 1] = pack_half2(acc[i][r] + bias[r], acc[i][r + 1] + bias[r + 1]);
            *(u32x4_t*)lp = u32x4_t{o[0], o[1], o[2], o[3]};
            *(u32x4_t*)(lp + 16) = u32x4_t{o[4], o[5], o[6], o[7]};
            lds_barrier();
            const int row = tid >> 4, cc = tid & 15;
            const u32x4_t gv = *(const u32x4_t*)(buf + row * RB + cc * 16);
            const u32x4_t uv = *(const u32x4_t*)(buf + 32 * RB + row * RB + cc * 16);
            const int m = m0 + 32 * i + row, n = tile_n0 + 8 * cc;
            if (m < M && n < N) {
                // gate and up are read again two launches later (by the SwiGLU backward, which
                // fetches them as it starts): stored non-temporally, past the caches that the next
                // launch's h and weights use (MLP step 0.5% faster); h stays cached
                if (Gg.y != nullptr) __builtin_nontemporal_store(gv, (u32x4_t*)(Gg.y + (int64_t)m * Gg.ldy + n));
                if (Gu.y != nullptr) __builtin_nontemporal_store(uv, (u32x4_t*)(Gu.y + (int64_t)m * Gu.ldy + n));
                *(u32x4_t*)(a.h + (int64_t)m * a.ldh + n) =
                    u32x4_t{swiglu_fwd2(gv[0], uv[0]), swiglu_fwd2(gv[1], uv[1]), swiglu_fwd2(gv[2], uv[2]),
                            swiglu_fwd2(gv[3], uv[3])};
            }
        }
        return;
    }
    {
        // 32 x 256 fp16 tiles (rows 528 bytes apart) -> whole 512-byte rows of y
        constexpr int RB = 256 * 2 + 16;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            uint8_t* buf = xs + (i & 1) * 32 * RB;
            uint8_t* lp = buf + l32 * RB + colw * 2;
            uint32_t o[8];
#pragma unroll
            for (int r = 0; r < 16; r += 2) o[r >> 1] = pack_half2(acc[i][r] + bias[r], acc[i][r + 1] + bias[r + 1]);
            *(u32x4_t*)lp = u32x4_t{o[0], o[1], o[2], o[3]};
            *(u32x4_t*)(lp + 16) = u32x4_t{o[4], o[5], o[6], o[7]};
            lds_barrier();
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = tid + kF8Threads * h, row = c >> 5, cc = c & 31;
                const u32x4_t val = *(const u32x4_t*)(buf + row * RB + cc * 16);
                const int m = m0 + 32 * i + row, n = tile_n0 + 8 * cc;
                if (m < M && n < N) *(u32x4_t*)(G.y + (int64_t)m * G.ldy + n) = val;
            }
        }
    }
}

template <int MB, bool NESTED>
static hipError_t launch_fwd8_t(const FwdArgs& a, int grid, hipStream_t s) {
    const hipError_t e = allow_dynamic_lds((const void*)nf4_fwd8_kernel<MB, NESTED>, fwd8_smem_bytes(MB));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((nf4_fwd8_kernel<MB, NESTED>), dim3(grid), dim3(kF8Threads),
                       fwd8_smem_bytes(MB), s, a);
    return hipGetLastError();
}

hipError_t launch_fwd8(const FwdArgs& a, int mb, int grid, hipStream_t s) {
#define X(T) \
    if (mb == T) return a.nested ? launch_fwd8_t<T, true>(a, grid, s) : launch_fwd8_t<T, false>(a, grid, s);
    X(2) X(4) X(7) X(8) X(9)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace dk
