// Rank-r LoRA products around the fused GEMMs (r = 16 for q/v in the reference run).
//
// The reference runs peft's branch as fp16 matmuls (solution/attn.py:225-228 forward,
// :251-257 backward). Here:
//   lora_down:  U  = fp16(X . A^T)                 [m, r]   (the forward epilogue adds s U.B^T)
//   lora_gu:    GU = fp16(s * dY . B)              [m, r]   (the backward epilogue adds GU.A)
//   lora_db:    dB = s * dY^T . U                  fp32 [n, r]
//   lora_da:    dA = GU^T . X                      fp32 [r, k]
// All four are small (about 2% of the flops of the projection they ride on) and run on
// v_mfma_f32_16x16x32_f16: a work-group of 8 waves owns one 16-row output tile (16 tokens for U
// and GU, 16 weight rows for dB, 16 columns of A for dA) and all r rank columns; its waves take
// the 32-wide contraction chunks in turn and their fp32 tiles are summed through LDS in wave
// order, so the summation order is fixed (no atomics) and every call gives the same bits.
// GU and dB are one launch (both read dY); dA, which needs GU, is a second one. The LoRA branches
// of one layer (q and v) share each launch: a job table gives every branch its own range of
// work-groups (a branch's tiles are those of a launch of it alone, so the bits are the same).
//
// X, as lora_down and lora_da read it, is the branch's input: fp16 or fp32 storage, optionally
// through dropout (LoRAPairFromNorm's packed path, solution/attn.py:153-165, 219-223, 241-243):
// fp16(x * (keep * scale)) with keep a packed bit ([m, k / 8] bytes, bit j % 8 of byte j / 8)
// and scale = 1 / (1 - p) a device scalar, in fp32 and in that order, as skc_lora_inputs_kernel
// rounds it; fp32 without dropout is fp16(x). The dropped-out input is never stored.
//
// MFMA operand layout (16x16x32, lane l, i = l % 16, g = l / 16): A operand A[i][8 g + e],
// B operand B[8 g + e][i], result D[4 g + r][i], e = 0..7, r = 0..3. Operands whose 8 contraction
// values are contiguous in memory are one 16-byte load; the others (the token-contracted products
// dB and dA, and B's rows in GU) are gathered with 2-byte loads, all from the L2-resident
// activations.
#include "dk_internal.h"

namespace dk {

constexpr int kLoraWaves = 8;
constexpr int kLoraThreads = 64 * kLoraWaves;

__device__ __forceinline__ half8_t gather8(rsrc_t r, uint32_t off0, uint32_t stride, bool ok0, int valid) {
    // 8 fp16 values at off0 + e * stride (bytes); element e reads zero unless ok0 && e < valid
    half8_t v;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        v[e] = __builtin_bit_cast(_Float16, (uint16_t)bload16(r, off_if(ok0 && e < valid, off0 + (uint32_t)e * stride)));
    return v;
}

// Sum the 8 waves' 16 x R tiles (lane: rows 4 g + r, column 16 h + i) in wave order; thread t
// of the work-group then holds element t of the tile (row t / R, column t % R) in *out for
// t < 16 R. red: 8 x 16 x R floats.
template <int R>
__device__ __forceinline__ void reduce_tiles(const float4_t (&acc)[R / 16], float* red, int wave, int lane) {
    const int i = lane & 15, g = lane >> 4;
#pragma unroll
    for (int h = 0; h < R / 16; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * 16 + 4 * g + r) * R + 16 * h + i] = acc[h][r];
    __syncthreads();
}

template <int R>
__device__ __forceinline__ float tile_sum(const float* red, int t) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kLoraWaves; ++w) s += red[w * 16 * R + t];
    return s;
}

// The branch input X (see above): descriptors and the keep scale.
struct XInput {
    rsrc_t x, keep;
    float scale;
    int ldx, kbytes;  // row strides: x in elements, keep in bytes (k / 8)
};

template <bool X32, bool KEEP>
__device__ __forceinline__ XInput x_input(const void* x, int m, int k, int ldx, const uint8_t* keep,
                                          const float* keep_scale) {
    XInput in;
    in.x = make_rsrc(x, (uint32_t)(((int64_t)(m - 1) * ldx + k) * (X32 ? 4 : 2)));
    in.keep = make_rsrc(keep, KEEP ? (uint32_t)m * (uint32_t)(k >> 3) : 0u);
    in.scale = KEEP ? *keep_scale : 0.0f;
    in.ldx = ldx;
    in.kbytes = k >> 3;
    return in;
}

// x * (keep * scale) for the 8 values of one keep byte's bits sh(e) (dropout), then fp16
template <bool KEEP>
__device__ __forceinline__ half8_t drop_round(const float (&xf)[8], const uint32_t (&bits)[8], float scale) {
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if constexpr (KEEP) {
            float v = xf[e] * ((float)(bits[e] & 1u) * scale);
            // the product is rounded to fp32 and then to fp16, as the reference rounds it: the
            // empty asm keeps the compiler from folding multiply and conversion into one
            // v_fma_mix (a single rounding, which differs at fp16 ties)
            asm("" : "+v"(v));
            o[e] = (_Float16)v;
        } else

            o[e] = (_Float16)xf[e];
    }
    return o;
}

// X[row, kk .. kk + 7] (kk % 8 == 0); zeros unless ok
template <bool X32, bool KEEP>
__device__ __forceinline__ half8_t x_row8(const XInput& in, int row, int kk, bool ok) {
    if constexpr (!X32 && !KEEP)
        return __builtin_bit_cast(half8_t, bload128(in.x, off_if(ok, (uint32_t)(row * in.ldx + kk) * 2u)));
    float xf[8];
    if constexpr (X32) {
        const uint32_t o = (uint32_t)(row * in.ldx + kk) * 4u;
        const float4_t lo = __builtin_bit_cast(float4_t, bload128(in.x, off_if(ok, o)));
        const float4_t hi = __builtin_bit_cast(float4_t, bload128(in.x, off_if(ok, o + 16u)));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xf[e] = lo[e];
            xf[e + 4] = hi[e];
        }
    } else {
        const half8_t h = __builtin_bit_cast(half8_t, bload128(in.x, off_if(ok, (uint32_t)(row * in.ldx + kk) * 2u)));
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = (float)h[e];
    }
    uint32_t bits[8];
    if constexpr (KEEP) {
        const uint32_t byte = bload8(in.keep, off_if(ok, (uint32_t)(row * in.kbytes + (kk >> 3))));
#pragma unroll
        for (int e = 0; e < 8; ++e) bits[e] = byte >> e;
    }
    return drop_round<KEEP>(xf, bits, in.scale);
}

// X[mm + e, col] for e < valid (zeros past it, or everywhere unless ok0)
template <bool X32, bool KEEP>
__device__ __forceinline__ half8_t x_col8(const XInput& in, int mm, int col, bool ok0, int valid) {
    if constexpr (!X32 && !KEEP)
        return gather8(in.x, (uint32_t)(mm * in.ldx + col) * 2u, 2u * (uint32_t)in.ldx, ok0, valid);
    float xf[8];
    uint32_t bits[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const bool ok = ok0 && e < valid;
        const uint32_t o = (uint32_t)((mm + e) * in.ldx + col);
        if constexpr (X32)
            xf[e] = bloadf(in.x, off_if(ok, o * 4u));
        else
            xf[e] = (float)__builtin_bit_cast(_Float16, (uint16_t)bload16(in.x, off_if(ok, o * 2u)));
        if constexpr (KEEP)
            bits[e] = bload8(in.keep, off_if(ok, (uint32_t)((mm + e) * in.kbytes + (col >> 3)))) >> (col & 7);
    }
    return drop_round<KEEP>(xf, bits, in.scale);
}

// Job tables of the grouped launches (kernel arguments): branch j owns the work-groups
// [start[j], start[j + 1]), and each of its work-groups computes what it computes in a launch of
// that branch alone.
struct DownJob {
    const void* x;
    const uint8_t* keep;
    const float* keep_scale;
    const _Float16* a;
    _Float16* u;
    int ldx;
};
struct GuDbJob {
    const _Float16* dy;
    const _Float16* u;
    const _Float16* b;
    _Float16* gu;
    float* db;
    float scale;
    int lddy, n;
};
struct DaJob {
    const _Float16* gu;
    const void* x;
    const uint8_t* keep;
    const float* keep_scale;
    float* da;
    int ldx;
};
template <typename J>
struct Jobs {
    J j[kLoraMaxBranches];
    int start[kLoraMaxBranches + 1];
    int nj, m, k;
};

// this work-group's branch (uniform) and its work-group index within the branch's range
template <typename J>
__device__ __forceinline__ int job_of(const Jobs<J>& jobs, int* local) {
    int jb = 0;
#pragma unroll
    for (int q = 1; q < kLoraMaxBranches; ++q)
        if (q < jobs.nj && (int)blockIdx.x >= jobs.start[q]) jb = q;
    *local = (int)blockIdx.x - jobs.start[jb];
    return __builtin_amdgcn_readfirstlane(jb);
}

// U[m, t] = fp16(sum_k X[m, k] A[t, k]): A operand X (16 tokens), B operand A^T (rows of A).
template <int R, bool X32, bool KEEP>
__global__ __launch_bounds__(kLoraThreads) void lora_down_kernel(const Jobs<DownJob> jobs) {
    __shared__ float red[kLoraWaves * 16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    int tile;
    const DownJob& J = jobs.j[job_of(jobs, &tile)];
    const int m = jobs.m, k = jobs.k;
    const int m0 = tile * 16;
    const XInput xin = x_input<X32, KEEP>(J.x, m, k, J.ldx, J.keep, J.keep_scale);
    const rsrc_t ar = make_rsrc(J.a, (uint32_t)R * (uint32_t)k * 2u);
    _Float16* const u = J.u;
    const bool rok = m0 + i < m;
    float4_t acc[R / 16];
#pragma unroll
    for (int h = 0; h < R / 16; ++h) acc[h] = float4_t{};
    const int nk = (k + 31) >> 5;
    // two chunks per iteration (the second reads zeros past the end): their loads overlap
    for (int kc = wave; kc < nk; kc += 2 * kLoraWaves) {
        half8_t xa[2], ab[2][R / 16];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int kk = 32 * (kc + q * kLoraWaves) + 8 * g;  // k % 8 == 0: wholly inside or past the end
            xa[q] = x_row8<X32, KEEP>(xin, m0 + i, kk, rok && kk < k);
#pragma unroll
            for (int h = 0; h < R / 16; ++h)
                ab[q][h] = __builtin_bit_cast(half8_t, bload128(ar, off_if(kk < k, (uint32_t)((16 * h + i) * k + kk) * 2u)));
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int h = 0; h < R / 16; ++h) acc[h] = mfma16x16x32(xa[q], ab[q][h], acc[h]);
    }
    reduce_tiles<R>(acc, red, wave, lane);
    for (int t = threadIdx.x; t < 16 * R; t += kLoraThreads) {
        const int row = m0 + t / R;
        if (row < m) u[(int64_t)row * R + t % R] = to_half(tile_sum<R>(red, t));
    }
}

// A branch's work-groups [0, m_tiles): GU tiles, GU[m, t] = fp16(s sum_n dY[m, n] B[n, t]);
// the next ones (when it wants dB): dB tiles, dB[n, t] = s sum_m dY[m, n] U[m, t].
template <int R>
__global__ __launch_bounds__(kLoraThreads) void lora_gu_db_kernel(const Jobs<GuDbJob> jobs) {
    __shared__ float red[kLoraWaves * 16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    int tile;
    const GuDbJob& J = jobs.j[job_of(jobs, &tile)];
    const int m = jobs.m, n = J.n, lddy = J.lddy;
    const int m_tiles = (m + 15) / 16;
    const float scale = J.scale;
    const rsrc_t dr = make_rsrc(J.dy, (uint32_t)(((int64_t)(m - 1) * lddy + n) * 2));
    float4_t acc[R / 16];
#pragma unroll
    for (int h = 0; h < R / 16; ++h) acc[h] = float4_t{};
    if (tile < m_tiles) {
        const int m0 = tile * 16;
        const rsrc_t br = make_rsrc(J.b, (uint32_t)n * (uint32_t)R * 2u);
        _Float16* const gu = J.gu;
        const bool rok = m0 + i < m;
        const int nc = (n + 31) >> 5;
        for (int c = wave; c < nc; c += 2 * kLoraWaves) {
            half8_t ya[2], bb[2][R / 16];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int nn = 32 * (c + q * kLoraWaves) + 8 * g;  // n % 8 == 0
                ya[q] = __builtin_bit_cast(half8_t, bload128(dr, off_if(rok && nn < n, (uint32_t)((m0 + i) * lddy + nn) * 2u)));
                // B[nn + e][16 h + i]: rows of B, R fp16 apart
#pragma unroll
                for (int h = 0; h < R / 16; ++h)
                    bb[q][h] = gather8(br, (uint32_t)(nn * R + 16 * h + i) * 2u, 2u * R, nn < n, 8);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int h = 0; h < R / 16; ++h) acc[h] = mfma16x16x32(ya[q], bb[q][h], acc[h]);
        }
        reduce_tiles<R>(acc, red, wave, lane);
        for (int t = threadIdx.x; t < 16 * R; t += kLoraThreads) {
            const int row = m0 + t / R;
            if (row < m) gu[(int64_t)row * R + t % R] = to_half(scale * tile_sum<R>(red, t));
        }
        return;
    }
    float* const db = J.db;
    if (db == nullptr) return;
    const int n0 = (tile - m_tiles) * 16;
    const rsrc_t ur = make_rsrc(J.u, (uint32_t)m * (uint32_t)R * 2u);
    const bool cok = n0 + i < n;
    const int mc = (m + 31) >> 5;
    for (int c = wave; c < mc; c += 2 * kLoraWaves) {
        half8_t ya[2], ub[2][R / 16];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int mm = min(32 * (c + q * kLoraWaves) + 8 * g, m);  // rows past m: zeros
            const int valid = m - mm;  // rows mm .. mm + 7 that exist
            // A = dY^T: A[n0 + i][mm + e] = dY[mm + e][n0 + i]
            ya[q] = gather8(dr, (uint32_t)(mm * lddy + n0 + i) * 2u, 2u * (uint32_t)lddy, cok, valid);
#pragma unroll
            for (int h = 0; h < R / 16; ++h)
                ub[q][h] = gather8(ur, (uint32_t)(mm * R + 16 * h + i) * 2u, 2u * R, true, valid);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int h = 0; h < R / 16; ++h) acc[h] = mfma16x16x32(ya[q], ub[q][h], acc[h]);
    }
    reduce_tiles<R>(acc, red, wave, lane);
    for (int t = threadIdx.x; t < 16 * R; t += kLoraThreads) {
        const int row = n0 + t / R;
        if (row < n) db[(int64_t)row * R + t % R] = scale * tile_sum<R>(red, t);
    }
}

// dA[t, k] = sum_m GU[m, t] X[m, k]: work-group = 16 columns k (all R rows t); A operand GU^T,
// B operand X, both gathered along the token dimension.
template <int R, bool X32, bool KEEP>
__global__ __launch_bounds__(kLoraThreads) void lora_da_kernel(const Jobs<DaJob> jobs) {
    __shared__ float red[kLoraWaves * 16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    int tile;
    const DaJob& J = jobs.j[job_of(jobs, &tile)];
    const int m = jobs.m, k = jobs.k;
    const int k0 = tile * 16;
    const rsrc_t gr = make_rsrc(J.gu, (uint32_t)m * (uint32_t)R * 2u);
    const XInput xin = x_input<X32, KEEP>(J.x, m, k, J.ldx, J.keep, J.keep_scale);
    float* const da = J.da;
    const bool cok = k0 + i < k;
    // acc[h]: D[t = 16 h + 4 g + r][k0 + i]
    float4_t acc[R / 16];
#pragma unroll
    for (int h = 0; h < R / 16; ++h) acc[h] = float4_t{};
    const int mc = (m + 31) >> 5;
    for (int c = wave; c < mc; c += 2 * kLoraWaves) {
        half8_t xb[2], ga[2][R / 16];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int mm = min(32 * (c + q * kLoraWaves) + 8 * g, m);  // rows past m: zeros
            const int valid = m - mm;
            xb[q] = x_col8<X32, KEEP>(xin, mm, k0 + i, cok, valid);
#pragma unroll
            for (int h = 0; h < R / 16; ++h)
                ga[q][h] = gather8(gr, (uint32_t)(mm * R + 16 * h + i) * 2u, 2u * R, true, valid);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int h = 0; h < R / 16; ++h) acc[h] = mfma16x16x32(ga[q][h], xb[q], acc[h]);
    }
    // lane holds D[16 h + 4 g + r][k0 + i]: write as a [R][16] tile (row t, column i)
#pragma unroll
    for (int h = 0; h < R / 16; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * R + 16 * h + 4 * g + r) * 16 + i] = acc[h][r];
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * R; t += kLoraThreads) {
        const int row = t / 16, col = k0 + t % 16;  // row = rank index
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kLoraWaves; ++w) s += red[w * 16 * R + t];
        if (col < k) da[(int64_t)row * k + col] = s;
    }
}

#define DK_XIN_CASES(X, R)                                                                             \
    X(R, false, false) X(R, false, true) X(R, true, false) X(R, true, true)

// the kind of a branch's input: fp16 / fp32, with or without dropout (one kernel instance each)
static int input_kind(const LoraBranch& b) { return (b.x32 ? 2 : 0) + (b.keep != nullptr ? 1 : 0); }

hipError_t launch_lora_down(const LoraBranch* br, int nbr, int64_t m, int64_t k, int rank, hipStream_t s) {
    if (m == 0 || nbr == 0) return hipSuccess;
    if (nbr > kLoraMaxBranches) return hipErrorInvalidValue;
    const int m_tiles = (int)((m + 15) / 16);
    for (int kind = 0; kind < 4; ++kind) {
        Jobs<DownJob> jobs{};
        jobs.m = (int)m;
        jobs.k = (int)k;
        int blocks = 0;
        for (int b = 0; b < nbr; ++b) {
            if (input_kind(br[b]) != kind) continue;
            jobs.j[jobs.nj] = DownJob{br[b].x, br[b].keep, br[b].keep_scale, br[b].a, br[b].u, (int)br[b].ldx};
            jobs.start[jobs.nj++] = blocks;
            blocks += m_tiles;
        }
        if (jobs.nj == 0) continue;
        jobs.start[jobs.nj] = blocks;
        const bool x32 = (kind & 2) != 0, kp = (kind & 1) != 0;
        hipError_t e = hipErrorInvalidValue;
#define X(R, X32, KEEP)                                                                                \
    if (rank == R && x32 == X32 && kp == KEEP) {                                                       \
        hipLaunchKernelGGL((lora_down_kernel<R, X32, KEEP>), dim3(blocks), dim3(kLoraThreads), 0, s, jobs); \
        e = hipGetLastError();                                                                         \
    }
        DK_XIN_CASES(X, 16)
        DK_XIN_CASES(X, 32)
#undef X
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_lora_bwd(const LoraBranch* br, int nbr, int64_t m, int64_t k, int rank, hipStream_t s) {
    if (m == 0 || nbr == 0) return hipSuccess;
    if (nbr > kLoraMaxBranches) return hipErrorInvalidValue;
    const int m_tiles = (int)((m + 15) / 16);
    // GU and dB of every branch: one launch (no dependence on the input's kind)
    {
        Jobs<GuDbJob> jobs{};
        jobs.m = (int)m;
        jobs.k = (int)k;
        int blocks = 0;
        for (int b = 0; b < nbr; ++b) {
            const LoraBranch& B = br[b];
            jobs.j[jobs.nj] = GuDbJob{B.dy, B.u, B.b, B.gu, B.db, B.scale, (int)B.lddy, (int)B.n};
            jobs.start[jobs.nj++] = blocks;
            blocks += m_tiles + (B.db != nullptr ? (int)((B.n + 15) / 16) : 0);
        }
        jobs.start[jobs.nj] = blocks;
        hipError_t e = hipErrorInvalidValue;
#define X(R)                                                                                           \
    if (rank == R) {                                                                                   \
        hipLaunchKernelGGL((lora_gu_db_kernel<R>), dim3(blocks), dim3(kLoraThreads), 0, s, jobs);      \
        e = hipGetLastError();                                                                         \
    }
        X(16)
        X(32)
#undef X
        if (e != hipSuccess) return e;
    }
    // dA (needs GU) of the branches that want it: one launch per kind of input
    const int k_tiles = (int)((k + 15) / 16);
    for (int kind = 0; kind < 4; ++kind) {
        Jobs<DaJob> jobs{};
        jobs.m = (int)m;
        jobs.k = (int)k;
        int blocks = 0;
        for (int b = 0; b < nbr; ++b) {
            if (br[b].da == nullptr || input_kind(br[b]) != kind) continue;
            jobs.j[jobs.nj] = DaJob{br[b].gu, br[b].x, br[b].keep, br[b].keep_scale, br[b].da, (int)br[b].ldx};
            jobs.start[jobs.nj++] = blocks;
            blocks += k_tiles;
        }
        if (jobs.nj == 0) continue;
        jobs.start[jobs.nj] = blocks;
        const bool x32 = (kind & 2) != 0, kp = (kind & 1) != 0;
        hipError_t e = hipErrorInvalidValue;
#define X(R, X32, KEEP)                                                                                \
    if (rank == R && x32 == X32 && kp == KEEP) {                                                       \
        hipLaunchKernelGGL((lora_da_kernel<R, X32, KEEP>), dim3(blocks), dim3(kLoraThreads), 0, s, jobs); \
        e = hipGetLastError();                                                                         \
    }
        DK_XIN_CASES(X, 16)
        DK_XIN_CASES(X, 32)
#undef X
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace dk
