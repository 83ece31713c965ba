// Kernel argument blocks and launch helpers shared by the C ABI (capi.hip) and the kernels.
#pragma once

#include "nf4_device.h"

namespace dk {

constexpr int kDequantThreads = 256;
constexpr int kMaxDequantBatch = 24;  // weights per launch (kernel arguments stay < 4 KB)
constexpr int kDequantUnits = 8;  // packed dwords per thread

struct DequantArgs {
    NF4Dev w[kMaxDequantBatch];
    uint16_t* out[kMaxDequantBatch];
    int64_t nbytes[kMaxDequantBatch];
    int32_t wg_begin[kMaxDequantBatch + 1];
    int32_t fast[kMaxDequantBatch];
    int32_t count;
};

__global__ void nf4_dequant_kernel(const DequantArgs a);
hipError_t launch_block_scales(const NF4Dev& w, int64_t nblocks, float* out, hipStream_t s);

// ------------------------------------------------------------------------------------------
// Fused dequant x GEMM. Forward: work-group = 4 waves, tile = 32*MB token rows by 256 weight
// rows (64 per wave), main-loop step 64 along k. Backward: work-group = 4 or 8 waves, tile =
// 32*MB token rows by 64 columns of dX per wave, main-loop step 64 along the contraction
// (weight rows).
//
// Split-K: with splits > 1 each work-group writes its fp32 partial sums (row-major, one slab of
// m x ncols floats per split) and splitk_reduce_kernel adds the slabs in split order (the same
// order on every run) and applies the epilogue.

constexpr int kGemmThreads = 256;
constexpr int kFwdBN = 256;
constexpr int kFwdBK = 64;
constexpr int kBwdBC = 64;
constexpr int kMaxGroups = DK_MAX_GROUPS;

struct FwdGroupDev {
    NF4Dev w;
    const _Float16* bias;
    const _Float16* lora_u;
    const _Float16* lora_b;
    _Float16* y;
    int64_t ldy;
    float lora_scale;
    int32_t tile_begin;  // first n-tile of this group in the launch's n-tile space
    int32_t col_begin;   // first column of this group in the partial slabs
};

struct FwdArgs {
    const _Float16* x;
    int64_t ldx;
    uint32_t x_bytes;
    int32_t m, k;
    int32_t ngroups, lora_rank;
    int32_t m_tiles, n_tiles, splits, ksteps, ksteps_per_split;
    int32_t nested;
    int32_t wide_stats;  // some group has blocksize 32 or k % 64 != 0: two statistics slots per lane
    int32_t ncols;       // columns of a partial slab (sum of the groups' n)
    float* partials;     // splits x m x ncols fp32 (splits > 1)
    // GLU mode: groups 0 (gate) and 1 (up) of one shape; a tile takes 128 rows of each and the
    // epilogue also writes h = fp16(silu(gate) up) (no split-K; narrow statistics; nested ones on
    // nf4_fwd8_kernel only)
    int32_t glu;
    _Float16* h;
    int64_t ldh;
    // work-group order of nf4_fwd8_kernel: column tiles fastest (1) or token tiles fastest (0)
    int32_t cols_first;
    FwdGroupDev g[kMaxGroups];
};

struct BwdGroupDev {
    NF4Dev w;
    const _Float16* dy;
    int32_t lddy;
    uint32_t dy_bytes;
    const _Float16* lora_gu;
    const _Float16* lora_a;
    const uint8_t* lora_keep;  // dropout keep bits of the LoRA branch's input [m, k / 8], or null
    float lora_keep_scale;     // 1 / (1 - p)
    int32_t step_begin;  // first contraction step of this group
    int32_t nsteps;
};

struct BwdArgs {
    void* dx;
    int64_t lddx;
    int32_t m, k;
    int32_t ngroups, lora_rank;
    int32_t m_tiles, k_tiles, splits, csteps, csteps_per_split;
    int32_t dx_fp32;
    int32_t nested;
    int32_t wide_stats;  // some group has blocksize 32 or k % 64 != 0: one scale per 32 columns
    float* partials;  // splits x m x k fp32 (splits > 1)
    // SwiGLU mode (no split-K): no dX; with G = fp16(dY.W), dgate / dup from G, gate and up
    // (may alias gate / up)
    int32_t swiglu;
    const _Float16* gate;
    const _Float16* up;
    int64_t ldgu;
    _Float16* dgate;
    _Float16* dup;
    int64_t ldd;
    // work-group order of nf4_bwd8_kernel: column tiles fastest (1) or token tiles fastest (0)
    int32_t cols_first;
    // the launch covers output column tiles k_tile0 .. k_tile0 + k_tiles - 1 (a remainder launch
    // starts past the tiles of a first one); split-K partial slabs are pcols columns wide and
    // start at column 256 k_tile0
    int32_t k_tile0;
    int32_t pcols;
    BwdGroupDev g[kMaxGroups];
};

// Split-K epilogue: out_g[r, c - col_begin_g] = round(sum_s partial[s, r, c] + bias_g[...]).
struct ReduceOut {
    void* out;
    int64_t ld;
    const _Float16* bias;
    int32_t col_begin, ncols;
};

struct ReduceArgs {
    const float* partials;
    int64_t slab;  // floats per split slab (m * ncols)
    int32_t splits, m, ncols, nout;
    int32_t out_fp32;
    ReduceOut o[kMaxGroups];
    // RoPE epilogue of the groups whose bit is set in rope_mask (fp16 out only): the group's
    // output, rounded to fp16, is rotated with cos / sin (fp32 [m, head_dim]) as
    // x cos + rotate_half(x) sin in fp32 and stored head-major to rope_out[g]
    // [n_g / head_dim, m, head_dim] instead of o[g].out
    int32_t rope_mask;
    int32_t head_dim;
    const float* cos;
    const float* sin;
    _Float16* rope_out[kMaxGroups];
};

// Launch plans (tile size, split-K factor) chosen by the host.
struct GemmPlan {
    int mt;        // 32-row token blocks per tile
    int waves;     // waves per work-group (forward: 4 = nf4_fwd_kernel, 8 = nf4_fwd8_kernel;
                   // backward: nf4_bwd8_kernel's 8 of 32 output columns)
    int m_tiles;
    int n_tiles;   // output column tiles (fwd: weight rows / 256; bwd: k / 256)
    int steps;     // main-loop steps over the whole contraction
    int splits;
    int steps_per_split;
    int64_t partial_floats;  // fp32 partial slabs (splits > 1)
    int row_tiles;           // nf4_skinny_kernel: 16-row tiles per work-group (4 to 6)
};

hipError_t launch_fwd(const FwdArgs& a, int mb, int grid, hipStream_t s);
// GEMV for launches of at most kGemvMaxM token rows (no LoRA terms, no GLU epilogue, no split);
// a work-group computes 1, 2 or 4 of them
constexpr int kGemvMaxM = 8;
// a: the groups' tile_begin fields become their first work-group. gemv_fits: the GEMV takes
// m token rows at this contraction length.
hipError_t launch_gemv(FwdArgs& a, hipStream_t s);
bool gemv_fits(int64_t m, int64_t k);
// CUs of the current device (256 where no device answers)
int device_cus();
// waves per work-group of a GEMV launch (k must fit: gemv_fits)
int gemv_waves(int64_t m, int64_t k, int64_t nrows);
// Forward launches of few token rows (no LoRA terms, no GLU epilogue): nf4_skinny_kernel. A
// work-group owns 16 * row_tiles weight rows (row_tiles 4 to 6); a.splits work-groups share them
// along the contraction, each covering a.ksteps_per_split 128-wide super-steps; g[].tile_begin =
// each group's first row group. splits > 1: fp32 partial slabs, then splitk_reduce_kernel.
constexpr int kSkinnyMaxM = 32;
hipError_t launch_skinny(const FwdArgs& a, int row_tiles, int grid, hipStream_t s);
// 8-wave forward kernel (32 weight rows x 32*mb tokens per wave), mb = 8 or 9
hipError_t launch_fwd8(const FwdArgs& a, int mb, int grid, hipStream_t s);
// 8-wave input-gradient kernel (32 output columns x 32*mb tokens per wave), mb = 2, 4, 7 or 8;
// the SwiGLU epilogue with mb <= 4
hipError_t launch_bwd8(const BwdArgs& a, int mb, int grid, hipStream_t s);
hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s);

// LoRA and SwiGLU helpers.
// x: fp16 or fp32 (x32) [m, ldx]; keep: packed dropout bits [m, k / 8] with keep_scale a device
// fp32 scalar, or null (no dropout)
// Several branches (the q and v adapters of one layer) share a launch of each product: every
// branch takes its own range of work-groups, which compute what a launch of that branch alone
// computes, in the same order.
constexpr int kLoraMaxBranches = 4;
struct LoraBranch {
    const void* x;           // the branch input (fp16, or fp32 with x32), [m, ldx]
    const uint8_t* keep;     // packed dropout bits [m, k / 8] or null
    const float* keep_scale; // device scalar 1 / (1 - p) with keep
    const _Float16* a;       // A [rank, k] (down: U = X.A^T)
    _Float16* u;             // U [m, rank]: written by the down product, read by the backward
    const _Float16* dy;      // backward: dY [m, n], row stride lddy
    const _Float16* b;       // backward: B [n, rank]
    _Float16* gu;            // backward: GU [m, rank]
    float* da;               // backward: dA fp32 [rank, k] or null
    float* db;               // backward: dB fp32 [n, rank] or null
    int64_t ldx, lddy, n;
    float scale;             // backward: the LoRA scaling s
    bool x32;
};
// All branches share m, k and the rank; a launch per kind of input (fp16 / fp32, with or without
// dropout) where they differ.
hipError_t launch_lora_down(const LoraBranch* br, int nbr, int64_t m, int64_t k, int rank, hipStream_t s);
hipError_t launch_lora_bwd(const LoraBranch* br, int nbr, int64_t m, int64_t k, int rank, hipStream_t s);
hipError_t launch_lora_keep_pack(const uint8_t* kq, const uint8_t* kv, uint8_t* bq, uint8_t* bv,
                                 int64_t nbytes, hipStream_t s);
hipError_t launch_lora_dropout_inputs(const void* x, bool x32, const uint8_t* bq, const uint8_t* bv,
                                      const float* sq, const float* sv, _Float16* xq, _Float16* xv,
                                      int64_t nbytes, hipStream_t s);
hipError_t launch_lora_input_grad(const _Float16* gq, const _Float16* gv, const uint8_t* bq, const uint8_t* bv,
                                  float sq, float sv, float* out, int64_t nbytes, hipStream_t s);
hipError_t launch_lora_up(const _Float16* gu, const _Float16* a, int rank, _Float16* out, int64_t m, int64_t k,
                          hipStream_t s);
// RoPE of the attention inputs (rope.hip): q [T, hq*d] (+ LoRA) and k [T, hk*d] token-major in,
// head-major [h, T, d] out; backward the transpose.
struct RopeArgs {
    const _Float16* q_base;
    const _Float16* q_lora;  // may be null
    const _Float16* k;
    int64_t ldq, ldl, ldk;
    const float* cos;        // fp32 [T, d]
    const float* sin;
    _Float16* q_out;
    _Float16* k_out;
    const _Float16* grad_q;  // head-major
    const _Float16* grad_k;
    _Float16* dq;            // token-major
    _Float16* dk;
    int64_t lddq, lddk;
    int64_t n_tok;
    int32_t hq, hk, d;
};
hipError_t launch_rope(const RopeArgs& a, bool backward, hipStream_t s);

// Let `fn` launch with `bytes` of dynamic LDS on the current device (hipFuncSetAttribute once per
// device and kernel; thread-safe). Needed above 64 KB.
hipError_t allow_dynamic_lds(const void* fn, size_t bytes);

// diagnostics
hipError_t launch_mfma_peak(int64_t work_groups, int iters, float* out, hipStream_t s);
hipError_t launch_hbm_probe(const void* src, void* dst, int64_t bytes, int mode, float* sums, hipStream_t s);
hipError_t launch_swiglu_fwd(const _Float16* g, const _Float16* u, _Float16* o, int64_t n,
                             hipStream_t s);
hipError_t launch_swiglu_bwd(const _Float16* gr, const _Float16* g, const _Float16* u,
                             _Float16* dg, _Float16* du, int64_t n, hipStream_t s);

}  // namespace dk
