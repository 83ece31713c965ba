// Kernel argument blocks and launch helpers shared by the C ABI (capi.hip) and the kernels.
#pragma once

#include "nf4_device.h"

namespace dk {

constexpr int kDequantThreads = 256;
constexpr int kMaxDequantBatch = 8;
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

// ------------------------------------------------------------------------------------------
// Fused dequant x GEMM. One work-group = 4 waves. Forward tile: 32*MB rows of X by 256 weight
// rows (64 per wave); main-loop step 64 along k. Backward tile: 16*MT rows of dY by 256 columns
// of dX (64 per wave); main-loop step 64 along the contraction (weight rows).

constexpr int kGemmThreads = 256;
constexpr int kFwdBN = 256;
constexpr int kFwdBK = 64;
constexpr int kBwdBN = 256;
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
};

struct FwdArgs {
    const _Float16* x;
    int64_t ldx;
    uint32_t x_bytes;
    int32_t m, k;
    int32_t ngroups, lora_rank;
    int32_t m_tiles, n_tiles, splits, ksteps, ksteps_per_split;
    int32_t nested;
    int32_t wide_stats;  // some group has blocksize 32: two statistics slots per lane
    float* partials;
    uint32_t partial_bytes;
    int32_t* counters;
    FwdGroupDev g[kMaxGroups];
};

struct BwdGroupDev {
    NF4Dev w;
    const _Float16* dy;
    int64_t lddy;
    uint32_t dy_bytes;
    const _Float16* lora_gu;
    const _Float16* lora_a;
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
    float* partials;
    uint32_t partial_bytes;
    int32_t* counters;
    BwdGroupDev g[kMaxGroups];
};

// Launch plans (tile size, split-K factor) chosen by the host.
struct GemmPlan {
    int mt;        // 16-row blocks per tile (tile rows = 16 * mt)
    int m_tiles;
    int n_tiles;   // output column tiles (fwd: weight rows / 256; bwd: k / 256)
    int steps;     // main-loop steps over the whole contraction
    int splits;
    int steps_per_split;
    int64_t partial_floats;  // fp32 partial-tile storage
    int counters;            // tile counters
};

hipError_t launch_fwd(const FwdArgs& a, int mb, int grid, hipStream_t s);
hipError_t launch_bwd(const BwdArgs& a, int mt, int grid, hipStream_t s);

// LoRA and SwiGLU helpers.
hipError_t launch_lora_down(const _Float16* x, int64_t m, int64_t k, int64_t ldx, const _Float16* a,
                            int rank, _Float16* u, hipStream_t s);
hipError_t launch_lora_bwd(const _Float16* dy, int64_t lddy, const _Float16* u, const _Float16* x,
                           int64_t ldx, const _Float16* b, int64_t m, int64_t n, int64_t k, int rank,
                           float scale, _Float16* gu, float* da, float* db, hipStream_t s);
hipError_t launch_swiglu_fwd(const _Float16* g, const _Float16* u, _Float16* o, int64_t n,
                             hipStream_t s);
hipError_t launch_swiglu_bwd(const _Float16* gr, const _Float16* g, const _Float16* u,
                             _Float16* dg, _Float16* du, int64_t n, hipStream_t s);

}  // namespace dk
