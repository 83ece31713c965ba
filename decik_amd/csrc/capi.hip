// C ABI (include/decik_nf4.h): argument checks, launch planning and launches.
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <set>
#include <tuple>
#include <unordered_map>
#include <string>

#include "dk_internal.h"

namespace dk {
namespace {

thread_local std::string g_error;

int fail(const std::string& msg) {
    g_error = msg;
    return 1;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

int log2_exact(int64_t v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int s = 0;
    while ((int64_t(1) << s) < v) ++s;
    return s;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int to_dev(const dk_nf4_weight* w, NF4Dev* d, const char* who) {
    if (w == nullptr) return fail(std::string(who) + ": null weight descriptor");
    const bool empty = w->n * w->k == 0;
    if (!empty && (w->packed == nullptr || w->absmax == nullptr || w->code == nullptr))
        return fail(std::string(who) + ": packed, absmax and code must be set");
    if (w->n < 0 || w->k < 0 || ((w->n * w->k) & 1))
        return fail(std::string(who) + ": n*k must be even and non-negative");
    if (w->blocksize < 2 || (w->blocksize & 1))
        return fail(std::string(who) + ": blocksize must be even and >= 2");
    if (w->nested && !empty) {
        if (w->absmax2 == nullptr || w->code2 == nullptr || w->offset == nullptr || w->blocksize2 < 1)
            return fail(std::string(who) + ": nested weights need absmax2, code2, offset, blocksize2");
    }
    d->packed = w->packed;
    d->absmax8 = w->nested ? static_cast<const uint8_t*>(w->absmax) : nullptr;
    d->absmaxf = w->nested ? nullptr : static_cast<const float*>(w->absmax);
    d->absmax2 = w->absmax2;
    d->code2 = w->code2;
    d->offset = w->offset;
    d->code = w->code;
    d->n = w->n;
    d->k = w->k;
    d->blocksize = w->blocksize;
    d->blocksize2 = w->nested ? w->blocksize2 : 256;
    d->bs_shift = log2_exact(w->blocksize);
    d->bs2_shift = log2_exact(d->blocksize2);
    const int64_t n_el = w->n * w->k;
    const int64_t n_blocks = (n_el + w->blocksize - 1) / w->blocksize;
    const int64_t packed = n_el / 2;
    const int64_t amax = w->nested ? n_blocks : 4 * n_blocks;
    const int64_t amax2 = w->nested ? 4 * ((n_blocks + d->blocksize2 - 1) / d->blocksize2) : 0;
    auto clamp32 = [](int64_t v) { return (uint32_t)(v < INT32_MAX ? v : INT32_MAX); };
    d->packed_bytes = clamp32(packed);
    d->absmax_bytes = clamp32(amax);
    d->absmax2_bytes = clamp32(amax2);
    return 0;
}

// The fused GEMMs index with 32-bit byte offsets and shift-only block arithmetic.
int gemm_weight_ok(const dk_nf4_weight& w, const char* who) {
    if (w.n * w.k / 2 >= INT32_MAX) return fail(std::string(who) + ": weight larger than 2^31 bytes");
    if (w.blocksize % 32 != 0 || log2_exact(w.blocksize) < 0)
        return fail(std::string(who) + ": blocksize must be a power of two >= 32");
    if (w.nested && log2_exact(w.blocksize2) < 0)
        return fail(std::string(who) + ": blocksize2 must be a power of two");
    // the kernels advance block indices by whole 64-row / 64-column steps
    if ((64 * w.k) % w.blocksize != 0) return fail(std::string(who) + ": blocksize must divide 64 * k");
    if (w.n > INT32_MAX / 2) return fail(std::string(who) + ": too many weight rows");
    return 0;
}

// CUs of the current device (cached per device; 256, MI355X's count, when no device answers:
// the planner also runs on hosts without a GPU).
int num_cus() {
    constexpr int kDevs = 64;
    static int cus[kDevs] = {};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevs) return 256;
    thread_local int t_dev = -1, t_cus = 0;  // this thread's last device: no lock on the planner's hot path
    if (dev == t_dev) return t_cus;
    std::lock_guard<std::mutex> lock(mu);
    t_dev = dev;
    if (cus[dev] == 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
            cus[dev] = prop.multiProcessorCount;
        else
            cus[dev] = 256;
    }
    t_cus = cus[dev];
    return cus[dev];
}

// Plans are pure functions of their arguments, the device's CU count and the tuning variables
// (DECIK_FWD_PLAN, DECIK_BWD_PLAN, DECIK_SMALL_M), and a plan evaluates hundreds of (variant,
// splits) estimates: every launch and workspace query would repeat them. PlanMemo keeps them per
// argument list (cleared past 4096 entries).
template <typename P>
class PlanMemo {
  public:
    template <typename F>
    P get(const std::string& key, F compute) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            const auto it = map_.find(key);
            if (it != map_.end()) return it->second;
        }
        const P p = compute();
        std::lock_guard<std::mutex> lock(mu_);
        if (map_.size() >= 4096) map_.clear();
        map_.emplace(key, p);
        return p;
    }

  private:
    std::mutex mu_;
    std::unordered_map<std::string, P> map_;
};

std::string plan_key(char kind, std::initializer_list<int64_t> vals, const int64_t* ns, int ngroups) {
    std::string key(1, kind);
    auto add = [&key](int64_t v) { key.append(reinterpret_cast<const char*>(&v), sizeof v); };
    for (const int64_t v : vals) add(v);
    for (int g = 0; g < ngroups; ++g) add(ns[g]);
    add(num_cus());
    for (const char* var : {"DECIK_FWD_PLAN", "DECIK_BWD_PLAN", "DECIK_SMALL_M"}) {
        const char* v = std::getenv(var);
        key.push_back('|');
        if (v != nullptr) key.append(v);
    }
    return key;
}

int pad8(int g) { return (g + 7) & ~7; }

// ---- planning -----------------------------------------------------------------------------

// Launch planning. A plan picks the kernel variant (token rows per tile) and the number of
// contraction splits by an estimate of the launch time:
//   full rounds of resident work-groups x steps per split x step time (all slots busy)
//   + a last, partial round: a full round's time if some CU holds two of its work-groups,
//     else faster (one work-group per CU)
//   + the split-K cost, proportional to the fp32 partial tiles written and read back.
// Resident work-groups per CU and the step times are per-variant constants measured on MI355X
// (Qwen2.5-1.5B MLP launches at M = 830).
struct VariantCost {
    int rows_blocks;   // kernel template argument: token rows per tile / 32
    int waves;         // work-group waves (backward: 64 output columns each)
    int bn;            // output columns per tile
    int per_cu;        // resident work-groups per CU
    double step_us;    // one 64-wide contraction step of one work-group, every slot busy
    double lone;       // step time relative to step_us with one work-group per CU
};

constexpr double kPartialUsPerMB = 0.36;  // split-K: partial slabs written, then read and summed
constexpr double kReduceLaunchUs = 4.0;   // split-K: the reduction launch
// Forward split-K with few outputs: the reduction is a few thousand threads, each adding its
// outputs' splits in order, so every split lengthens a chain of dependent loads -- a cost per
// split that the slab bytes miss. Graph-replayed forwards at 33-512 tokens (7B q/o, k/v, qkv;
// 1.5B o, down; splits 2..28) fit 0.26 us per split; with it the plans of launches of at most
// 300K outputs split 2-4x less and run 3-20% faster. Larger reductions fill the GPU (the term
// made them pick smaller tiles and run up to 28% slower), and input-gradient launches with few
// work-groups are slower unsplit than the model says, so neither takes the term.
constexpr double kSplitUs = 0.26;
constexpr int64_t kSmallReduceOutputs = 300000;
constexpr int kRowUnit = 32;              // token rows per row block

// col_tiles: output column tiles of the launch for this variant's tile width.
double plan_time(const VariantCost& v, int64_t m, int64_t col_tiles, int64_t ncols, int steps,
                 int splits, bool split_chain) {
    const int64_t rows = (int64_t)kRowUnit * v.rows_blocks;
    const int64_t tiles = ((m + rows - 1) / rows) * col_tiles;
    const int64_t slots = (int64_t)num_cus() * v.per_cu;
    const int per = (steps + splits - 1) / splits;
    const int64_t wgs = tiles * splits;
    const int64_t full = wgs / slots, rem = wgs - full * slots;
    double t = (double)full * per * v.step_us;
    if (rem > num_cus()) {
        // some CU holds two work-groups of the last round: it takes a full round's time
        t += per * v.step_us;
    } else if (rem > 0) {
        // one work-group per CU at most: each runs faster than with a busy neighbour
        t += per * v.step_us * v.lone;
    }
    if (splits > 1) t += (double)splits * m * ncols * 4.0 * 1e-6 * kPartialUsPerMB + kReduceLaunchUs;
    if (splits > 1 && split_chain && m * ncols <= kSmallReduceOutputs) t += splits * kSplitUs;
    return t;
}

// Best (variant, splits) for a launch; col_tiles_of(v) gives the column tiles for variant v.
// max_partial_bytes: plans whose fp32 partial slabs exceed it are not considered.
// min_splits: plans with fewer splits are not considered (the RoPE epilogue lives in the split-K
// reduction), unless the contraction has fewer steps.
template <typename ColTiles>
const VariantCost* choose_plan(const VariantCost* vs, int nv, int64_t m, int64_t ncols, int steps,
                               ColTiles col_tiles_of, int* splits, int max_splits = 32,
                               int64_t max_partial_bytes = INT64_MAX, int min_splits = 1,
                               bool split_chain = false) {
    double best = 1e300;
    const VariantCost* pick = &vs[0];
    *splits = 1;
    for (int i = 0; i < nv; ++i) {
        const VariantCost& v = vs[i];
        const int max_s = steps < max_splits ? steps : max_splits;
        for (int s = min_splits <= max_s ? min_splits : 1; s <= (max_s > 0 ? max_s : 1); ++s) {
            const int per = steps > 0 ? (steps + s - 1) / s : 0;
            if (steps > 0 && (steps + per - 1) / per != s) continue;  // s splits must all get work
            if (s > 1 && (double)s * m * ncols * 4.0 > (double)max_partial_bytes) continue;
            const double t = plan_time(v, m, col_tiles_of(v), ncols, steps, s, split_chain);
            if (t < best * 0.999) {
                best = t;
                pick = &v;
                *splits = s;
            }
        }
    }
    return pick;
}

// Work-group order of the eight-wave kernels. Consecutive logical work-groups run on one XCD
// and share its L2: with token tiles fastest an XCD reads the weight columns of its tiles once
// and every token row, with column tiles fastest the reverse. Column tiles go first when there
// are many token tiles and the activations (2 bytes per token and contraction index) outweigh
// the packed weights (half a byte per output column and contraction index): measured on MI355X,
// 3-6% faster at M = 8192 for the 7B projections, 3% slower at M = 830 for the 1.5B MLP.
bool cols_first(int m_tiles, int64_t m, int64_t out_cols) { return m_tiles >= 8 && 4 * m > out_cols; }

// Split-K workspace: the fp32 partial slabs (splits x m x ncols), nothing else. Contents need not
// be initialised and are dead after the call.
int64_t workspace_bytes(const GemmPlan& p) { return p.splits > 1 ? p.partial_floats * 4 : 0; }

void no_split(GemmPlan& p) {
    p.splits = 1;
    p.steps_per_split = p.steps;
    p.partial_floats = 0;
}

// Tuning hook: DECIK_FWD_PLAN / DECIK_BWD_PLAN = "rows_blocks,splits[,waves[,columns]]" forces a
// plan (a compiled variant and 1 <= splits <= steps; waves and columns per tile default to the
// variant list's first match).
// Unset in normal use; read on every call so a sweep can change it between calls.
const VariantCost* plan_override(const char* var, const VariantCost* vs, int nv, int steps, int* splits) {
    const char* v = std::getenv(var);
    if (v == nullptr || *v == 0) return nullptr;
    int a = 0, b = 0, w = 0, c = 0;
    const int got = std::sscanf(v, "%d,%d,%d,%d", &a, &b, &w, &c);
    if (got < 2 || b < 1 || b > (steps > 0 ? steps : 1)) return nullptr;
    for (int i = 0; i < nv; ++i)
        if (vs[i].rows_blocks == a && (got < 3 || vs[i].waves == w) && (got < 4 || vs[i].bn == c)) {
            *splits = b;
            return &vs[i];
        }
    return nullptr;
}

void finish_plan(GemmPlan& p, int64_t m, int64_t ncols) {
    p.steps_per_split = p.steps > 0 ? (p.steps + p.splits - 1) / p.splits : 0;
    if (p.steps > 0) p.splits = (p.steps + p.steps_per_split - 1) / p.steps_per_split;
    p.partial_floats = p.splits > 1 ? (int64_t)p.splits * m * ncols : 0;
    if (p.partial_floats * 4 >= (int64_t(1) << 34)) no_split(p);  // 16 GiB: never worth it
}

// waves 4: nf4_fwd_kernel (two work-groups per CU for mb <= 4); waves 8: nf4_fwd8_kernel (one
// work-group of eight waves per CU, 32*mb tokens x 256 weight rows)
// (nf4_fwd_kernel<8> and nf4_bwd8_kernel<9> are not offered: they spilled registers to scratch)
constexpr VariantCost kFwdVariants[] = {{1, 4, kFwdBN, 3, 2.35, 0.65},
                                       {2, 4, kFwdBN, 2, 2.23, 0.65},
                                       {4, 4, kFwdBN, 2, 3.10, 0.65},
                                       {2, 8, kFwdBN, 1, 1.00, 0.80},
                                       {4, 8, kFwdBN, 1, 1.40, 0.80},
                                       {7, 8, kFwdBN, 1, 2.00, 0.90},
                                       {8, 8, kFwdBN, 1, 2.25, 0.90},
                                       {9, 8, kFwdBN, 1, 2.45, 0.90}};
constexpr int kNumFwdVariants = sizeof(kFwdVariants) / sizeof(kFwdVariants[0]);
// nf4_bwd8_kernel: eight waves of 32 output columns (256-column tiles); its SwiGLU epilogue
// exists for rows_blocks <= 4, which come first.
constexpr VariantCost kBwdVariants[] = {{2, 8, 256, 1, 1.00, 1.0},
                                       {4, 8, 256, 1, 1.75, 0.90},
                                       {7, 8, 256, 1, 2.10, 0.90},
                                       {8, 8, 256, 1, 2.25, 0.90}};
constexpr int kNumBwdVariants = sizeof(kBwdVariants) / sizeof(kBwdVariants[0]);
constexpr int kNumBwdSwigluVariants = 2;  // rows_blocks 2 and 4
static_assert(kBwdVariants[kNumBwdSwigluVariants - 1].rows_blocks == 4 &&
              kBwdVariants[kNumBwdSwigluVariants].rows_blocks > 4, "SwiGLU-capable variants first");

// The eight-wave variants come last: nf4_fwd8_kernel advances its load descriptors by whole
// steps, so it needs k % 64 == 0 and blocks that do not straddle rows (k % blocksize == 0).
constexpr int kNumFwd4Variants = 3;
static_assert(kFwdVariants[kNumFwd4Variants - 1].waves == 4 && kFwdVariants[kNumFwd4Variants].waves == 8,
              "four-wave variants first");

// glu: two weights of ns[0] rows, a tile takes 128 rows of each; never split (the epilogue
// needs the finished sums). fwd8_ok: the eight-wave kernel may run (see above). fwd4_ok: the
// four-wave kernel may run (not for GLU launches on nested statistics: its GLU waves mix the two
// weights' rows and keep one code2 table).
GemmPlan plan_fwd_compute(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool glu, bool fwd8_ok,
                          bool no_split, int min_splits, bool fwd4_ok) {
    GemmPlan p{};
    p.steps = (int)((k + kFwdBK - 1) / kFwdBK);
    p.n_tiles = 0;
    int64_t ncols = 0;
    if (glu) {
        p.n_tiles = (int)((ns[0] + kFwdBN / 2 - 1) / (kFwdBN / 2));
        ncols = 2 * ns[0];
    } else {
        for (int g = 0; g < ngroups; ++g) {
            p.n_tiles += (int)((ns[g] + kFwdBN - 1) / kFwdBN);
            ncols += ns[g];
        }
    }
    const int nv = fwd8_ok ? kNumFwdVariants : kNumFwd4Variants;
    const int v0 = fwd4_ok || !fwd8_ok ? 0 : kNumFwd4Variants;  // the first variant offered
    const VariantCost* v = plan_override("DECIK_FWD_PLAN", kFwdVariants + v0, nv - v0, p.steps, &p.splits);
    if (v != nullptr && (glu || no_split)) p.splits = 1;
    if (v != nullptr && p.splits < min_splits && p.steps >= min_splits) v = nullptr;
    if (v == nullptr) {
        const int64_t nt = p.n_tiles;
        v = choose_plan(kFwdVariants + v0, nv - v0, m, ncols, p.steps, [nt](const VariantCost&) { return nt; },
                        &p.splits, (glu || no_split) ? 1 : 32, INT64_MAX, min_splits, true);
    }
    p.mt = v->rows_blocks;
    p.waves = v->waves;
    p.m_tiles = (int)((m + kRowUnit * p.mt - 1) / (kRowUnit * p.mt));
    finish_plan(p, m, ncols);
    return p;
}

// swiglu: the SwiGLU epilogue of dk_nf4_linear_bwd_swiglu (never split; the variants that have it).
// max_partial_bytes: the split-K partial slabs must fit in that many bytes.
GemmPlan plan_bwd_compute(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool swiglu, bool no_split,
                          int64_t max_partial_bytes) {
    GemmPlan p{};
    p.steps = 0;
    for (int g = 0; g < ngroups; ++g) p.steps += (int)((ns[g] + kBwdBC - 1) / kBwdBC);
    const int nv = swiglu ? kNumBwdSwigluVariants : kNumBwdVariants;
    no_split = no_split || swiglu;
    const VariantCost* v = plan_override("DECIK_BWD_PLAN", kBwdVariants, nv, p.steps, &p.splits);
    if (v != nullptr && no_split) p.splits = 1;
    if (v != nullptr && p.splits > 1 && (double)p.splits * m * k * 4.0 > (double)max_partial_bytes) v = nullptr;
    if (v == nullptr)
        v = choose_plan(kBwdVariants, nv, m, k, p.steps,
                        [k](const VariantCost& c) { return (k + c.bn - 1) / c.bn; }, &p.splits,
                        no_split ? 1 : 32, max_partial_bytes);
    p.mt = v->rows_blocks;
    p.waves = v->waves;
    p.n_tiles = (int)((k + v->bn - 1) / v->bn);
    p.m_tiles = (int)((m + kRowUnit * p.mt - 1) / (kRowUnit * p.mt));
    finish_plan(p, m, k);
    return p;
}

GemmPlan plan_fwd(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool glu, bool fwd8_ok,
                  bool no_split = false, int min_splits = 1, bool fwd4_ok = true) {
    static PlanMemo<GemmPlan> memo;
    return memo.get(plan_key('f', {m, k, glu, fwd8_ok, no_split, min_splits, fwd4_ok}, ns, ngroups),
                    [&] { return plan_fwd_compute(m, k, ns, ngroups, glu, fwd8_ok, no_split, min_splits, fwd4_ok); });
}

GemmPlan plan_bwd(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool swiglu, bool no_split = false,
                  int64_t max_partial_bytes = INT64_MAX) {
    static PlanMemo<GemmPlan> memo;
    return memo.get(plan_key('b', {m, k, swiglu, no_split, max_partial_bytes}, ns, ngroups),
                    [&] { return plan_bwd_compute(m, k, ns, ngroups, swiglu, no_split, max_partial_bytes); });
}

// Input-gradient launches whose tiles overrun whole rounds of resident work-groups by a partial
// round (the 7B down projection at 830 tokens: 296 tiles of 224 x 256 for 256 CUs) leave most
// CUs idle in that last round. The column tiles that fill whole rounds then run as one launch
// (unsplit), and the remaining output columns as a second launch planned on its own -- usually
// split over every CU, then reduced -- when the time model says two launches are faster.
struct BwdParts {
    GemmPlan a;      // the whole launch, or the first part: column tiles 0 .. a.n_tiles - 1
    GemmPlan b;      // the second part (two only): column tiles kt_b .., k - 256 kt_b columns
    int kt_b = 0;
    bool two = false;
};

constexpr double kSecondLaunchUs = 3.0;  // a second GEMM launch and its gap
constexpr double kTwoPartGain = 0.95;    // two launches only for an estimated gain of 5% or more

const VariantCost* bwd_variant(int mt) {
    for (int i = 0; i < kNumBwdVariants; ++i)
        if (kBwdVariants[i].rows_blocks == mt) return &kBwdVariants[i];
    return &kBwdVariants[0];
}

BwdParts plan_bwd_parts_compute(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool swiglu,
                                int64_t max_partial_bytes) {
    BwdParts r;
    r.a = plan_bwd(m, k, ns, ngroups, swiglu, false, max_partial_bytes);
    const char* forced = std::getenv("DECIK_BWD_PLAN");
    if (swiglu || (forced != nullptr && *forced != 0)) return r;
    const int64_t slots = num_cus();  // one work-group per CU
    const int64_t tiles = (int64_t)r.a.m_tiles * r.a.n_tiles;  // unsplit
    if (tiles <= slots || tiles % slots == 0) return r;
    const int kt_a = (int)((tiles / slots) * slots / r.a.m_tiles);  // whole column tiles of the full rounds
    if (kt_a < 1 || kt_a >= r.a.n_tiles) return r;
    const int64_t k_b = k - (int64_t)kt_a * 256;
    const GemmPlan b = plan_bwd(m, k_b, ns, ngroups, false, false, max_partial_bytes);
    const VariantCost* va = bwd_variant(r.a.mt);
    const VariantCost* vb = bwd_variant(b.mt);
    const double t_one = plan_time(*va, m, r.a.n_tiles, k, r.a.steps, r.a.splits, false);
    const double t_two = plan_time(*va, m, kt_a, (int64_t)kt_a * 256, r.a.steps, 1, false) +
                         plan_time(*vb, m, b.n_tiles, k_b, b.steps, b.splits, false) + kSecondLaunchUs;
    if (t_two >= kTwoPartGain * t_one) return r;
    no_split(r.a);
    r.a.n_tiles = kt_a;
    r.b = b;
    r.kt_b = kt_a;
    r.two = true;
    return r;
}

int64_t workspace_bytes(const BwdParts& p) {
    return std::max(workspace_bytes(p.a), p.two ? workspace_bytes(p.b) : (int64_t)0);
}

BwdParts plan_bwd_parts(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool swiglu,
                        int64_t max_partial_bytes = INT64_MAX) {
    static PlanMemo<BwdParts> memo;
    return memo.get(plan_key('p', {m, k, swiglu, max_partial_bytes}, ns, ngroups),
                    [&] { return plan_bwd_parts_compute(m, k, ns, ngroups, swiglu, max_partial_bytes); });
}

// nf4_skinny_kernel (forward, m <= kSkinnyMaxM): row groups of 4 tiles of 16 rows, or of 5 or 6
// where that is the fewest that keep the row groups to one per CU: a weight of more 64-row groups
// than CUs would otherwise run a second round of only its left-over groups, as long as the first
// (7B gate: 296 groups of 64 rows on 256 CUs, 237 of 80); contraction splits while the launch
// still has at most one work-group per CU and every split keeps at least two 128-wide
// super-steps per wave (16 per work-group). no_split: a single pass (no workspace).
constexpr int kSkinnyStep = 128, kSkinnyWaves = 8;
int64_t skinny_row_groups(const int64_t* ns, int ngroups, int row_tiles) {
    int64_t rgroups = 0;
    for (int g = 0; g < ngroups; ++g) rgroups += (ns[g] + 16 * row_tiles - 1) / (16 * row_tiles);
    return rgroups;
}
int skinny_row_tiles(const int64_t* ns, int ngroups) {
    for (int rt = 4; rt <= 6; ++rt)
        if (skinny_row_groups(ns, ngroups, rt) <= num_cus()) return rt;
    return 4;
}
GemmPlan plan_skinny_compute(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool no_split) {
    GemmPlan p{};
    p.row_tiles = skinny_row_tiles(ns, ngroups);
    const int64_t rgroups = skinny_row_groups(ns, ngroups, p.row_tiles);
    int64_t ncols = 0;
    for (int g = 0; g < ngroups; ++g) ncols += ns[g];
    p.steps = (int)((k + kSkinnyStep - 1) / kSkinnyStep);
    // split the contraction as far as the work-groups still fit one per CU and every split keeps
    // at least two super-steps (all splits non-empty). Weights of few row groups (k/v) gain most
    // from the extra work-groups pulling them: graph-replayed forced splits at 8 and 24 tokens,
    // 7B k/v 10.4 / 12.4 us at 3 splits (the earlier rule: one super-step per wave, 8 a split)
    // -> 8.4 / 9.7 at 12, 7B q/o 11.9 / 14.0 at 3 -> 11.2 / 13.2 at 4, 1.5B q/o and k/v 10%
    // faster at 24 tokens with 6 splits than unsplit; the wide weights (7B gate, 1.5B gate) stay
    // unsplit
    p.splits = 1;
    for (int s = 2; !no_split && s <= 32 && s <= p.steps / 2 && rgroups * s <= num_cus(); ++s) {
        const int per = (p.steps + s - 1) / s;
        if ((p.steps + per - 1) / per == s) p.splits = s;
    }
    p.n_tiles = (int)rgroups;
    p.m_tiles = 1;
    p.mt = m <= 16 ? 1 : 2;
    p.waves = kSkinnyWaves;
    finish_plan(p, m, ncols);
    return p;
}

GemmPlan plan_skinny(int64_t m, int64_t k, const int64_t* ns, int ngroups, bool no_split = false) {
    static PlanMemo<GemmPlan> memo;
    return memo.get(plan_key('s', {m, k, no_split}, ns, ngroups),
                    [&] { return plan_skinny_compute(m, k, ns, ngroups, no_split); });
}

// Forward launches of at most kSkinnyMaxM token rows without LoRA terms or the GLU epilogue run
// the GEMV kernel (at most kGemvMaxM rows) or nf4_skinny_kernel, unless DECIK_FWD_PLAN forces an
// MFMA plan. Measured on Qwen2.5-7B shapes: at one row the GEMV is faster on every shape (gate
// 18 us against 25, q/o 10 against 16), and at two rows on all but the long contraction of down;
// from 3 rows on the skinny kernel wins on all but small weights (gemv_requested; 7B gate at 8
// rows: 28 us against 39 for the MFMA kernels). DECIK_SMALL_M = gemv / skinny forces one of them for launches both may take.
// Past 16 rows (two 16-token blocks a work-group), weights of more row groups than CUs (even at
// 6 tiles a group) go to the MFMA kernels: the skinny kernel's second round would hold few
// work-groups (7B gate, 296 groups of 64 rows: 38.8 / 39.6 us at 24 / 32 rows against 34.2 /
// 34.9 on 64-token MFMA tiles).
bool small_m_forward(int64_t m, bool glu, bool lora, const int64_t* ns, int ngroups) {
    if (glu || lora || m < 1 || m > kSkinnyMaxM) return false;
    const char* forced = std::getenv("DECIK_FWD_PLAN");
    if (forced != nullptr && *forced != 0) return false;
    if (m > 16 && skinny_row_groups(ns, ngroups, skinny_row_tiles(ns, ngroups)) > num_cus()) return false;
    return true;
}
bool gemv_requested(int64_t m, int64_t k, const int64_t* ns, int ngroups) {
    if (!gemv_fits(m, k)) return false;
    const char* v = std::getenv("DECIK_SMALL_M");
    if (v != nullptr && std::string(v) == "gemv") return true;
    if (v != nullptr && std::string(v) == "skinny") return false;
    if (m == 1) return true;
    // Two rows: the GEMV's second dot product per weight costs in proportion to the weight, the
    // small-M kernel hardly depends on the row count, so large launches take the small-M kernel.
    // Graph-replayed at two rows, GEMV against small-M kernel: 7B gate 21.3-21.6 against 17.4 us
    // (67.9M weights), 1.5B gate 8.1 against 8.8 (13.8M), 7B q/o 7.5 against 11.1 (12.8M); a
    // long contraction also favours the small-M kernel's split (7B down, k = 18944: 23.7 against
    // 35.1; the 1.5B down, k = 8960: 8.6 against 10.5 on the GEMV).
    int64_t weights = 0;
    for (int g = 0; g < ngroups; ++g) weights += ns[g] * k;
    // Long rows at two rows: up to 2^24 weights the GEMV still wins ([256, 20480] 8.2 against
    // 11.0 us, [1024, 16384] 9.0 against 11.7); the 7B down projection (67.9M) does not.
    if (m == 2) return weights < (int64_t(1) << 25) && (k <= 12288 || weights <= (int64_t(1) << 24));
    // 3-8 rows (a GEMV work-group computes 4; past 4 rows two work-groups share each weight row
    // range): small weights, whose small-M launches are bound by their fixed cost (a split and
    // its reduction launch). At 3-4 rows every weight of up to 2^24: graph-replayed, GEMV against
    // small-M kernel, us: 7B q/o 9.3 against 11.2, 1.5B gate 8.6 against 8.9, 1.5B down [1536,
    // 8960] 10.4-10.7 against 11.5, [2048, 8192] 10.1 against 12.3, [1024, 12288] 10.3-10.4
    // against 10.9-11.0, [896, 4864] 7.9-8.1 against 8.9-9.0 ([3584, 8192], 2^24.8 weights: 17.7
    // against 15.1-15.2). Past 4 rows, X of 4 rows must stay within 32 KB of LDS per work-group. Graph-replayed, GEMV against small-M kernel, us:
    // 1.5B k/v 4.3-4.5 / 6.3 against 8.1 / 8.3 at 3-4 / 8 rows, 1.5B q/o 4.9-5.0 / 6.9 against
    // 8.4-8.6, the 1.5B q/k/v launch 5.1-5.3 / 7.1 against 8.6-8.8, 7B k/v 5.2 against 9.2 at
    // 3-4 rows (11.6 against 9.4 at 8: X of 8 rows 56 KB); larger weights lose (7B q/o 11.9
    // against 11.0, 7B gate 26 against 18, at 3 rows).
    if (m <= 4) return weights <= (int64_t(1) << 24);
    return weights < (int64_t(1) << 23) && 4 * k * 2 <= 32768;
}



}  // namespace

int device_cus() { return num_cus(); }

hipError_t allow_dynamic_lds(const void* fn, size_t bytes) {
    static std::mutex mu;
    static std::set<std::tuple<int, const void*, size_t>> done;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({dev, fn, bytes})) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) done.insert({dev, fn, bytes});
    return e;
}

}  // namespace dk

using namespace dk;

extern "C" {

const char* dk_last_error(void) { return g_error.c_str(); }

int dk_version(void) { return 100; }

int dk_nf4_dequant_batched(const dk_nf4_weight* ws, uint16_t* const* outs, int count, void* stream) {
    g_error.clear();
    if (count < 0 || (count > 0 && (ws == nullptr || outs == nullptr)))
        return fail("dk_nf4_dequant_batched: bad arguments");
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int base = 0; base < count; base += kMaxDequantBatch) {
        DequantArgs a{};
        int wg = 0;
        a.count = 0;
        for (int i = 0; i < kMaxDequantBatch && base + i < count; ++i) {
            const dk_nf4_weight* w = &ws[base + i];
            if (to_dev(w, &a.w[i], "dk_nf4_dequant")) return 1;
            if (outs[base + i] == nullptr && w->n * w->k > 0) return fail("dk_nf4_dequant: null output");
            a.out[i] = outs[base + i];
            a.nbytes[i] = w->n * w->k / 2;
            a.wg_begin[i] = wg;
            const int64_t span = (int64_t)kDequantThreads * 4 * kDequantUnits;
            const int64_t g = (a.nbytes[i] + span - 1) / span;
            if (wg + g > INT32_MAX / 2) return fail("dk_nf4_dequant: tensor too large");
            wg += (int)g;
            a.fast[i] = (w->blocksize % 32 == 0) && log2_exact(w->blocksize) >= 0 &&
                        (!w->nested || log2_exact(w->blocksize2) >= 0) && aligned(w->packed, 16) &&
                        aligned(outs[base + i], 16);
            a.count = i + 1;
        }
        a.wg_begin[a.count] = wg;
        for (int i = a.count; i < kMaxDequantBatch; ++i) a.wg_begin[i] = wg;
        if (wg == 0) continue;
        hipLaunchKernelGGL(nf4_dequant_kernel, dim3(wg), dim3(kDequantThreads), 0, s, a);
        if (check_hip(hipGetLastError(), "dk_nf4_dequant launch")) return 1;
    }
    return 0;
}

int dk_nf4_dequant(const dk_nf4_weight* w, uint16_t* out, void* stream) {
    return dk_nf4_dequant_batched(w, &out, 1, stream);
}

int dk_nf4_block_scales(const dk_nf4_weight* w, float* scales, void* stream) {
    g_error.clear();
    NF4Dev d{};
    if (to_dev(w, &d, "dk_nf4_block_scales")) return 1;
    const int64_t nblocks = (w->n * w->k + w->blocksize - 1) / w->blocksize;
    if (nblocks > 0 && scales == nullptr) return fail("dk_nf4_block_scales: null output");
    if (nblocks / 256 >= INT32_MAX) return fail("dk_nf4_block_scales: tensor too large");
    return check_hip(launch_block_scales(d, nblocks, scales, static_cast<hipStream_t>(stream)),
                     "dk_nf4_block_scales launch");
}

int64_t dk_nf4_linear_fwd_workspace(int64_t m, int64_t k, const int64_t* ns, int ngroups) {
    if (ngroups < 1 || ngroups > kMaxGroups || ns == nullptr || m <= 0 || k <= 0) return 0;
    // the plan also depends on the block sizes (eight-wave kernel or not) and, for few token rows,
    // on LoRA terms (which keep such launches off the small-M kernel): cover every case
    const int64_t tiled = std::max(workspace_bytes(plan_fwd(m, k, ns, ngroups, false, true)),
                                   workspace_bytes(plan_fwd(m, k, ns, ngroups, false, false)));
    if (small_m_forward(m, false, false, ns, ngroups))
        return std::max(tiled, workspace_bytes(plan_skinny(m, k, ns, ngroups)));
    return tiled;
}

int dk_nf4_linear_plan(int backward, int64_t m, int64_t k, const int64_t* ns, int ngroups, int flags,
                       int blocksize, int32_t* out) {
    g_error.clear();
    if (ngroups < 1 || ngroups > kMaxGroups || ns == nullptr || out == nullptr || m <= 0 || k <= 0 ||
        blocksize < 32 || log2_exact(blocksize) < 0)
        return fail("dk_nf4_linear_plan: bad arguments");
    const bool glu = (flags & DK_PLAN_GLU) != 0, lora = (flags & DK_PLAN_LORA) != 0;
    const bool single = (flags & DK_PLAN_NO_SPLIT) != 0;
    GemmPlan p;
    int kernel;
    int launches = 1, splits_b = 0;
    if (backward) {
        if (single) {
            p = plan_bwd(m, k, ns, ngroups, glu, true);
        } else {
            const BwdParts parts = plan_bwd_parts(m, k, ns, ngroups, glu);
            p = parts.a;
            if (parts.two) {
                launches = 2;
                splits_b = parts.b.splits;
            }
        }
        kernel = 3;  // nf4_bwd8_kernel
    } else if (small_m_forward(m, glu, lora, ns, ngroups) && gemv_requested(m, k, ns, ngroups)) {
        p = GemmPlan{};
        int64_t nrows = 0;
        for (int g = 0; g < ngroups; ++g) nrows += ns[g];
        p.waves = gemv_waves(m, k, nrows);
        p.splits = 1;
        kernel = 4;  // nf4_gemv_kernel
    } else if (small_m_forward(m, glu, lora, ns, ngroups)) {
        p = plan_skinny(m, k, ns, ngroups, single);
        kernel = 5;  // nf4_skinny_kernel
    } else {
        p = plan_fwd(m, k, ns, ngroups, glu, k % 64 == 0 && k % blocksize == 0, single, 1,
                     !(glu && (flags & DK_PLAN_NESTED) != 0));
        kernel = p.waves == 8 ? 1 : 0;
    }
    out[0] = p.mt;
    out[1] = p.waves;
    out[2] = p.splits;
    out[3] = kernel;
    if (flags & DK_PLAN_PARTS) {
        out[4] = launches;
        out[5] = splits_b;
    }
    return 0;
}

int64_t dk_nf4_linear_bwd_workspace(int64_t m, int64_t k, const int64_t* ns, int ngroups) {
    if (ngroups < 1 || ngroups > kMaxGroups || ns == nullptr || m <= 0 || k <= 0) return 0;
    return workspace_bytes(plan_bwd_parts(m, k, ns, ngroups, false));
}

}  // extern "C"


// The RoPE epilogue of dk_nf4_linear_rope_fwd: groups in `mask` are rotated and stored head-major.
struct RopeSpec {
    const float* cos;
    const float* sin;
    int head_dim;
    int mask;
    uint16_t* const* out;
};

// The forward launch behind dk_nf4_linear_fwd, dk_nf4_glu_fwd and dk_nf4_linear_rope_fwd. h != NULL:
// GLU mode (two groups of one shape, plain narrow statistics; gate/up outputs optional).
// no_split: a single pass (no workspace). rope != NULL: at least two splits, the RoPE epilogue in
// the split-K reduction (the small-M kernels are not used).
static int linear_fwd_impl(const std::string& name, const uint16_t* x, int64_t m, int64_t k,
                           int64_t ldx, const dk_linear_fwd_group* groups, int ngroups, int lora_rank,
                           void* workspace, int64_t workspace_bytes_, void* stream, uint16_t* h,
                           int64_t ldh, bool no_split, const RopeSpec* rope = nullptr) {
    const bool glu = h != nullptr;
    if (ngroups < 1 || ngroups > kMaxGroups || groups == nullptr)
        return fail(name + ": need 1..4 groups");
    if (m < 0 || k <= 0 || (k % 32) != 0)
        return fail(name + ": k must be a positive multiple of 32");
    if (m > INT32_MAX / 2 || k > INT32_MAX / 2) return fail(name + ": m or k too large");
    // zero token rows: nothing is read or written, and row pointers may be NULL
    if (m > 0 && (x == nullptr || !aligned(x, 16) || ldx < k || (ldx % 8) != 0))
        return fail(name + ": x must be 16-byte aligned with ldx >= k, ldx % 8 == 0");
    if (lora_rank != 0 && lora_rank != 16 && lora_rank != 32)
        return fail(name + ": lora_rank must be 0, 16 or 32");
    FwdArgs a{};
    int64_t ns[kMaxGroups];
    int nested = -1;
    int tile = 0;
    int64_t ncols = 0;
    for (int g = 0; g < ngroups; ++g) {
        const dk_linear_fwd_group& G = groups[g];
        if (to_dev(&G.w, &a.g[g].w, name.c_str())) return 1;
        if (G.w.k != k) return fail(name + ": weight k differs from x");
        if (gemm_weight_ok(G.w, name.c_str())) return 1;
        if (!aligned(G.w.packed, 16)) return fail(name + ": packed weights must be 16-byte aligned");
        // every epilogue (direct stores, split-K partial slabs and their reduction, the GLU
        // tile) moves whole 8-column chunks: a chunk must lie wholly inside a group's rows
        if ((G.w.n % 8) != 0) return fail(name + ": weight rows must be a multiple of 8");
        if (nested >= 0 && nested != G.w.nested)
            return fail(name + ": all groups must be nested or all plain");
        nested = G.w.nested;
        // one statistics slot per row block and step needs 64-wide steps inside one block
        if (G.w.blocksize < 64 || k % 64 != 0) a.wide_stats = 1;
        const bool roped = rope != nullptr && ((rope->mask >> g) & 1);
        if (roped) {
            if ((m > 0 && (rope->out == nullptr || rope->out[g] == nullptr || !aligned(rope->out[g], 16))) ||
                G.w.n % rope->head_dim != 0)
                return fail(name + ": a rotated group needs a 16-byte aligned head-major output and n % head_dim == 0");
        } else if (m > 0 && ((G.y == nullptr && !glu) ||
                             (G.y != nullptr && (!aligned(G.y, 16) || G.ldy < G.w.n || (G.ldy % 8) != 0)))) {
            return fail(name + ": y must be 16-byte aligned with ldy >= n, ldy % 8 == 0");
        }
        if (G.lora_u != nullptr && (lora_rank == 0 || G.lora_b == nullptr))
            return fail(name + ": LoRA needs lora_rank > 0 and lora_b");
        if (G.lora_u != nullptr && (!aligned(G.lora_u, 16) || !aligned(G.lora_b, 16)))
            return fail(name + ": LoRA operands must be 16-byte aligned");
        if (G.lora_u != nullptr && (m * lora_rank * 2 >= INT32_MAX || G.w.n * lora_rank * 2 >= INT32_MAX))
            return fail(name + ": LoRA operands larger than 2^31 bytes");
        if (G.bias != nullptr && !aligned(G.bias, 16))
            return fail(name + ": bias must be 16-byte aligned");
        a.g[g].bias = reinterpret_cast<const _Float16*>(G.bias);
        a.g[g].lora_u = reinterpret_cast<const _Float16*>(G.lora_u);
        a.g[g].lora_b = reinterpret_cast<const _Float16*>(G.lora_b);
        a.g[g].lora_scale = G.lora_scale;
        a.g[g].y = reinterpret_cast<_Float16*>(G.y);
        a.g[g].ldy = G.ldy;
        a.g[g].tile_begin = tile;
        a.g[g].col_begin = (int32_t)ncols;
        tile += (int)((G.w.n + kFwdBN - 1) / kFwdBN);
        ncols += G.w.n;
        ns[g] = G.w.n;
    }
    if (glu && (ngroups != 2 || ns[0] != ns[1] || groups[0].w.nested != groups[1].w.nested || a.wide_stats ||
                groups[0].w.blocksize != groups[1].w.blocksize || k % 64 != 0))
        return fail(name + ": GLU mode needs two weights of one shape and statistics kind, blocksize >= 64, k % 64 == 0");
    if (m == 0 || tile == 0) return 0;
    if ((m - 1) * ldx + k >= INT32_MAX / 2) return fail(name + ": x too large");
    bool any_lora = false;
    for (int g = 0; g < ngroups; ++g) any_lora = any_lora || groups[g].lora_u != nullptr;
    if (rope == nullptr && small_m_forward(m, glu, any_lora, ns, ngroups)) {
        // few token rows, no LoRA terms: one pass over the packed weights
        a.x = reinterpret_cast<const _Float16*>(x);
        a.ldx = ldx;
        a.x_bytes = (uint32_t)(((m - 1) * ldx + k) * 2);
        a.m = (int)m;
        a.k = (int)k;
        a.ngroups = ngroups;
        a.nested = nested;
        a.ncols = (int32_t)ncols;
        if (ncols > INT32_MAX / 2) return fail(name + ": problem too large");
        const hipStream_t st = static_cast<hipStream_t>(stream);
        if (gemv_requested(m, k, ns, ngroups)) return check_hip(launch_gemv(a, st), "dk_nf4_linear_fwd GEMV launch");
        const GemmPlan p = plan_skinny(m, k, ns, ngroups, no_split);
        const int64_t need = workspace_bytes(p);
        if (need > 0 && (workspace == nullptr || workspace_bytes_ < need || !aligned(workspace, 256)))
            return fail(name + ": workspace too small (need " + std::to_string(need) + " bytes)");
        const int rows = 16 * p.row_tiles;
        int rg = 0;
        for (int g = 0; g < ngroups; ++g) {
            a.g[g].tile_begin = rg;
            rg += (int)((ns[g] + rows - 1) / rows);
        }
        a.splits = p.splits;
        a.ksteps = p.steps;
        a.ksteps_per_split = p.steps_per_split;
        if (need > 0) a.partials = static_cast<float*>(workspace);
        const int64_t wgs = (int64_t)rg * p.splits;
        if (wgs > INT32_MAX / 2) return fail(name + ": problem too large");
        if (check_hip(launch_skinny(a, p.row_tiles, (int)wgs, st), "dk_nf4_linear_fwd small-M launch")) return 1;
        if (p.splits <= 1) return 0;
        ReduceArgs r{};
        r.partials = a.partials;
        r.slab = m * ncols;
        r.splits = p.splits;
        r.m = (int)m;
        r.ncols = (int)ncols;
        r.nout = ngroups;
        r.out_fp32 = 0;
        for (int g = 0; g < ngroups; ++g)
            r.o[g] = ReduceOut{groups[g].y, groups[g].ldy, a.g[g].bias, a.g[g].col_begin, (int32_t)ns[g]};
        return check_hip(launch_splitk_reduce(r, st), "dk_nf4_linear_fwd split-K reduction");
    }
    bool fwd8_ok = k % 64 == 0;
    for (int g = 0; g < ngroups; ++g) fwd8_ok = fwd8_ok && k % groups[g].w.blocksize == 0;
    const GemmPlan p = plan_fwd(m, k, ns, ngroups, glu, fwd8_ok, no_split, rope != nullptr ? 2 : 1, !(glu && nested));
    if (rope != nullptr && p.splits < 2) return fail(name + ": the RoPE epilogue needs k >= 128 (two contraction steps)");
    const int64_t need = workspace_bytes(p);
    if (need > 0 && (workspace == nullptr || workspace_bytes_ < need || !aligned(workspace, 256)))
        return fail(name + ": workspace too small (need " + std::to_string(need) + " bytes)");
    a.x = reinterpret_cast<const _Float16*>(x);
    a.ldx = ldx;
    a.x_bytes = (uint32_t)(((m - 1) * ldx + k) * 2);
    a.m = (int)m;
    a.k = (int)k;
    a.ngroups = ngroups;
    a.lora_rank = lora_rank;
    a.m_tiles = p.m_tiles;
    a.n_tiles = p.n_tiles;
    a.splits = p.splits;
    a.ksteps = p.steps;
    a.ksteps_per_split = p.steps_per_split;
    a.nested = nested;
    a.ncols = (int32_t)ncols;
    a.glu = glu ? 1 : 0;
    a.h = reinterpret_cast<_Float16*>(h);
    a.ldh = ldh;
    a.cols_first = cols_first(p.m_tiles, m, ncols) ? 1 : 0;
    if (need > 0) a.partials = static_cast<float*>(workspace);
    const int64_t wgs = (int64_t)p.m_tiles * p.n_tiles * p.splits;
    if (wgs > INT32_MAX / 2 || ncols > INT32_MAX / 2) return fail(name + ": problem too large");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t le = p.waves == 8 ? launch_fwd8(a, p.mt, pad8((int)wgs), st) : launch_fwd(a, p.mt, pad8((int)wgs), st);
    if (check_hip(le, "dk_nf4_linear_fwd launch")) return 1;
    if (p.splits <= 1) return 0;
    ReduceArgs r{};
    r.partials = a.partials;
    r.slab = m * ncols;
    r.splits = p.splits;
    r.m = (int)m;
    r.ncols = (int)ncols;
    r.nout = ngroups;
    r.out_fp32 = 0;
    for (int g = 0; g < ngroups; ++g)
        r.o[g] = ReduceOut{groups[g].y, groups[g].ldy, a.g[g].bias, a.g[g].col_begin, (int32_t)ns[g]};
    if (rope != nullptr) {
        r.rope_mask = rope->mask;
        r.head_dim = rope->head_dim;
        r.cos = rope->cos;
        r.sin = rope->sin;
        for (int g = 0; g < ngroups; ++g)
            if ((rope->mask >> g) & 1) r.rope_out[g] = reinterpret_cast<_Float16*>(rope->out[g]);
    }
    return check_hip(launch_splitk_reduce(r, st), "dk_nf4_linear_fwd split-K reduction");
}


extern "C" {

int64_t dk_nf4_linear_rope_fwd_workspace(int64_t m, int64_t k, const int64_t* ns, int ngroups) {
    if (ngroups < 1 || ngroups > kMaxGroups || ns == nullptr || m <= 0 || k <= 0) return 0;
    return std::max(workspace_bytes(plan_fwd(m, k, ns, ngroups, false, true, false, 2)),
                    workspace_bytes(plan_fwd(m, k, ns, ngroups, false, false, false, 2)));
}

int dk_nf4_linear_rope_fwd(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                           const dk_linear_fwd_group* groups, int ngroups, int lora_rank, const float* cos,
                           const float* sin, int head_dim, int rope_mask, uint16_t* const* rope_out,
                           void* workspace, int64_t workspace_bytes_, void* stream) {
    g_error.clear();
    const char* who = "dk_nf4_linear_rope_fwd";
    if (head_dim <= 0 || head_dim % 16 != 0) return fail(std::string(who) + ": head_dim must be a positive multiple of 16");
    if (rope_mask <= 0 || rope_mask >= (1 << ngroups)) return fail(std::string(who) + ": rope_mask must name some of the groups");
    if (cos == nullptr || sin == nullptr) return fail(std::string(who) + ": cos and sin are required");
    const RopeSpec rope{cos, sin, head_dim, rope_mask, rope_out};
    return linear_fwd_impl(who, x, m, k, ldx, groups, ngroups, lora_rank, workspace, workspace_bytes_, stream,
                           nullptr, 0, false, &rope);
}


int dk_nf4_linear_fwd(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                      const dk_linear_fwd_group* groups, int ngroups, int lora_rank, void* workspace,
                      int64_t workspace_bytes_, void* stream) {
    g_error.clear();
    return linear_fwd_impl("dk_nf4_linear_fwd", x, m, k, ldx, groups, ngroups, lora_rank, workspace,
                           workspace_bytes_, stream, nullptr, 0, false);
}

int dk_nf4_glu_fwd(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                   const dk_linear_fwd_group* groups, int lora_rank, uint16_t* h, int64_t ldh,
                   void* stream) {
    g_error.clear();
    if (groups == nullptr || (h == nullptr && m > 0)) return fail("dk_nf4_glu_fwd: groups and h are required");
    const dk_nf4_weight& wg = groups[0].w;
    const dk_nf4_weight& wu = groups[1].w;
    if (wg.n != wu.n || wg.k != wu.k) return fail("dk_nf4_glu_fwd: gate and up shapes differ");
    const int64_t n = wg.n;
    if (m > 0 && (!aligned(h, 16) || ldh < n || (ldh % 8) != 0))
        return fail("dk_nf4_glu_fwd: h must be 16-byte aligned with ldh >= n, ldh % 8 == 0");
    const bool fused = wg.nested == wu.nested && wg.blocksize == wu.blocksize && wg.blocksize >= 64 &&
                       k % 64 == 0;
    if (fused)
        return linear_fwd_impl("dk_nf4_glu_fwd", x, m, k, ldx, groups, 2, lora_rank, nullptr, 0, stream,
                               h, ldh, true);
    // other statistics: gate and up by the grouped launch (one pass), then the SwiGLU kernel
    if (m > 0 && (groups[0].y == nullptr || groups[1].y == nullptr || groups[0].ldy != n ||
                  groups[1].ldy != n || ldh != n))
        return fail("dk_nf4_glu_fwd: narrow-block or mixed-statistics weights need gate and up outputs, all rows contiguous");
    if (linear_fwd_impl("dk_nf4_glu_fwd", x, m, k, ldx, groups, 2, lora_rank, nullptr, 0, stream, nullptr,
                        0, true))
        return 1;
    if (m == 0) return 0;
    return check_hip(launch_swiglu_fwd(reinterpret_cast<const _Float16*>(groups[0].y),
                                       reinterpret_cast<const _Float16*>(groups[1].y),
                                       reinterpret_cast<_Float16*>(h), m * n, static_cast<hipStream_t>(stream)),
                     "dk_nf4_glu_fwd SwiGLU");
}

}  // extern "C"

// SwiGLU backward fused into the epilogue of an input-gradient launch (dk_nf4_linear_bwd_swiglu).
struct SwigluBwdOut {
    const uint16_t* gate;
    const uint16_t* up;
    int64_t ldgu;
    uint16_t* dgate;
    uint16_t* dup;
    int64_t ldd;
};

// One input-gradient launch (plan p) over the output columns 256 kt0 .. 256 kt0 + cols - 1, then
// its split-K reduction into the same columns of dX. `a` carries everything but the tiling.
static int launch_bwd_part(BwdArgs a, const GemmPlan& p, int kt0, int64_t cols, void* workspace,
                           hipStream_t st) {
    a.m_tiles = p.m_tiles;
    a.k_tiles = p.n_tiles;
    a.k_tile0 = kt0;
    a.pcols = (int32_t)cols;
    a.splits = p.splits;
    a.csteps = p.steps;
    a.csteps_per_split = p.steps_per_split;
    a.cols_first = cols_first(p.m_tiles, a.m, cols) ? 1 : 0;
    a.partials = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const int64_t wgs = (int64_t)p.m_tiles * p.n_tiles * p.splits;
    if (wgs > INT32_MAX / 2) return fail("dk_nf4_linear_bwd: problem too large");
    if (check_hip(launch_bwd8(a, p.mt, pad8((int)wgs), st), "dk_nf4_linear_bwd launch")) return 1;
    if (p.splits <= 1) return 0;
    const int64_t c0 = (int64_t)kt0 * 256;
    ReduceArgs r{};
    r.partials = a.partials;
    r.slab = (int64_t)a.m * cols;
    r.splits = p.splits;
    r.m = a.m;
    r.ncols = (int)cols;
    r.nout = 1;
    r.out_fp32 = a.dx_fp32;
    void* out = static_cast<uint8_t*>(a.dx) + c0 * (a.dx_fp32 ? 4 : 2);
    r.o[0] = ReduceOut{out, a.lddx, nullptr, 0, (int32_t)cols};
    return check_hip(launch_splitk_reduce(r, st), "dk_nf4_linear_bwd split-K reduction");
}

// The input-gradient launch behind dk_nf4_linear_bwd and dk_nf4_linear_bwd_swiglu (sw != NULL:
// no dX; the epilogue turns fp16(dY.W) into dgate / dup; never split).
// max_partial_bytes: a cap on the split-K workspace the plan may use (the static-scratch entry).
static int linear_bwd_impl(const std::string& name, const dk_linear_bwd_group* groups, int ngroups,
                           int64_t m, int64_t k, void* dx, int64_t lddx, int dx_fp32, int lora_rank,
                           void* workspace, int64_t workspace_bytes_, void* stream,
                           const SwigluBwdOut* sw, int64_t max_partial_bytes = INT64_MAX) {
    if (ngroups < 1 || ngroups > kMaxGroups || groups == nullptr)
        return fail(name + ": need 1..4 groups");
    if (m < 0 || k <= 0 || (k % 32) != 0)
        return fail(name + ": k must be a positive multiple of 32");
    if (m > INT32_MAX / 2 || k > INT32_MAX / 2) return fail(name + ": m or k too large");
    if (sw == nullptr && m > 0 && (dx == nullptr || !aligned(dx, 16) || lddx < k || (lddx % 8) != 0))
        return fail(name + ": dx must be 16-byte aligned with lddx >= k, lddx % 8 == 0");
    if (lora_rank != 0 && lora_rank != 16 && lora_rank != 32)
        return fail(name + ": lora_rank must be 0, 16 or 32");
    BwdArgs a{};
    int64_t ns[kMaxGroups];
    int nested = -1;
    int step = 0;
    for (int g = 0; g < ngroups; ++g) {
        const dk_linear_bwd_group& G = groups[g];
        if (to_dev(&G.w, &a.g[g].w, name.c_str())) return 1;
        if (G.w.k != k) return fail(name + ": weight k differs from dx");
        if (gemm_weight_ok(G.w, name.c_str())) return 1;
        if ((m - 1) * G.lddy + G.w.n >= INT32_MAX / 2) return fail(name + ": dy too large");
        if (!aligned(G.w.packed, 16)) return fail(name + ": packed weights must be 16-byte aligned");
        if ((G.w.n % 8) != 0) return fail(name + ": weight rows must be a multiple of 8");
        if (nested >= 0 && nested != G.w.nested)
            return fail(name + ": all groups must be nested or all plain");
        nested = G.w.nested;
        if (m > 0 && (G.dy == nullptr || !aligned(G.dy, 16) || G.lddy < G.w.n || (G.lddy % 8) != 0))
            return fail(name + ": dy must be 16-byte aligned with lddy >= n, lddy % 8 == 0");
        if (G.lora_gu != nullptr && (lora_rank == 0 || G.lora_a == nullptr || !aligned(G.lora_gu, 16)))
            return fail(name + ": LoRA needs lora_rank > 0, lora_a and 16-byte aligned gu");
        if (G.lora_gu != nullptr && (m * lora_rank * 2 >= INT32_MAX || k * lora_rank * 2 >= INT32_MAX))
            return fail(name + ": LoRA operands larger than 2^31 bytes");
        if (G.lora_keep != nullptr && (G.lora_gu == nullptr || (k % 8) != 0 || m * (k / 8) >= INT32_MAX / 2 ||
                                       !(G.lora_keep_scale >= 0.0f)))
            return fail(name + ": lora_keep needs a LoRA term, k % 8 == 0, fewer than 2^30 bytes and a scale >= 0");
        if (G.lora_keep != nullptr && sw != nullptr)
            return fail(name + ": the SwiGLU epilogue takes no dropout-masked LoRA term");
        if (G.w.blocksize < 64 || k % 64 != 0) a.wide_stats = 1;
        a.g[g].dy = reinterpret_cast<const _Float16*>(G.dy);
        a.g[g].lddy = (int32_t)G.lddy;
        a.g[g].dy_bytes = m > 0 ? (uint32_t)(((m - 1) * G.lddy + G.w.n) * 2) : 0;
        a.g[g].lora_gu = reinterpret_cast<const _Float16*>(G.lora_gu);
        a.g[g].lora_a = reinterpret_cast<const _Float16*>(G.lora_a);
        a.g[g].lora_keep = G.lora_keep;
        a.g[g].lora_keep_scale = G.lora_keep_scale;
        a.g[g].step_begin = step;
        a.g[g].nsteps = (int)((G.w.n + kBwdBC - 1) / kBwdBC);
        step += a.g[g].nsteps;
        ns[g] = G.w.n;
    }
    if (m == 0) return 0;
    const BwdParts parts = plan_bwd_parts(m, k, ns, ngroups, sw != nullptr, max_partial_bytes);
    const int64_t need = workspace_bytes(parts);
    if (need > 0 && (workspace == nullptr || workspace_bytes_ < need || !aligned(workspace, 256)))
        return fail(name + ": workspace too small (need " + std::to_string(need) + " bytes)");
    a.dx = dx;
    a.lddx = lddx;
    a.m = (int)m;
    a.k = (int)k;
    a.ngroups = ngroups;
    a.lora_rank = lora_rank;
    a.dx_fp32 = dx_fp32 ? 1 : 0;
    a.nested = nested;
    if (sw != nullptr) {
        a.swiglu = 1;
        a.gate = reinterpret_cast<const _Float16*>(sw->gate);
        a.up = reinterpret_cast<const _Float16*>(sw->up);
        a.ldgu = sw->ldgu;
        a.dgate = reinterpret_cast<_Float16*>(sw->dgate);
        a.dup = reinterpret_cast<_Float16*>(sw->dup);
        a.ldd = sw->ldd;
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (launch_bwd_part(a, parts.a, 0, k, workspace, st)) return 1;
    return parts.two ? launch_bwd_part(a, parts.b, parts.kt_b, k - (int64_t)parts.kt_b * 256, workspace, st) : 0;
}

extern "C" {

int dk_nf4_linear_bwd(const dk_linear_bwd_group* groups, int ngroups, int64_t m, int64_t k, void* dx,
                      int64_t lddx, int dx_fp32, int lora_rank, void* workspace,
                      int64_t workspace_bytes_, void* stream) {
    g_error.clear();
    return linear_bwd_impl("dk_nf4_linear_bwd", groups, ngroups, m, k, dx, lddx, dx_fp32, lora_rank,
                           workspace, workspace_bytes_, stream, nullptr);
}

}  // extern "C"

// ---- input gradient without allocation -----------------------------------------------------
// The split-K partial slabs of dk_nf4_linear_bwd_noalloc live in this file-scope device array.
// Every GPU the library runs on holds its own copy (kNoAllocScratchBytes) until the process
// ends. Host code never uses the array's name as an address (on the host it is a stand-in, not a
// device pointer): each device's copy is looked up once, with that device current, and kept.
constexpr int64_t kNoAllocScratchBytes = DK_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// This device's copy of `scratch` (nullptr with g_error set on failure).
static void* device_scratch(const char* who) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fail(std::string(who) + ": no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            fail(std::string(who) + ": hipGetSymbolAddress(scratch): " + hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

extern "C" {

int dk_nf4_linear_bwd_noalloc(const dk_linear_bwd_group* groups, int ngroups, int64_t m, int64_t k, void* dx,
                              int64_t lddx, int dx_fp32, int lora_rank, void* stream) {
    g_error.clear();
    const char* who = "dk_nf4_linear_bwd_noalloc";
    void* ws = device_scratch(who);
    if (ws == nullptr) return 1;
    // plans are capped to the scratch size (fewer splits, or none), so no shape needs more; the
    // check below guards that contract
    const int rc = linear_bwd_impl(who, groups, ngroups, m, k, dx, lddx, dx_fp32, lora_rank, ws,
                                   kNoAllocScratchBytes, stream, nullptr, kNoAllocScratchBytes);
    if (rc != 0 && g_error.find("workspace too small") != std::string::npos)
        return fail(std::string(who) + ": split-K partials exceed the " +
                    std::to_string(kNoAllocScratchBytes) + "-byte scratch");
    return rc;
}

int dk_nf4_linear_bwd_swiglu(const dk_linear_bwd_group* group, int64_t m, int64_t k, int lora_rank,
                             const uint16_t* gate, const uint16_t* up, int64_t ldgu, uint16_t* dgate,
                             uint16_t* dup, int64_t ldd, void* stream) {
    g_error.clear();
    if (m > 0 && (gate == nullptr || up == nullptr || dgate == nullptr || dup == nullptr))
        return fail("dk_nf4_linear_bwd_swiglu: gate, up, dgate and dup are required");
    if (m > 0 && (!aligned(gate, 16) || !aligned(up, 16) || !aligned(dgate, 16) || !aligned(dup, 16) ||
                  ldgu < k || ldd < k || (ldgu % 8) != 0 || (ldd % 8) != 0))
        return fail("dk_nf4_linear_bwd_swiglu: gate/up/dgate/dup must be 16-byte aligned, row strides >= k and % 8 == 0");
    const SwigluBwdOut sw{gate, up, ldgu, dgate, dup, ldd};
    return linear_bwd_impl("dk_nf4_linear_bwd_swiglu", group, 1, m, k, nullptr, 0, 0, lora_rank, nullptr, 0,
                           stream, &sw);
}

}  // extern "C"

// The LoRA entries: every branch is checked as the per-branch entries check it, then handed to the
// grouped launchers (one branch for dk_lora_down / dk_lora_bwd and their dropout forms).
static int lora_check_common(const std::string& who, int rank, int64_t m, int64_t k) {
    if (rank != 16 && rank != 32) return fail(who + ": rank must be 16 or 32");
    if (m < 0 || k <= 0) return fail(who + ": bad shapes");
    return 0;
}

// x fp16 or fp32 (x32), keep null or packed dropout bits
static int lora_down_check(const std::string& who, const LoraBranch& b, int64_t m, int64_t k, int rank) {
    if ((k % 8) != 0 || b.ldx < k || (b.ldx % 8) != 0) return fail(who + ": k and ldx must be multiples of 8");
    if (b.x == nullptr || b.a == nullptr || b.u == nullptr || !aligned(b.x, 16) || !aligned(b.a, 16))
        return fail(who + ": x and a must be 16-byte aligned");
    if (b.keep != nullptr && b.keep_scale == nullptr) return fail(who + ": keep bits need keep_scale");
    // 32-bit byte offsets (with a 32-row margin for the tile past the last row)
    if ((m + 32) * b.ldx * (b.x32 ? 4 : 2) >= INT32_MAX || k * rank * 2 >= INT32_MAX || (m + 32) * (k / 8) >= INT32_MAX)
        return fail(who + ": tensors too large");
    return 0;
}

static int lora_bwd_check(const std::string& who, const LoraBranch& b, int64_t m, int64_t k, int rank) {
    const int64_t n = b.n;
    if (n <= 0 || b.lddy < n || b.ldx < k) return fail(who + ": bad shapes");
    if (b.dy == nullptr || b.u == nullptr || b.x == nullptr || b.b == nullptr || b.gu == nullptr)
        return fail(who + ": null pointer");
    if (!aligned(b.u, 16) || !aligned(b.b, 16) || !aligned(b.gu, 16) || !aligned(b.dy, 16) ||
        !aligned(b.x, b.x32 ? 4 : 2))
        return fail(who + ": dy, u, b, gu must be 16-byte aligned (x aligned to its element)");
    if ((n % 8) != 0 || (b.lddy % 8) != 0) return fail(who + ": n and lddy must be multiples of 8");
    if (b.keep != nullptr && (b.keep_scale == nullptr || (k % 8) != 0))
        return fail(who + ": keep bits need keep_scale and k % 8 == 0");
    // 32-bit byte offsets (with a 32-row margin for the tile past the last row)
    if ((m + 32) * b.lddy * 2 >= INT32_MAX || (m + 32) * b.ldx * (b.x32 ? 4 : 2) >= INT32_MAX ||
        (m + 32) * rank * 2 >= INT32_MAX || n * rank * 2 >= INT32_MAX || (m + 32) * (k / 8) >= INT32_MAX)
        return fail(who + ": tensors too large");
    return 0;
}

static LoraBranch lora_branch(const void* x, bool x32, int64_t ldx, const uint8_t* keep, const float* keep_scale) {
    LoraBranch b{};
    b.x = x;
    b.x32 = x32;
    b.ldx = ldx;
    b.keep = keep;
    b.keep_scale = keep_scale;
    return b;
}

static int lora_down_impl(const std::string& who, const void* x, bool x32, int64_t m, int64_t k, int64_t ldx,
                          const uint8_t* keep, const float* keep_scale, const uint16_t* a, int rank, uint16_t* u,
                          void* stream) {
    if (lora_check_common(who, rank, m, k)) return 1;
    LoraBranch b = lora_branch(x, x32, ldx, keep, keep_scale);
    b.a = reinterpret_cast<const _Float16*>(a);
    b.u = reinterpret_cast<_Float16*>(u);
    if (lora_down_check(who, b, m, k, rank)) return 1;
    return check_hip(launch_lora_down(&b, 1, m, k, rank, static_cast<hipStream_t>(stream)), (who + " launch").c_str());
}

static int lora_bwd_impl(const std::string& who, const uint16_t* dy, int64_t lddy, const uint16_t* u, const void* x,
                         bool x32, int64_t ldx, const uint8_t* keep, const float* keep_scale, const uint16_t* b,
                         int64_t m, int64_t n, int64_t k, int rank, float scale, uint16_t* gu, float* da, float* db,
                         void* stream) {
    if (lora_check_common(who, rank, m, k)) return 1;
    LoraBranch br = lora_branch(x, x32, ldx, keep, keep_scale);
    br.dy = reinterpret_cast<const _Float16*>(dy);
    br.lddy = lddy;
    br.n = n;
    br.u = const_cast<_Float16*>(reinterpret_cast<const _Float16*>(u));
    br.b = reinterpret_cast<const _Float16*>(b);
    br.scale = scale;
    br.gu = reinterpret_cast<_Float16*>(gu);
    br.da = da;
    br.db = db;
    if (lora_bwd_check(who, br, m, k, rank)) return 1;
    return check_hip(launch_lora_bwd(&br, 1, m, k, rank, static_cast<hipStream_t>(stream)), (who + " launch").c_str());
}

// The branches of a grouped call as the launchers take them (every one checked).
static int lora_group(const std::string& who, const dk_lora_branch* in, int nb, int64_t m, int64_t k, int rank,
                      bool backward, LoraBranch* out) {
    if (in == nullptr || nb < 1 || nb > kLoraMaxBranches) return fail(who + ": need 1..4 branches");
    if (lora_check_common(who, rank, m, k)) return 1;
    for (int i = 0; i < nb; ++i) {
        const dk_lora_branch& s = in[i];
        LoraBranch b = lora_branch(s.x, s.x_fp32 != 0, s.ldx, s.keep_bits, s.keep_scale);
        b.a = reinterpret_cast<const _Float16*>(s.a);
        b.u = reinterpret_cast<_Float16*>(s.u);
        b.dy = reinterpret_cast<const _Float16*>(s.dy);
        b.lddy = s.lddy;
        b.n = s.n;
        b.b = reinterpret_cast<const _Float16*>(s.b);
        b.gu = reinterpret_cast<_Float16*>(s.gu);
        b.da = s.da;
        b.db = s.db;
        b.scale = s.scale;
        const std::string w = who + " branch " + std::to_string(i);
        if (backward ? lora_bwd_check(w, b, m, k, rank) : lora_down_check(w, b, m, k, rank)) return 1;
        out[i] = b;
    }
    return 0;
}

extern "C" {

int dk_lora_down(const uint16_t* x, int64_t m, int64_t k, int64_t ldx, const uint16_t* a, int rank,
                 uint16_t* u, void* stream) {
    g_error.clear();
    return lora_down_impl("dk_lora_down", x, false, m, k, ldx, nullptr, nullptr, a, rank, u, stream);
}

int dk_lora_down_dropout(const void* x, int x_fp32, int64_t m, int64_t k, int64_t ldx, const uint8_t* keep_bits,
                         const float* keep_scale, const uint16_t* a, int rank, uint16_t* u, void* stream) {
    g_error.clear();
    return lora_down_impl("dk_lora_down_dropout", x, x_fp32 != 0, m, k, ldx, keep_bits, keep_scale, a, rank, u,
                          stream);
}

int dk_lora_bwd(const uint16_t* dy, int64_t lddy, const uint16_t* u, const uint16_t* x, int64_t ldx,
                const uint16_t* b, int64_t m, int64_t n, int64_t k, int rank, float scale, uint16_t* gu,
                float* da, float* db, void* stream) {
    g_error.clear();
    return lora_bwd_impl("dk_lora_bwd", dy, lddy, u, x, false, ldx, nullptr, nullptr, b, m, n, k, rank, scale, gu,
                         da, db, stream);
}

int dk_lora_bwd_dropout(const uint16_t* dy, int64_t lddy, const uint16_t* u, const void* x, int x_fp32,
                        int64_t ldx, const uint8_t* keep_bits, const float* keep_scale, const uint16_t* b,
                        int64_t m, int64_t n, int64_t k, int rank, float scale, uint16_t* gu, float* da,
                        float* db, void* stream) {
    g_error.clear();
    return lora_bwd_impl("dk_lora_bwd_dropout", dy, lddy, u, x, x_fp32 != 0, ldx, keep_bits, keep_scale, b, m, n,
                         k, rank, scale, gu, da, db, stream);
}

int dk_lora_down_group(const dk_lora_branch* branches, int nbranches, int64_t m, int64_t k, int rank,
                       void* stream) {
    g_error.clear();
    LoraBranch br[kLoraMaxBranches];
    if (lora_group("dk_lora_down_group", branches, nbranches, m, k, rank, false, br)) return 1;
    return check_hip(launch_lora_down(br, nbranches, m, k, rank, static_cast<hipStream_t>(stream)),
                     "dk_lora_down_group launch");
}

int dk_lora_bwd_group(const dk_lora_branch* branches, int nbranches, int64_t m, int64_t k, int rank,
                      void* stream) {
    g_error.clear();
    LoraBranch br[kLoraMaxBranches];
    if (lora_group("dk_lora_bwd_group", branches, nbranches, m, k, rank, true, br)) return 1;
    return check_hip(launch_lora_bwd(br, nbranches, m, k, rank, static_cast<hipStream_t>(stream)),
                     "dk_lora_bwd_group launch");
}

int dk_lora_keep_pack(const uint8_t* keep_q, const uint8_t* keep_v, uint8_t* bits_q, uint8_t* bits_v,
                      int64_t rows, int64_t width, void* stream) {
    g_error.clear();
    if (rows < 0 || width < 0 || (width % 8) != 0) return fail("dk_lora_keep_pack: width must be a multiple of 8");
    if (rows * width == 0) return 0;
    if (keep_q == nullptr || keep_v == nullptr || bits_q == nullptr || bits_v == nullptr)
        return fail("dk_lora_keep_pack: null pointer");
    if (!aligned(keep_q, 8) || !aligned(keep_v, 8)) return fail("dk_lora_keep_pack: masks must be 8-byte aligned");
    return check_hip(launch_lora_keep_pack(keep_q, keep_v, bits_q, bits_v, rows * width / 8,
                                           static_cast<hipStream_t>(stream)),
                     "dk_lora_keep_pack launch");
}

int dk_lora_dropout_inputs(const void* x, int x_fp32, const uint8_t* bits_q, const uint8_t* bits_v,
                           const float* scale_q, const float* scale_v, uint16_t* xq, uint16_t* xv,
                           int64_t rows, int64_t width, void* stream) {
    g_error.clear();
    if (rows < 0 || width < 0 || (width % 8) != 0) return fail("dk_lora_dropout_inputs: width must be a multiple of 8");
    if (rows * width == 0) return 0;
    if (x == nullptr || bits_q == nullptr || bits_v == nullptr || scale_q == nullptr || scale_v == nullptr ||
        xq == nullptr || xv == nullptr)
        return fail("dk_lora_dropout_inputs: null pointer");
    if (!aligned(x, 16) || !aligned(xq, 16) || !aligned(xv, 16))
        return fail("dk_lora_dropout_inputs: x, xq and xv must be 16-byte aligned");
    return check_hip(launch_lora_dropout_inputs(x, x_fp32 != 0, bits_q, bits_v, scale_q, scale_v,
                                                reinterpret_cast<_Float16*>(xq), reinterpret_cast<_Float16*>(xv),
                                                rows * width / 8, static_cast<hipStream_t>(stream)),
                     "dk_lora_dropout_inputs launch");
}

int dk_lora_input_grad(const uint16_t* gq, const uint16_t* gv, const uint8_t* bits_q, const uint8_t* bits_v,
                       float scale_q, float scale_v, float* out, int64_t rows, int64_t width, void* stream) {
    g_error.clear();
    if (rows < 0 || width < 0 || (width % 8) != 0) return fail("dk_lora_input_grad: width must be a multiple of 8");
    if (rows * width == 0) return 0;
    if (gq == nullptr || gv == nullptr || bits_q == nullptr || bits_v == nullptr || out == nullptr)
        return fail("dk_lora_input_grad: null pointer");
    if (!aligned(gq, 16) || !aligned(gv, 16) || !aligned(out, 16))
        return fail("dk_lora_input_grad: gq, gv and out must be 16-byte aligned");
    return check_hip(launch_lora_input_grad(reinterpret_cast<const _Float16*>(gq), reinterpret_cast<const _Float16*>(gv),
                                            bits_q, bits_v, scale_q, scale_v, out, rows * width / 8,
                                            static_cast<hipStream_t>(stream)),
                     "dk_lora_input_grad launch");
}

int dk_lora_up(const uint16_t* gu, const uint16_t* a, int rank, uint16_t* out, int64_t m, int64_t k, void* stream) {
    g_error.clear();
    if (rank != 16 && rank != 32) return fail("dk_lora_up: rank must be 16 or 32");
    if (m < 0 || k < 0 || (k % 8) != 0) return fail("dk_lora_up: k must be a multiple of 8");
    if (m * k == 0) return 0;
    if (gu == nullptr || a == nullptr || out == nullptr) return fail("dk_lora_up: null pointer");
    if (!aligned(a, 16) || !aligned(out, 16)) return fail("dk_lora_up: a and out must be 16-byte aligned");
    return check_hip(launch_lora_up(reinterpret_cast<const _Float16*>(gu), reinterpret_cast<const _Float16*>(a), rank,
                                    reinterpret_cast<_Float16*>(out), m, k, static_cast<hipStream_t>(stream)),
                     "dk_lora_up launch");
}

int dk_rope_qk_fwd(const uint16_t* q_base, const uint16_t* q_lora, int64_t ldq, int64_t ldl, const uint16_t* k,
                   int64_t ldk, const float* cos, const float* sin, uint16_t* q_out, uint16_t* k_out, int64_t n_tok,
                   int n_heads, int n_kv_heads, int head_dim, void* stream) {
    g_error.clear();
    if (n_tok < 0 || n_heads < 0 || n_kv_heads < 0 || head_dim <= 0 || (head_dim % 16) != 0)
        return fail("dk_rope_qk_fwd: head_dim must be a positive multiple of 16");
    if (n_tok == 0) return 0;
    if (q_base == nullptr || k == nullptr || cos == nullptr || sin == nullptr || q_out == nullptr || k_out == nullptr)
        return fail("dk_rope_qk_fwd: null pointer");
    if (ldq < (int64_t)n_heads * head_dim || ldk < (int64_t)n_kv_heads * head_dim || (ldq % 8) || (ldk % 8) ||
        (q_lora != nullptr && (ldl < (int64_t)n_heads * head_dim || (ldl % 8))))
        return fail("dk_rope_qk_fwd: row strides must cover the heads and be multiples of 8");
    if (!aligned(q_base, 16) || !aligned(k, 16) || !aligned(cos, 16) || !aligned(sin, 16) || !aligned(q_out, 16) ||
        !aligned(k_out, 16) || (q_lora != nullptr && !aligned(q_lora, 16)))
        return fail("dk_rope_qk_fwd: tensors must be 16-byte aligned");
    RopeArgs a{};
    a.q_base = reinterpret_cast<const _Float16*>(q_base);
    a.q_lora = reinterpret_cast<const _Float16*>(q_lora);
    a.k = reinterpret_cast<const _Float16*>(k);
    a.ldq = ldq;
    a.ldl = ldl;
    a.ldk = ldk;
    a.cos = cos;
    a.sin = sin;
    a.q_out = reinterpret_cast<_Float16*>(q_out);
    a.k_out = reinterpret_cast<_Float16*>(k_out);
    a.n_tok = n_tok;
    a.hq = n_heads;
    a.hk = n_kv_heads;
    a.d = head_dim;
    return check_hip(launch_rope(a, false, static_cast<hipStream_t>(stream)), "dk_rope_qk_fwd launch");
}

int dk_rope_qk_bwd(const uint16_t* grad_q, const uint16_t* grad_k, const float* cos, const float* sin, uint16_t* dq,
                   int64_t lddq, uint16_t* dk, int64_t lddk, int64_t n_tok, int n_heads, int n_kv_heads, int head_dim,
                   void* stream) {
    g_error.clear();
    if (n_tok < 0 || n_heads < 0 || n_kv_heads < 0 || head_dim <= 0 || (head_dim % 16) != 0)
        return fail("dk_rope_qk_bwd: head_dim must be a positive multiple of 16");
    if (n_tok == 0) return 0;
    if (grad_q == nullptr || grad_k == nullptr || cos == nullptr || sin == nullptr || dq == nullptr || dk == nullptr)
        return fail("dk_rope_qk_bwd: null pointer");
    if (lddq < (int64_t)n_heads * head_dim || lddk < (int64_t)n_kv_heads * head_dim || (lddq % 8) || (lddk % 8))
        return fail("dk_rope_qk_bwd: row strides must cover the heads and be multiples of 8");
    if (!aligned(grad_q, 16) || !aligned(grad_k, 16) || !aligned(dq, 16) || !aligned(dk, 16))
        return fail("dk_rope_qk_bwd: tensors must be 16-byte aligned");
    RopeArgs a{};
    a.cos = cos;
    a.sin = sin;
    a.grad_q = reinterpret_cast<const _Float16*>(grad_q);
    a.grad_k = reinterpret_cast<const _Float16*>(grad_k);
    a.dq = reinterpret_cast<_Float16*>(dq);
    a.dk = reinterpret_cast<_Float16*>(dk);
    a.lddq = lddq;
    a.lddk = lddk;
    a.n_tok = n_tok;
    a.hq = n_heads;
    a.hk = n_kv_heads;
    a.d = head_dim;
    return check_hip(launch_rope(a, true, static_cast<hipStream_t>(stream)), "dk_rope_qk_bwd launch");
}

int dk_swiglu_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, void* stream) {
    g_error.clear();
    if (n < 0 || (n > 0 && (gate == nullptr || up == nullptr || out == nullptr)))
        return fail("dk_swiglu_fwd: bad arguments");
    if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(out, 16))
        return fail("dk_swiglu_fwd: pointers must be 16-byte aligned");
    return check_hip(launch_swiglu_fwd(reinterpret_cast<const _Float16*>(gate),
                                       reinterpret_cast<const _Float16*>(up),
                                       reinterpret_cast<_Float16*>(out), n,
                                       static_cast<hipStream_t>(stream)),
                     "dk_swiglu_fwd launch");
}

int dk_swiglu_bwd(const uint16_t* grad, const uint16_t* gate, const uint16_t* up, uint16_t* dgate,
                  uint16_t* dup, int64_t n, void* stream) {
    g_error.clear();
    if (n < 0 || (n > 0 && (grad == nullptr || gate == nullptr || up == nullptr || dgate == nullptr ||
                            dup == nullptr)))
        return fail("dk_swiglu_bwd: bad arguments");
    if (!aligned(grad, 16) || !aligned(gate, 16) || !aligned(up, 16) || !aligned(dgate, 16) ||
        !aligned(dup, 16))
        return fail("dk_swiglu_bwd: pointers must be 16-byte aligned");
    return check_hip(launch_swiglu_bwd(reinterpret_cast<const _Float16*>(grad),
                                       reinterpret_cast<const _Float16*>(gate),
                                       reinterpret_cast<const _Float16*>(up),
                                       reinterpret_cast<_Float16*>(dgate), reinterpret_cast<_Float16*>(dup),
                                       n, static_cast<hipStream_t>(stream)),
                     "dk_swiglu_bwd launch");
}

int dk_probe_hbm(const void* src, void* dst, int64_t bytes, int mode, float* sums, void* stream) {
    g_error.clear();
    const int kind = mode & 3;
    if (bytes <= 0 || (bytes % 16) != 0 || mode < 0 || (mode & ~63) != 0 || ((mode >> 4) & 3) == 3 || kind > 2 || bytes / 16 / 1024 >= INT32_MAX ||
        (kind != 1 && (src == nullptr || !aligned(src, 16))) || (kind != 0 && (dst == nullptr || !aligned(dst, 16))) ||
        (kind == 0 && sums == nullptr))
        return fail("dk_probe_hbm: bad arguments");
    return check_hip(launch_hbm_probe(src, dst, bytes, mode, sums, static_cast<hipStream_t>(stream)),
                     "dk_probe_hbm launch");
}

int dk_probe_mfma_f16(int64_t work_groups, int32_t iters, float* out, void* stream) {
    g_error.clear();
    if (work_groups <= 0 || work_groups > INT32_MAX / 512 || iters <= 0 || out == nullptr)
        return fail("dk_probe_mfma_f16: bad arguments");
    return check_hip(launch_mfma_peak(work_groups, iters, out, static_cast<hipStream_t>(stream)),
                     "dk_probe_mfma_f16 launch");
}

}  // extern "C"
