// The C ABI (include/moe_amd.h): argument checks, the grow-only workspace,
// kernel timing, and the orchestration of the MoE layer forward.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace {

thread_local std::string g_last_error;

// Scratch of moe_layer_forward_noalloc: one array per GPU the library runs
// on, held until the process ends.  Host code never uses the array's name
// as an address (on the host it names a stand-in, not device memory): each
// device's address comes from hipGetSymbolAddress, taken once per device
// when the first context on it is created, and is what every kernel gets.
constexpr size_t kNoAllocScratchBytes = size_t(256) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch (the device must be current).
void* bind_scratch(int device) {
    moe::require(device < kMaxDevices, "device ordinal beyond the library's device table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        void* p = nullptr;
        moe::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                       "hipGetSymbolAddress(scratch)");
        moe::require(p != nullptr, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[device] = p;
    }
    return g_scratch_ptr[device];
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return MOE_OK;
    } catch (const moe::InvalidArg& e) {
        g_last_error = e.what();
        return MOE_ERR_INVALID;
    } catch (const moe::Unsupported& e) {
        g_last_error = e.what();
        return MOE_ERR_UNSUPPORTED;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return MOE_ERR_RUNTIME;
    } catch (...) {
        g_last_error = "unknown error";
        return MOE_ERR_RUNTIME;
    }
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Makes the context's device current for the duration of a call.
struct DeviceScope {
    int prev = -1, want;
    explicit DeviceScope(int d) : want(d) {
        moe::hip_check(hipGetDevice(&prev), "hipGetDevice");
        if (prev != want) moe::hip_check(hipSetDevice(want), "hipSetDevice");
    }
    ~DeviceScope() {
        if (prev >= 0 && prev != want) (void)hipSetDevice(prev);
    }
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Carves typed sub-buffers out of one allocation, 256-byte aligned.
struct Carve {
    char* base;
    size_t off = 0;
    explicit Carve(void* b) : base(static_cast<char*>(b)) {}
    template <class T>
    T* take(int64_t n) {
        off = (off + 255) & ~size_t(255);
        T* p = reinterpret_cast<T*>(base + off);
        off += static_cast<size_t>(n > 0 ? n : 1) * sizeof(T);
        return p;
    }
};

void check_ctx(moe_ctx* ctx) { moe::require(ctx != nullptr, "null moe_ctx"); }

void check_dims(int64_t a, const char* what) {
    moe::require(a >= 0, std::string(what) + " must be >= 0");
    moe::require(a <= INT32_MAX, std::string(what) + " exceeds int32 range");
}

void check_ptr(const void* p, const char* what) {
    moe::require(p != nullptr, std::string("null pointer: ") + what);
}

void check_routing(int64_t T, int64_t E, int64_t k) {
    check_dims(T, "T");
    moe::require(E >= 1 && E <= moe::kMaxExperts, "E must be in [1, 1024]");
    moe::require(k >= 1 && k <= E && k <= moe::kMaxTopK, "k must be in [1, min(E, 32)]");
    moe::require(T * k <= INT32_MAX, "T*k exceeds int32 range");
}

// ---- dense GEMM
int env_int(const char* name, int fallback) {
    const char* v = std::getenv(name);
    return v != nullptr ? std::atoi(v) : fallback;
}

// Tile shape and K splits of a dense SGEMM, from a cost model fitted to a
// tile x split sweep of the SGEMM shapes on MI355X (its choices there are on
// average 2 % and at worst 15 % slower than the best measured one; the
// sweep's run-to-run spread is about 5 %).  Per CU, the workgroups
// dealt to it run `occupancy` at a time; each K step of the resident ones
// costs the larger of their matrix-core time (the rows a wave really
// computes: 32-row blocks past M are skipped) and the latency of one load
// stage; HBM time counts A once, B once per m-tile and the split partials
// twice; launches and the split reduction add fixed costs.  Small and
// skinny products thereby get small tiles and a few K splits that fill all
// CUs; large ones keep the 128 x 128 tile.  MOE_DENSE_TILE /
// MOE_DENSE_SPLITS pin the choice for tuning.
struct DensePlan {
    int tile = 0, splits = 1;
};

#ifndef MOE_DENSE_KW_MIN
#define MOE_DENSE_KW_MIN 128  // fewest K columns per group
#endif
#ifndef MOE_DENSE_KW_PLAN
#define MOE_DENSE_KW_PLAN 1  // 0: the planner never deals the K-group tile (tuning builds)
#endif

constexpr int64_t kDenseSplitBytes = int64_t(512) << 20;  // cap on the partials

DensePlan plan_dense(moe_ctx* ctx, bool nn, bool direct, int64_t M, int64_t N, int64_t K) {
    DensePlan best;
    if (!direct || K == 0) return best;  // the register-staged kernel: 128 x 128, one pass
    static const int env_tile = env_int("MOE_DENSE_TILE", -1);
    static const int env_splits = env_int("MOE_DENSE_SPLITS", 0);
    auto split_ok = [&](int S) {
        return S == 1 || (K % (16 * S) == 0 && K / S >= 64 &&
                          int64_t(S) * M * N * 4 <= kDenseSplitBytes);
    };
    // fitted constants: MFMA efficiency per tile shape, latency of one load
    // stage, start-up and drain of a round of workgroups, achievable HBM
    // bandwidth, launch and reduction overheads, and the slowdown of a
    // workgroup alone on its CU (4096 x 1024 x 1024: 128 x 128 tiles, one
    // per CU, 95.6 us; 64 x 128 tiles, two per CU, 87.4 us)
    // (tile 3 reads NN B fragments 16 bytes at a time, as NT reads them)
    static constexpr double kEff[moe::kDenseTiles] = {0.80, 0.80, 0.50, 0.86, 0.0, 0.0};
    constexpr double kStageLatency = 0.6e-6, kRound = 1e-6, kHbm = 5.0e12, kLaunch = 2e-6,
                     kReduce = 2e-6, kSolo = 1.15;
    // each tile shape runs 4 waves, one per SIMD
    const double simd_rate = 157.3e12 / (4.0 * ctx->cus);
    double best_t = 1e30;
    // Up to 32 rows the skinny kernel (B streamed once into registers, 16-row
    // MFMAs, no LDS) takes every aligned shape: measured on MI355X at N =
    // 14336, K = 4096, M = 16 NN 40.5 us against 50-54 us on the best tile
    // and split (0.73 of the HBM roofline), M = 32 51 us; at M = 64, where the
    // product turns MFMA-bound, the tiles are as fast and keep it.  Its waves
    // need K splits to keep HBM busy: the most (up to 16) that keep the grid
    // at about 1024 waves (measured best at 896: 4 splits of N = 14336; 8 or
    // 16 add split-sum reads, 1 or 2 leave HBM idle).
    if (M <= 32 && (!nn || N % 4 == 0) && (env_tile < 0 || env_tile == moe::kSkinnyTile)) {
        best.tile = moe::kSkinnyTile;
        best.splits = 1;
        for (int S = 2; S <= moe::kMaxDenseSplits; S *= 2)
            if (split_ok(S) && moe::ceil_div(N, 64) * S <= 1024) best.splits = S;
        if (env_splits > 0 && split_ok(env_splits)) best.splits = env_splits;
        return best;
    }
    // The K-group tile (32 x 128, K split among the waves of one workgroup)
    // where its tiles give 3/4 to all of the CUs one workgroup each, every
    // group gets 128-512 K columns and the model's best plan would split K
    // into a second launch.  Measured on MI355X against the plans without
    // it: 1024 x 1024 x K 15-20 % faster at K = 512-1024, 8-10 % at 2048,
    // level at 4096; with fewer tiles (512 x 1024 x 1024: half the CUs) the
    // split plans that fill every CU were 15-50 % faster.  It needs the
    // ring, so its buffer-load offsets (from the tile's first A row; from B's
    // first row (NT) or column (NN)) must fit 31 bits, as the launch checks,
    // and K whole steps per group.  The cost model below does not weigh it:
    // its HBM term counts B once per m-tile, which the L2 and Infinity Cache
    // serve at these sizes.
    const moe::GemmTile kwt = moe::dense_tile(moe::kDenseKwTile);
    const int kwg = moe::dense_tile_groups(moe::kDenseKwTile);
    const bool kw_ok = MOE_DENSE_KW_PLAN && (env_tile < 0 || env_tile == moe::kDenseKwTile) && M >= 128 &&
                       K % (16 * kwg) == 0 && K / kwg >= MOE_DENSE_KW_MIN && K / kwg <= 512 &&
                       moe::ceil_div(M, kwt.bm) * moe::ceil_div(N, kwt.bn) <= ctx->cus &&
                       moe::ceil_div(M, kwt.bm) * moe::ceil_div(N, kwt.bn) * 4 >= 3 * ctx->cus &&
                       int64_t(kwt.bm + 1) * K * 4 < (int64_t(1) << 31) &&
                       (nn ? (K + 16) * N * 4 + int64_t(kwt.bn) * 4
                           : int64_t(kwt.bn + 1) * K * 4) < (int64_t(1) << 31);
    for (int t = 0; t < moe::kDenseTiles; ++t) {
        if (env_tile >= 0 && t != env_tile) continue;
        if (t == moe::kSkinnyTile || t == moe::kDenseKwTile) continue;  // weighed apart
        int& occ = ctx->dense_blocks_per_cu[nn ? 1 : 0][t];
        if (occ == 0) occ = moe::dense_blocks_per_cu(t, nn);
        const moe::GemmTile g = moe::dense_tile(t);
        // wave grid: 2x2; 1x4 for the 32-row tile; 4x1 for the 256-row tile
        const int wm = g.bm >= 256 ? 4 : (g.bm >= 64 ? 2 : 1);
        const int wn = 4 / wm;
        const int64_t mt = moe::ceil_div(M, g.bm), nt = moe::ceil_div(N, g.bn);
        const int64_t rows_w = std::min<int64_t>(g.bm / wm, 32 * moe::ceil_div(std::min<int64_t>(M, g.bm), 32));
        const double step_mma = 2.0 * rows_w * (g.bn / wn) * 16 / (kEff[t] * simd_rate);
        for (int S = 1; S <= moe::kMaxDenseSplits; S *= 2) {
            if (env_splits > 0 && S != env_splits) continue;
            if (!split_ok(S) || mt * nt * S > INT32_MAX) continue;
            const int64_t blocks = mt * nt * S;
            const double steps = double(K / S / 16);
            // rounds of `occ` resident workgroups, then a last partial round
            const int64_t per_cu = moe::ceil_div(blocks, ctx->cus);
            const int64_t full = per_cu / occ, rest = per_cu % occ;
            // a round of r resident workgroups; alone on its CU a workgroup's
            // waves cannot hide their own fragment reads and barriers
            auto round_time = [&](int64_t r) {
                const double mma = double(r) * step_mma * (r == 1 ? kSolo : 1.0);
                return steps * std::max(mma, kStageLatency) + kRound;
            };
            double t_cu = double(full) * round_time(occ);
            if (rest > 0) t_cu += round_time(rest);
            double bytes = 4.0 * (double(M) * K + double(K) * N * mt + double(M) * N);
            if (S > 1) bytes += 8.0 * S * double(M) * N;
            double est = std::max(t_cu, bytes / kHbm) + kLaunch;
            // the split reduction: a second launch reading every partial once,
            // and the partial stores, which the model cannot hide under the MFMAs
            const double part_bytes = 4.0 * S * double(M) * N;
            if (S > 1) est += kReduce + (part_bytes + 4.0 * M * N) / 4e12 + part_bytes / kHbm;
            if (est < best_t) {
                best_t = est;
                best.tile = t;
                best.splits = S;
            }
        }
    }
    if (kw_ok && (best.splits > 1 || env_tile == moe::kDenseKwTile)) {
        best.tile = moe::kDenseKwTile;
        best.splits = 1;
    }
    return best;
}

// C = A B (+ bias) (+ resid): resid [M, N] (may be C itself) is added after
// the bias in the GEMM's store, or in the split reduction when K is split,
// so C is bit-identical to the GEMM followed by moe_add.
void sgemm(moe_ctx* ctx, bool nn, const float* A, const float* B,
           const float* bias, float* C, int64_t M, int64_t N, int64_t K,
           void* stream, const float* resid = nullptr) {
    check_ctx(ctx);
    check_dims(M, "M");
    check_dims(N, "N");
    check_dims(K, "K");
    if (M == 0 || N == 0) return;
    check_ptr(C, "C");
    if (K > 0) {
        check_ptr(A, "A");
        check_ptr(B, "B");
    }
    DeviceScope dev(ctx->device);
    const bool vec = (K % 4 == 0) && aligned16(A) && (nn || aligned16(B));
    // the direct-load kernels (every tile shape; split K): see launch_cfg
    const bool direct = vec && K % 16 == 0 && (!nn || (N % 4 == 0 && aligned16(B)));
    const DensePlan plan = plan_dense(ctx, nn, direct, M, N, K);
    const moe::GemmTile tile = moe::dense_tile(plan.tile);
    const int64_t mt = moe::ceil_div(M, tile.bm), ntl = moe::ceil_div(N, tile.bn);
    moe::require(mt * ntl * plan.splits <= INT32_MAX, "GEMM grid too large");
    moe::GemmArgs a{};
    a.A = A;
    a.lda = K;
    a.B0 = B;
    a.B1 = B;
    a.ldb = nn ? N : K;
    a.bias = bias;
    a.resid = resid;
    a.C = C;
    a.ldc = N;
    a.M = M;
    a.N = N;
    a.K = K;
    a.m_tiles = static_cast<int32_t>(mt);
    a.n_tiles = static_cast<int32_t>(ntl);
    a.tile = plan.tile;
    // K == 0 leaves the kernel with no K step: C = bias (or 0) still gets written.
    if (K == 0) {
        a.A = C;  // any valid pointer; never read
        a.B0 = a.B1 = C;
    }
    hipStream_t s = as_stream(stream);
    float* parts = nullptr;
    if (plan.splits > 1) {
        // split K: each split writes its partial product to the workspace,
        // [splits, M, N]; the reduction adds them in order, then the bias.
        parts = static_cast<float*>(ctx->workspace(size_t(plan.splits) * M * N * sizeof(float)));
        a.C = parts;
        a.ldc = N;
        a.bias = nullptr;
        a.resid = nullptr;
        a.k_splits = plan.splits;
        a.k_split_len = K / plan.splits;
        a.c_split_stride = M * N;
    }
    ctx->launch(nn ? "sgemm_nn" : "sgemm_nt", s, [&] {
        moe::launch_gemm(a, nn, false, moe::EPI_BIAS, vec, s);
        if (parts != nullptr)
            moe::launch_split_sum(parts, plan.splits, M * N, bias, resid, C, M, N, s);
    });
}

// ---- expert FFN (the part shared by moe_expert_ffn_grouped and the layer)
// Upper bound of sum_e ceil(n_e / bm) over the experts: the grouped
// kernels launch this many m-tiles and the surplus ones exit at once.
int64_t grouped_m_tiles(int64_t pairs, int64_t E, int bm) {
    return std::min<int64_t>(moe::ceil_div(pairs, bm) + E, pairs);
}

// K splits S of the layer's w2 on the one-tile-per-workgroup kernel.  Its
// tiles run in rounds of `slots` concurrent workgroups; a last, partly
// filled round of long-K tiles wastes the rest of the GPU for a whole tile
// time.  Splitting K S ways makes the rounds S times shorter, but every
// split adds a partial row buffer w2 writes and the combine reads; the S in
// {1, 2, 4} with the least modelled time is taken (choose_w2_split_plan).  Each
// split must be a multiple of 16 columns.  MOE_W2_SPLITS overrides for
// tuning.
struct FfnPlan {
    int w13_tile = 0;  // GemmArgs::tile of w1/w3: 0 128x128 (W13), 1 256x64 (W13Tall)
    int w13_sk = 0;    // stream-K grid of w1/w3 (0: one tile per workgroup)
    int tile = 0;      // GemmArgs::tile of w2: 0 wide (W2), 1 128x128 (W2Narrow)
    int splits = 1;    // K splits of w2 (1 under stream-K)
    int w2_sk = 0;     // stream-K grid of w2
    int64_t sk_floats = 0;  // partial-tile floats the stream-K launches need
    bool skinny13 = false;  // w1/w3 on the grouped skinny kernel (choose_skinny)
    bool skinny2 = false;   // w2 on it
    int w13_splits = 1;     // K splits of the skinny w1/w3 (their raw sums in sk_part)
};

// The K splits of w2 on one w2 tile and their modelled time (choose_w2_split_plan).
struct W2SplitPlan {
    int splits = 1;
    double us = 0.0;
};

W2SplitPlan choose_w2_split_plan(moe_ctx* ctx, int64_t pairs, int64_t d, int64_t d_ff, int64_t E,
                                 int w2_tile);

// The w1/w3 tile: 128 rows x 128 columns of each operand, or, when d_ff is
// a multiple of 64 but not of 128 (the reference's 448), 256 rows x 64
// columns, so the n-tiles cover d_ff exactly instead of leaving the last one
// half empty -- while the experts average more than 128 rows: with fewer the
// 256-row tiles run mostly empty (same box, ms per layer, 256 x 64 -> 128 x
// 128: the reference's layer at 256 / 512 / 1,024 tokens 0.290 / 0.333 / 0.398
// -> 0.271-0.283 / 0.267 / 0.346; at 1,536 tokens, 192 rows per expert,
// 0.435 -> 0.439, and level from 2,048 tokens up).
// MOE_W13_TILE = 0 / 1 overrides.
int choose_w13_tile(int64_t d_ff, int64_t pairs, int64_t E) {
    static const int env_tile = env_int("MOE_W13_TILE", -1);
    if (env_tile == 0 || env_tile == 1) return env_tile;
    return (d_ff % 128 != 0 && d_ff % 64 == 0 && pairs > 128 * E) ? 1 : 0;
}

// Expected real m-tiles of a grouped launch: ceil(pairs / BM) plus half a
// tile per expert (each expert's last tile half full), at most the bound.
int64_t expected_m_tiles(int64_t pairs, int64_t E, int bm) {
    return std::min<int64_t>(moe::ceil_div(pairs, bm) + E / 2, grouped_m_tiles(pairs, E, bm));
}

// Stream-K or one tile per workgroup.  One tile per workgroup runs the
// tiles in rounds of `slots` (w2: of its S K splits); its fill is w /
// ceil(w), w = tiles * S / slots.  Stream-K runs the full rounds the same
// way and deals the K steps of the tiles left over to its G workgroups in
// contiguous ranges, at the price of partial stores and a fix-up launch for
// the cut tiles and of L2 sharing in the dealt part (its workgroups read
// unrelated K offsets).  Measured on MI355X at configs 1, 3-5 and the
// reference's layer shape with 64 tokens to full size, it wins where the
// one-tile fill is under 96 % and
//   w1/w3 (no K splits there): always -- also at short K (config 5's
//     K = 64 steps: 128 / 256 / 512 / 2,048 tokens 0.133 / 0.134 / 0.248 /
//     0.491 ms one tile per workgroup against 0.099 / 0.112 / 0.161 / 0.415
//     stream-K; 1,024 tokens, fill 0.86, level; full size, fill 0.97, stays
//     one tile per workgroup);
//   w2 (against its best split plan, whose combine reads every split's
//     partial rows): each workgroup's dealt range is at least 64 K steps.
// Pieces are kept at 32 K steps or more (with fewer tiles than slots, G is
// cut to tiles x K-steps / 32, at least the tiles), except for w1/w3 tiles
// under 128 K steps, which are dealt to every slot: there the short pieces
// measured faster (config 1's 64 tokens, 24 tiles of 32 K steps: 0.032 ms
// on all slots, 0.061 ms cut to whole tiles, 0.041 ms one tile per
// workgroup; config 5's 128 tokens 0.099 against 0.142 ms).  MOE_SK = 0 / 1 (or
// moe_ctx_set_stream_k) forces either (1: on every launch the direct
// buffer-load path applies to, on all slots).  Returns the stream-K grid, 0
// for one tile per workgroup.
int choose_sk(moe_ctx* ctx, moe::GemmUse use, int64_t pairs, int64_t E, int64_t N, int64_t K,
              int dp_splits, int dp_slots) {
    static const int env_mode = env_int("MOE_SK", -1);
    const int env = ctx->sk_mode >= 0 ? ctx->sk_mode : env_mode;
    if (env == 0 || pairs == 0 || K % 16 != 0 || K < 32) return 0;
    const moe::GemmTile t = moe::gemm_tile(use);
    const int64_t bound_tiles = grouped_m_tiles(pairs, E, t.bm) * moe::ceil_div(N, t.bn);
    if (bound_tiles * (K / 16) > INT32_MAX) return 0;
    int& occ = ctx->sk_blocks_per_cu[static_cast<int>(use)];
    if (occ == 0) occ = moe::gemm_sk_blocks_per_cu(use);
    const int slots = ctx->cus * occ;
    if (env == 1) return slots;
    const double nk = double(K / 16);
    const double tiles = double(expected_m_tiles(pairs, E, t.bm) * moe::ceil_div(N, t.bn));
    const int S = std::max(dp_splits, 1);
    const double w = tiles * S / dp_slots;
    if (w / std::ceil(w) >= 0.96) return 0;
    const bool w2 = use == moe::GemmUse::W2 || use == moe::GemmUse::W2Narrow;
    const double left = tiles - std::floor(tiles / slots) * slots;
    if (w2 && left * nk / slots < 64) return 0;
    double G = slots;
    if (tiles < G && (w2 || nk >= 128))
        G = std::min(G, std::max(tiles, std::floor(tiles * nk / 32.0)));
    return static_cast<int>(G);
}

// The FFN plan of a layer.  w2: the wide tile (its 256 columns halve the B
// traffic per MFMA) unless d gives it at most 4 n-tiles: then each expert's
// rows form so few tiles that the 128x128 tile's extra parallelism wins (a
// tile x split sweep on MI355X: config 5, d = 1024, 1.545 -> 1.488 ms per
// layer; configs 3 and 4, with 16 and 8 wide n-tiles, 3-5 % slower on the
// narrow tile).  Where the wide tile runs one tile per workgroup, the
// narrow one is taken if its rounds' modelled time is less: both tiles
// move the same work per CU and microsecond, so the choice is the rounds'
// fill (the reference's shape at 16,080 rows: wide 9 rounds, 8.1 full,
// narrow 11 rounds, 10.8 full: w2 1.039 -> 0.996 ms; 8,192 rows 0.581 ->
// 0.522 ms; 15,583 rows equal, wide kept).  MOE_W2_TILE = 0 / 1 overrides.
// Then stream-K where the one-tile rounds fill badly (choose_sk), else K
// splits for w2.
// Few rows per expert (at most 32 on average): a launch whose waves would
// each run a short K loop goes to the grouped skinny kernel, whose
// workgroups stream one expert's 16 or 32 rows against 64 columns of its
// weights, four waves to a quarter of K, instead of 128-row tiles that are
// mostly empty.  A wave's work is its K steps (K / 64, over S for w2's K
// splits) times its 16-row blocks times the B operands (2 assumed: w1 and
// w3).  Measured on MI355X, ms per launch, tiles -> skinny (units):
//   w1/w3: config 1 (64 tokens) 0.029 -> 0.014 (32); config 5 at 64 tokens
//     0.083 -> 0.069 (32), its decoder's last rows (16 pairs) about 0.075
//     -> 0.04 (32); config 5 at 128 tokens 0.101 -> 0.107 (64); the
//     reference's at 64 tokens 0.117 -> 0.167 (128): up to 32 units.
//   w2: config 1 0.024 -> 0.014 (8, d 512); the reference's at 64 tokens
//     0.044 -> 0.034 (7, 8 rows per expert); but at 128 tokens 0.044 ->
//     0.045 (7, 16 rows per expert, d 4096: 64 column blocks of short
//     workgroups), at 256 0.063 -> 0.064 (14) and config 5 at 64 tokens
//     0.037 -> 0.051 (22): up to 12 units, and only with at most 8 rows
//     per expert or d up to 1024.
// w2 takes the K splits S that keep about two workgroups per CU, each wave
// at least 4 K steps.  A context or process that forces the tiles' dealing
// (moe_ctx_set_stream_k, MOE_SK) keeps the tiles; MOE_FFN_SKINNY = 0 / 1
// turns the skinny kernel off / on for every launch the shape allows.
void choose_skinny(moe_ctx* ctx, FfnPlan& f, int64_t pairs, int64_t d, int64_t d_ff, int64_t E) {
    static const int env_skinny = env_int("MOE_FFN_SKINNY", -1);
    static const int env_sk = env_int("MOE_SK", -1);
    const bool sk_forced = (ctx->sk_mode >= 0 ? ctx->sk_mode : env_sk) >= 0;
    const int64_t rows_wg = pairs <= 16 * E ? 16 : 32;
    const int64_t rb_max = moe::ceil_div(pairs, rows_wg);
    if (env_skinny == 0 || sk_forced || d % 16 != 0 || d_ff % 16 != 0 || E * rb_max > 65535 ||
        (env_skinny != 1 && pairs > 32 * E))
        return;
    const int64_t blocks16 = rows_wg / 16;
    // w1/w3: the fewest K splits (1, 2 or 4; each split a multiple of 16
    // columns and at least 4 K steps per wave) that bring the units to 32 --
    // splits only while the experts average at most 16 rows (with 32, the
    // tiles run as fast: config 5 at 128 tokens, 2 splits, 0.104 against
    // 0.102 ms).  More splits than that lost (config 1, config 5 at 8-64
    // tokens: 2 or 4 splits 1-29 % slower per launch); fewer left the long K
    // loops (the reference at 64 tokens: 1 / 2 / 4 splits 0.168 / 0.094 /
    // 0.077 ms).  MOE_SKINNY_W13_SPLITS = 1 / 2 / 4 pins them for tuning.
    int S13 = 0;
    const int max_s13 = blocks16 == 1 ? 4 : 1;
    for (int s1 = 1; s1 <= max_s13 && S13 == 0; s1 *= 2)
        if (d % (16 * s1) == 0 && (s1 == 1 || d / (64 * s1) >= 4) &&
            (d / (64 * s1)) * blocks16 * 2 <= 32)
            S13 = s1;
    // expected row blocks: the pairs' blocks plus a partial one per expert
    const double blocks = std::min(double(E) * double(rb_max),
                                   double(pairs) / double(rows_wg) + 0.5 * double(E));
    // and at most about four workgroups per CU: with more, the tiles stream
    // the weights faster (config 3 at 64 tokens, 10,752 workgroups of 16 K
    // steps: w1/w3 1.151 against 0.931 ms)
    if (S13 > 0 && blocks * double(moe::ceil_div(d_ff, 64)) * S13 > 4.0 * ctx->cus) S13 = 0;
    if (env_skinny == 1 && S13 == 0) S13 = 1;
    static const int env_s13 = env_int("MOE_SKINNY_W13_SPLITS", 0);
    if (S13 > 0 && (env_s13 == 1 || env_s13 == 2 || env_s13 == 4) && d % (16 * env_s13) == 0)
        S13 = env_s13;
    if (S13 > 0) {
        f.skinny13 = true;
        f.w13_tile = moe::kGroupedSkinnyTile;
        f.w13_sk = 0;
        f.w13_splits = S13;
    }
    const double wgs = blocks * double(moe::ceil_div(d, 64));
    int S = 1;
    for (int s2 = 2; s2 <= moe::kMaxW2Splits; s2 *= 2)
        if (d_ff % (16 * s2) == 0 && d_ff / (64 * s2) >= 4 && wgs * s2 <= 2.0 * ctx->cus) S = s2;
    // (measured, µs per w2 launch at S = 1 / 2 / 4 against the tiles: config 1
    // 18.8 / 13.4 / 14.2 against 24.0; config 5 at 8 tokens 30.4 / 20.2 /
    // 20.5 against 36.1; the reference at 64 tokens 34.3 / 36.5 / 40.5
    // against 43.2.)  MOE_SKINNY_W2_SPLITS = 1 / 2 / 4 pins S for tuning.
    static const int env_s2 = env_int("MOE_SKINNY_W2_SPLITS", 0);
    if ((env_s2 == 1 || env_s2 == 2 || env_s2 == 4) && d_ff % (16 * env_s2) == 0) S = env_s2;
    if (env_skinny == 1 ||
        ((d_ff / (64 * S)) * blocks16 <= 12 && (pairs <= 8 * E || d <= 1024))) {
        f.skinny2 = true;
        f.tile = moe::kGroupedSkinnyTile;
        f.w2_sk = 0;
        f.splits = S;
    }
}

FfnPlan choose_ffn_plan(moe_ctx* ctx, int64_t pairs, int64_t d, int64_t d_ff, int64_t E) {
    FfnPlan f;
    static const int env_tile = env_int("MOE_W2_TILE", -1);
    const bool tile_pinned = env_tile == 0 || env_tile == 1;
    f.tile = moe::ceil_div(d, moe::gemm_tile(moe::GemmUse::W2).bn) <= 4 ? 1 : 0;
    if (tile_pinned) f.tile = env_tile;
    f.w13_tile = choose_w13_tile(d_ff, pairs, E);
    if (d_ff == 0 || d == 0) {
        f.splits = 1;
        return f;
    }
    // workgroups of the one-tile-per-workgroup kernel of `use` the GPU holds
    auto slots_of = [&](moe::GemmUse use) {
        int& occ = use == moe::GemmUse::W2Narrow ? ctx->w2n_blocks_per_cu
                   : use == moe::GemmUse::W2     ? ctx->w2_blocks_per_cu
                                                 : ctx->w13_blocks_per_cu[f.w13_tile];
        if (occ == 0) occ = moe::gemm_blocks_per_cu(use);
        return ctx->cus * occ;
    };
    const moe::GemmUse u13 = f.w13_tile == 1 ? moe::GemmUse::W13Tall : moe::GemmUse::W13;
    auto use_of = [](int tile) { return tile == 1 ? moe::GemmUse::W2Narrow : moe::GemmUse::W2; };
    W2SplitPlan w2 = choose_w2_split_plan(ctx, pairs, d, d_ff, E, f.tile);
    f.w13_sk = choose_sk(ctx, u13, pairs, E, d_ff, d, 1, slots_of(u13));
    // w2: stream-K against its best split plan
    f.w2_sk = choose_sk(ctx, use_of(f.tile), pairs, E, d, d_ff, w2.splits, slots_of(use_of(f.tile)));
    if (!tile_pinned && f.tile == 0 && f.w2_sk == 0) {
        const W2SplitPlan narrow = choose_w2_split_plan(ctx, pairs, d, d_ff, E, 1);
        if (narrow.us < w2.us) {
            f.tile = 1;
            w2 = narrow;
            f.w2_sk = choose_sk(ctx, use_of(1), pairs, E, d, d_ff, w2.splits, slots_of(use_of(1)));
        }
    }
    f.splits = f.w2_sk > 0 ? 1 : w2.splits;
    const moe::GemmUse u2 = use_of(f.tile);
    choose_skinny(ctx, f, pairs, d, d_ff, E);
    if (f.w13_sk > 0) f.sk_floats = moe::gemm_sk_part_floats(u13, f.w13_sk);
    if (f.w2_sk > 0) f.sk_floats = std::max(f.sk_floats, moe::gemm_sk_part_floats(u2, f.w2_sk));
    // the skinny w1/w3's split sums: both B operands (the SwiGLU case) per split
    if (f.skinny13 && f.w13_splits > 1)
        f.sk_floats = std::max<int64_t>(f.sk_floats, int64_t(f.w13_splits) * pairs * d_ff * 2);
    return f;
}

W2SplitPlan choose_w2_split_plan(moe_ctx* ctx, int64_t pairs, int64_t d, int64_t d_ff, int64_t E,
                                 int w2_tile) {
    static const int env = [] {
        const char* v = std::getenv("MOE_W2_SPLITS");
        return v != nullptr ? std::atoi(v) : 0;
    }();
    auto allowed = [&](int S) { return S == 1 || (d_ff > 0 && d_ff % (16 * S) == 0); };
    const bool pinned = env == 1 || env == 2 || env == 4;
    const moe::GemmUse use = w2_tile == 1 ? moe::GemmUse::W2Narrow : moe::GemmUse::W2;
    int& occ = w2_tile == 1 ? ctx->w2n_blocks_per_cu : ctx->w2_blocks_per_cu;
    if (occ == 0) occ = moe::gemm_blocks_per_cu(use);
    const moe::GemmTile tile = moe::gemm_tile(use);
    // the kernel deals only real tiles: sum over experts of ceil(n_e / BM),
    // expected ceil(pairs / BM) + E / 2 (each expert's last tile half full)
    const double tiles = double(expected_m_tiles(pairs, E, tile.bm) * moe::ceil_div(d, tile.bn));
    const double slots = double(int64_t(ctx->cus) * occ);
    // Time of S splits: ceil(tiles * S / slots) rounds of K / S steps, plus
    // the S - 1 extra partial row buffers w2 writes and the combine reads.
    // A round of n K steps: 3.9 n + 9 us on the wide tile (64 MFMAs per wave
    // and step, two workgroups per CU), 3.2 n us on the 128 x 128 one (32,
    // three per CU): fitted to rounds measured on MI355X at n = 28 (the
    // reference's d_ff 448), 88 (config 4) and 896 (config 3).
    const double nk = double(std::max<int64_t>(d_ff / 16, 1));
    auto round_us = [&](double n) { return w2_tile == 1 ? 3.2 * n : 3.9 * n + 9.0; };
    auto time_of = [&](int S) {
        const double rounds = std::ceil(tiles * S / slots);
        return rounds * round_us(nk / S) + (S - 1) * double(pairs) * d * 8.0 / 6e6;
    };
    if (pinned) {
        const int S = allowed(env) ? env : 1;
        return {S, time_of(S)};
    }
    W2SplitPlan best{1, 1e30};
    for (int S : {1, 2, 4}) {
        if (S > moe::kMaxW2Splits || !allowed(S)) continue;
        const double t = time_of(S);
        if (t < best.us * 0.99) best = {S, t};
    }
    return best;
}

// w2 with f.splits > 1 (layer path only): out_rows holds f.splits partial
// row buffers of pairs x d, one per K range, that the combine adds up.
// sk_part: f.sk_floats floats for the stream-K launches' partial tiles.
void expert_ffn(moe_ctx* ctx, const float* x, const int32_t* perm,
                const int32_t* offsets, const float* w1, const float* w3,
                const float* w2, int act, int64_t T, int64_t k, int64_t d,
                int64_t d_ff, int64_t E, float* h, float* out_rows, hipStream_t s,
                const FfnPlan& f, float* sk_part) {
    const int64_t pairs = T * k;
    if (pairs == 0 || d == 0) return;
    const bool swiglu = act == MOE_ACT_SWIGLU;
    if (d_ff > 0) {
        const moe::GemmTile tile =
            moe::gemm_tile(f.w13_tile == 1 ? moe::GemmUse::W13Tall : moe::GemmUse::W13);
        moe::GemmArgs a{};
        a.tile = f.w13_tile;
        a.A = x;
        a.lda = d;
        a.gather = perm;
        a.gather_rows = T;
        a.B0 = w1;
        a.B1 = swiglu ? w3 : w1;
        a.ldb = d;
        a.b_expert_stride = d_ff * d;
        a.C = h;
        a.ldc = d_ff;
        a.N = d_ff;
        a.K = d;
        a.offsets = offsets;
        a.rows_limit = pairs;
        a.E = static_cast<int32_t>(E);
        a.m_tiles = static_cast<int32_t>(grouped_m_tiles(pairs, E, tile.bm));
        a.n_tiles = static_cast<int32_t>(moe::ceil_div(d_ff, tile.bn));
        moe::require(int64_t(a.m_tiles) * a.n_tiles <= INT32_MAX, "w13 grid too large");
        if (f.w13_sk > 0) {
            a.sk_grid = f.w13_sk;
            a.sk_part = sk_part;
        }
        if (f.skinny13 && f.w13_splits > 1) {
            a.k_splits = f.w13_splits;
            a.k_split_len = d / f.w13_splits;
            a.sk_part = sk_part;
        }
        const bool vec = d % 4 == 0 && aligned16(x) && aligned16(w1) && (!swiglu || aligned16(w3));
        if (f.skinny13 && !vec) {  // unaligned rows: one 128x128 tile per workgroup, K whole
            a.tile = 0;
            a.k_splits = 1;
            a.k_split_len = 0;
            a.sk_part = nullptr;
        }
        ctx->launch(swiglu ? "expert_w13_swiglu" : "expert_w1_silu", s, [&] {
            moe::launch_gemm(a, false, true, swiglu ? moe::EPI_SWIGLU : moe::EPI_SILU, vec, s);
        });
    }
    const moe::GemmTile tile =
        moe::gemm_tile(f.tile == 1 ? moe::GemmUse::W2Narrow : moe::GemmUse::W2);
    moe::GemmArgs b{};
    b.tile = f.tile;
    b.A = d_ff > 0 ? h : out_rows;
    b.lda = d_ff;
    b.B0 = d_ff > 0 ? w2 : out_rows;
    b.B1 = b.B0;
    b.ldb = d_ff;
    b.b_expert_stride = d * d_ff;
    b.C = out_rows;
    b.ldc = d;
    b.N = d;
    b.K = d_ff;
    b.offsets = offsets;
    b.rows_limit = pairs;
    b.E = static_cast<int32_t>(E);
    b.m_tiles = static_cast<int32_t>(grouped_m_tiles(pairs, E, tile.bm));
    b.n_tiles = static_cast<int32_t>(moe::ceil_div(d, tile.bn));
    if (f.splits > 1) {
        b.k_splits = f.splits;
        b.k_split_len = moe::ceil_div(moe::ceil_div(d_ff, f.splits), 16) * 16;
        b.c_split_stride = pairs * d;
    }
    if (f.w2_sk > 0 && d_ff > 0) {
        b.sk_grid = f.w2_sk;
        b.sk_part = sk_part;
    }
    moe::require(int64_t(b.m_tiles) * b.n_tiles * std::max(f.splits, 1) <= INT32_MAX,
                 "w2 grid too large");
    const bool vec = d_ff % 4 == 0 && aligned16(h) && aligned16(w2);
    if (f.skinny2 && !vec) b.tile = 0;  // unaligned rows: the wide tile, the same K splits
    ctx->launch("expert_w2", s, [&] { moe::launch_gemm(b, false, true, moe::EPI_STORE, vec, s); });
}

void check_desc(const moe_layer_desc* desc) {
    check_ptr(desc, "desc");
    check_routing(desc->T, desc->E, desc->k);
    check_dims(desc->d, "d");
    check_dims(desc->d_ff, "d_ff");
    moe::require(desc->act == MOE_ACT_SWIGLU || desc->act == MOE_ACT_SILU_MLP, "unknown act");
    moe::require(desc->router == MOE_ROUTER_PHI_QUANT || desc->router == MOE_ROUTER_SOFTMAX_TOPK,
                 "unknown router mode");
    moe::require(desc->contract == MOE_CONTRACT_NONE || desc->contract == MOE_CONTRACT_FMA,
                 "unknown contract mode");
    moe::require(desc->norm == MOE_NORM_NONE || desc->norm == MOE_NORM_LAYER ||
                     desc->norm == MOE_NORM_RMS,
                 "unknown norm");
    moe::require(desc->residual == 0 || desc->residual == 1, "residual must be 0 or 1");
}

// Workspace layout of moe_layer_forward; with base == nullptr it only sizes.
struct LayerWs {
    float* logits;
    int32_t* idx;
    float* w;
    int32_t* counts;
    int32_t* offsets;
    int32_t* perm;
    int32_t* inv;
    float* h;
    float* out_rows;
    float* sk_part;    // stream-K partial tiles of w1/w3 and w2 (FfnPlan::sk_floats)
    float* norm_mean;  // MOE_NORM_LAYER / RMS: per-token statistics
    float* norm_inv;
    float* xnorm;      // MOE_NORM_LAYER / RMS: the normalised x [T, d] the experts read
    size_t bytes;
};

// f: the layer's FFN plan (choose_ffn_plan); out_rows holds f.splits
// partial row buffers, sk_part the stream-K partial tiles.
LayerWs carve_layer(void* base, const moe_layer_desc& d, const FfnPlan& f) {
    Carve c(base);
    LayerWs w{};
    const int64_t pairs = d.T * d.k;
    const int64_t nb = moe::ceil_div(d.T, moe::kPermTokens);
    w.logits = c.take<float>(d.T * d.E);
    w.idx = c.take<int32_t>(pairs);
    w.w = c.take<float>(pairs);
    w.counts = c.take<int32_t>(d.E * nb);
    w.offsets = c.take<int32_t>(d.E + 1);
    w.perm = c.take<int32_t>(pairs);
    w.inv = c.take<int32_t>(pairs);
    w.h = c.take<float>(pairs * d.d_ff);
    w.out_rows = c.take<float>(pairs * d.d * std::max(f.splits, 1));
    w.sk_part = f.sk_floats > 0 ? c.take<float>(f.sk_floats) : nullptr;
    if (d.norm != MOE_NORM_NONE) {
        w.norm_mean = c.take<float>(d.T);
        w.norm_inv = c.take<float>(d.T);
        w.xnorm = c.take<float>(d.T * d.d);
    }
    w.bytes = c.off + 256;
    return w;
}

// The MoE layer forward on a workspace at `base` carved by carve_layer
// (the context's grow-only workspace, or the no-alloc scratch).
void layer_forward(moe_ctx* ctx, const moe_layer_desc& D, const moe_layer_weights& weights,
                   const float* x, float* y, int32_t* topk_idx_out, float* topk_w_out,
                   hipStream_t s, void* base, const FfnPlan& plan) {
    check_ptr(x, "x");
    check_ptr(y, "y");
    check_ptr(weights.gate_w, "gate_w");
    if (D.d_ff > 0) {
        check_ptr(weights.w1, "w1");
        check_ptr(weights.w2, "w2");
        if (D.act == MOE_ACT_SWIGLU) check_ptr(weights.w3, "w3");
    }
    moe::require(D.d % 4 != 0 || (aligned16(x) && aligned16(y)),
                 "layer: x and y must be 16-byte aligned");
    const bool norm = D.norm != MOE_NORM_NONE, rms = D.norm == MOE_NORM_RMS;
    if (norm) {
        moe::require(D.d > 0, "norm: d must be > 0");
        check_ptr(weights.norm_w, "norm_w");
        if (!rms) check_ptr(weights.norm_b, "norm_b");
    }
    const int splits = plan.splits;
    LayerWs ws = carve_layer(base, D, plan);
    int32_t* idx = topk_idx_out != nullptr ? topk_idx_out : ws.idx;
    float* w = topk_w_out != nullptr ? topk_w_out : ws.w;

    // The experts' input: x, or its normalised copy (written once, read
    // by the gate and the w1/w3 GEMM; the residual stays x).
    const float* xin = x;
    if (norm) {
        ctx->launch(rms ? "rms_norm" : "layer_norm", s, [&] {
            moe::launch_layer_norm(x, weights.norm_w, rms ? nullptr : weights.norm_b, D.T, D.d,
                                   D.norm_eps, D.contract, rms, ws.norm_mean, ws.norm_inv,
                                   ws.xnorm, ctx->cus, s);
        });
        xin = ws.xnorm;
    }

    // the gate also clears the counts route_count adds into (none for one block)
    const int64_t nb = moe::ceil_div(D.T, moe::kPermTokens);
    const bool one_block = moe::route_place_one_fits(D.T, D.E, D.k, D.router);
    ctx->launch("gate_logits", s, [&] {
        moe::launch_gate_logits(xin, weights.gate_w, ws.logits, D.T, D.d, D.E, D.contract, s,
                                reinterpret_cast<uint32_t*>(ws.counts), one_block ? 0 : D.E * nb);
    });
    if (one_block) {
        // one permutation block: routing, offsets and placement in one launch
        ctx->launch("route_place", s, [&] {
            moe::launch_route_place_one(ws.logits, weights.expert_bias, D.T, D.E, D.k, D.router,
                                        D.quantum, D.tie_eps, idx, w, ws.perm, ws.inv,
                                        ws.offsets, s);
        });
    } else {
        // routing and the per-block expert counts: one launch
        ctx->launch("route_count", s, [&] {
            moe::launch_route_count(ws.logits, weights.expert_bias, D.T, D.E, D.k, D.router,
                                    D.quantum, D.tie_eps, idx, w, ws.counts, s);
        });
        if (D.E * nb <= moe::kPlaceScanMax) {
            // the scan folded into the placement: one launch
            ctx->launch("perm_place", s, [&] {
                moe::launch_perm_place_scan(idx, D.T, D.k, D.E, ws.counts, ws.perm, ws.inv,
                                            ws.offsets, s);
            });
        } else {
            ctx->launch("perm_scan", s,
                        [&] { moe::launch_perm_scan(ws.counts, nb, D.E, ws.offsets, s); });
            ctx->launch("perm_place", s, [&] {
                moe::launch_perm_place(idx, D.T, D.k, D.E, ws.counts, ws.perm, ws.inv, s);
            });
        }
    }
    expert_ffn(ctx, xin, ws.perm, ws.offsets, weights.w1, weights.w3, weights.w2, D.act, D.T, D.k,
               D.d, D.d_ff, D.E, ws.h, ws.out_rows, s, plan, ws.sk_part);
    ctx->launch("combine", s, [&] {
        moe::launch_combine(ws.out_rows, idx, w, ws.inv, D.residual ? x : nullptr, y, D.T, D.k,
                            D.d, D.T * D.k, D.contract, splits, D.T * D.k * D.d, s);
    });
}

// Suspends a context's kernel timing for the duration of a call.
struct TimingPause {
    moe_ctx* ctx;
    bool was;
    explicit TimingPause(moe_ctx* c) : ctx(c), was(c->timing) { c->timing = false; }
    ~TimingPause() { ctx->timing = was; }
};

}  // namespace

void* moe_ctx::workspace(size_t bytes) {
    if (bytes > ws_bytes) {
        if (ws != nullptr) {
            // the old buffer may still be read by queued kernels
            moe::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
            moe::hip_check(hipFree(ws), "hipFree workspace");
            ws = nullptr;
            ws_bytes = 0;
        }
        const size_t grow = std::max(bytes, ws_bytes + ws_bytes / 2);
        moe::hip_check(hipMalloc(&ws, grow), "hipMalloc workspace");
        ws_bytes = grow;
    }
    return ws;
}

void moe_ctx::collect() {
    for (auto& p : pending) {
        moe::hip_check(hipEventSynchronize(p.stop), "hipEventSynchronize");
        float ms = 0.0f;
        moe::hip_check(hipEventElapsedTime(&ms, p.start, p.stop), "hipEventElapsedTime");
        auto& slot = totals[p.name];
        slot.first += ms;
        slot.second += 1;
        event_pool.emplace_back(p.start, p.stop);
    }
    pending.clear();
}

extern "C" {

const char* moe_last_error(void) { return g_last_error.c_str(); }

const char* moe_version(void) { return "moe_amd 0.1 gfx950"; }

int moe_ctx_create(int device, moe_ctx** out) {
    return guarded([&] {
        check_ptr(out, "out");
        *out = nullptr;
        int n = 0;
        moe::hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
        moe::require(device >= 0 && device < n, "device ordinal out of range");
        hipDeviceProp_t prop;
        moe::hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            throw moe::Unsupported(std::string("kernels are built for gfx950, device is ") +
                                   prop.gcnArchName);
        void* scr = nullptr;
        {
            DeviceScope dev(device);
            scr = bind_scratch(device);
        }
        auto* c = new moe_ctx();
        c->device = device;
        c->cus = prop.multiProcessorCount;
        c->scratch = scr;
        *out = c;
    });
}

int moe_ctx_destroy(moe_ctx* ctx) {
    return guarded([&] {
        if (ctx == nullptr) return;
        DeviceScope dev(ctx->device);
        moe::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        for (auto& p : ctx->pending) ctx->event_pool.emplace_back(p.start, p.stop);
        for (auto& e : ctx->event_pool) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        if (ctx->ws != nullptr) (void)hipFree(ctx->ws);
        delete ctx;
    });
}

int moe_ctx_reserve(moe_ctx* ctx, const moe_layer_desc* desc) {
    return guarded([&] {
        check_ctx(ctx);
        check_desc(desc);
        DeviceScope dev(ctx->device);
        const FfnPlan plan =
            choose_ffn_plan(ctx, desc->T * desc->k, desc->d, desc->d_ff, desc->E);
        ctx->workspace(carve_layer(nullptr, *desc, plan).bytes);
    });
}

int moe_ctx_workspace_bytes(moe_ctx* ctx, int64_t* bytes) {
    return guarded([&] {
        check_ctx(ctx);
        check_ptr(bytes, "bytes");
        *bytes = static_cast<int64_t>(ctx->ws_bytes);
    });
}

int moe_ctx_set_stream_k(moe_ctx* ctx, int mode) {
    return guarded([&] {
        check_ctx(ctx);
        moe::require(mode >= -1 && mode <= 1, "stream-K mode must be -1, 0 or 1");
        ctx->sk_mode = mode;
    });
}

int moe_sgemm_plan(moe_ctx* ctx, int nn, int64_t M, int64_t N, int64_t K, int32_t* tile,
                   int32_t* splits) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(M, "M");
        check_dims(N, "N");
        check_dims(K, "K");
        check_ptr(tile, "tile");
        check_ptr(splits, "splits");
        DeviceScope dev(ctx->device);
        // the direct-load condition of sgemm() for 16-byte aligned operands
        const bool direct = K % 16 == 0 && (nn == 0 || N % 4 == 0);
        const DensePlan plan = plan_dense(ctx, nn != 0, direct, M, N, K);
        *tile = plan.tile;
        *splits = plan.splits;
    });
}

int moe_ctx_set_timing(moe_ctx* ctx, int enabled) {
    return guarded([&] {
        check_ctx(ctx);
        ctx->timing = enabled != 0;
    });
}

int moe_ctx_reset_timing(moe_ctx* ctx) {
    return guarded([&] {
        check_ctx(ctx);
        DeviceScope dev(ctx->device);
        ctx->collect();
        ctx->totals.clear();
    });
}

int moe_ctx_kernel_times(moe_ctx* ctx, const char** names, double* total_ms,
                         int64_t* launches, int cap) {
    int count = 0;
    const int rc = guarded([&] {
        check_ctx(ctx);
        DeviceScope dev(ctx->device);
        ctx->collect();
        ctx->name_store.clear();
        for (auto& kv : ctx->totals) ctx->name_store.push_back(kv.first);
        int i = 0;
        for (auto& kv : ctx->totals) {
            if (i < cap) {
                if (names) names[i] = ctx->name_store[i].c_str();
                if (total_ms) total_ms[i] = kv.second.first;
                if (launches) launches[i] = kv.second.second;
            }
            ++i;
        }
        count = i;
    });
    return rc == MOE_OK ? count : -rc;
}

int moe_sgemm_nt(moe_ctx* ctx, const float* A, const float* B, const float* bias,
                 float* C, int64_t M, int64_t N, int64_t K, void* stream) {
    return guarded([&] { sgemm(ctx, false, A, B, bias, C, M, N, K, stream); });
}

int moe_sgemm_nn(moe_ctx* ctx, const float* A, const float* B, const float* bias,
                 float* C, int64_t M, int64_t N, int64_t K, void* stream) {
    return guarded([&] { sgemm(ctx, true, A, B, bias, C, M, N, K, stream); });
}

int moe_sgemm_nt_residual(moe_ctx* ctx, const float* A, const float* B, const float* bias,
                          const float* R, float* C, int64_t M, int64_t N, int64_t K,
                          void* stream) {
    return guarded([&] {
        if (M > 0 && N > 0) check_ptr(R, "R");
        sgemm(ctx, false, A, B, bias, C, M, N, K, stream, R);
    });
}

int moe_launch_floor(moe_ctx* ctx, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("empty", s, [&] { moe::launch_empty(s); });
    });
}

int moe_silu(moe_ctx* ctx, const float* x, float* y, int64_t n, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        moe::require(n >= 0, "n must be >= 0");
        if (n == 0) return;
        check_ptr(x, "x");
        check_ptr(y, "y");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("silu", s, [&] { moe::launch_silu(x, y, n, s); });
    });
}

int moe_mul(moe_ctx* ctx, const float* a, const float* b, float* c, int64_t n, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        moe::require(n >= 0, "n must be >= 0");
        if (n == 0) return;
        check_ptr(a, "a");
        check_ptr(b, "b");
        check_ptr(c, "c");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("mul", s, [&] { moe::launch_mul(a, b, c, n, s); });
    });
}

int moe_gate_logits(moe_ctx* ctx, const float* x, const float* gate_w, float* logits,
                    int64_t T, int64_t d, int64_t E, int contract, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(T, "T");
        check_dims(d, "d");
        moe::require(E >= 1 && E <= moe::kMaxExperts, "E must be in [1, 1024]");
        moe::require(contract == MOE_CONTRACT_NONE || contract == MOE_CONTRACT_FMA,
                     "unknown contract mode");
        if (T == 0) return;
        check_ptr(logits, "logits");
        if (d > 0) {
            check_ptr(x, "x");
            check_ptr(gate_w, "gate_w");
        }
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("gate_logits", s, [&] {
            moe::launch_gate_logits(x, gate_w, logits, T, d, E, contract, s);
        });
    });
}

int moe_layer_norm(moe_ctx* ctx, const float* x, const float* weight, const float* bias,
                   float eps, int64_t rows, int64_t h, int contract, float* y, float* row_mean,
                   float* row_inv, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(rows, "rows");
        check_dims(h, "h");
        moe::require(contract == MOE_CONTRACT_NONE || contract == MOE_CONTRACT_FMA,
                     "unknown contract mode");
        if (rows == 0) return;
        moe::require(h > 0, "layer norm: h must be > 0");
        check_ptr(x, "x");
        if (y != nullptr) {
            check_ptr(weight, "weight");
            check_ptr(bias, "bias");
        }
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        if (row_mean == nullptr || row_inv == nullptr) {
            // statistics the caller does not keep live in the workspace
            Carve c(ctx->workspace(size_t(2 * rows) * sizeof(float) + 512));
            if (row_mean == nullptr) row_mean = c.take<float>(rows);
            if (row_inv == nullptr) row_inv = c.take<float>(rows);
        }
        ctx->launch("layer_norm", s, [&] {
            moe::launch_layer_norm(x, weight, bias, rows, h, eps, contract, false, row_mean,
                                   row_inv, y, ctx->cus, s);
        });
    });
}

int moe_rope_table(float theta, int64_t head_dim, int64_t positions, float* table) {
    return guarded([&] {
        moe::require(head_dim > 0 && head_dim % 2 == 0, "head_dim must be even and > 0");
        check_dims(positions, "positions");
        if (positions == 0) return;
        check_ptr(table, "table");
        // the libm calls of the reference's host-built table, in float
        const int64_t half = head_dim / 2;
        for (int64_t si = 0; si < positions; ++si)
            for (int64_t j = 0; j < half; ++j) {
                const float inv = powf(theta, -2.0f * static_cast<float>(j) /
                                                  static_cast<float>(head_dim));
                table[(si * half + j) * 2] = cosf(static_cast<float>(si) * inv);
                table[(si * half + j) * 2 + 1] = sinf(static_cast<float>(si) * inv);
            }
    });
}

int moe_rope(moe_ctx* ctx, float* q, float* k, const float* table, int64_t table_positions,
             int64_t batch, int64_t seq_len, int64_t first_pos, int64_t q_heads,
             int64_t kv_heads, int64_t head_dim, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(batch, "batch");
        check_dims(seq_len, "seq_len");
        moe::require(q_heads >= 0 && kv_heads >= 0, "heads must be >= 0");
        moe::require(head_dim > 0 && head_dim % 2 == 0, "head_dim must be even and > 0");
        const int64_t rows = batch * seq_len;
        if (rows == 0 || q_heads + kv_heads == 0) return;
        moe::require(first_pos >= 0, "first_pos must be >= 0");
        moe::require(table_positions >= first_pos + seq_len,
                     "the rope table needs first_pos + seq_len positions");
        check_ptr(table, "table");
        if (q_heads > 0) check_ptr(q, "q");
        if (kv_heads > 0) check_ptr(k, "k");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("rope", s, [&] {
            moe::launch_rope(q, k, table, rows, seq_len, first_pos, q_heads, kv_heads, head_dim,
                             s);
        });
    });
}

int moe_attention(moe_ctx* ctx, const float* q, const float* k, const float* v, float* out,
                  int64_t batch, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                  int64_t head_dim, int64_t window, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(batch, "batch");
        check_dims(seq_len, "seq_len");
        moe::require(kv_heads >= 1 && q_heads >= kv_heads && q_heads % kv_heads == 0,
                     "q_heads must be a positive multiple of kv_heads");
        moe::require(head_dim > 0, "head_dim must be > 0");
        moe::require(window >= 0, "window must be >= 0 (0 = unlimited)");
        if (batch == 0 || seq_len == 0) return;
        check_ptr(q, "q");
        check_ptr(k, "k");
        check_ptr(v, "v");
        check_ptr(out, "out");
        const int64_t w = window >= seq_len ? 0 : window;
        const int64_t zb = batch * q_heads;
        moe::require(zb <= 65535, "attention: batch * q_heads exceeds the grid's y range");
        const bool aligned = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        // head_dim 64 / 128: one fused pass, any seq_len, no workspace
        // (MOE_ATTN_FLASH=0 keeps the three-launch path, for comparison)
        static const int flash = env_int("MOE_ATTN_FLASH", 1);
        if (flash != 0 && aligned && (head_dim == 64 || head_dim == 128) &&
            seq_len <= INT32_MAX) {
            ctx->launch("attn_flash", s, [&] {
                moe::launch_flash_attention(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                            head_dim, w, s);
            });
            return;
        }
        if (head_dim % 16 != 0 || seq_len % 16 != 0 || !aligned)
            throw moe::Unsupported(
                "attention needs head_dim 64 or 128, or head_dim and seq_len multiples of 16, "
                "and 16-byte aligned q/k/v/out");
        const int64_t S = seq_len, qw = q_heads * head_dim, kw = kv_heads * head_dim;
        float* scores = static_cast<float*>(ctx->workspace(size_t(zb) * S * S * sizeof(float)));
        // scores[b, h] = Q[b, :, h] K[b, :, h / group]^T   (queries x keys)
        moe::GemmArgs a{};
        a.A = q;
        a.lda = qw;
        a.B0 = a.B1 = k;
        a.ldb = kw;
        a.C = scores;
        a.ldc = S;
        a.M = S;
        a.N = S;
        a.K = head_dim;
        a.batch_inner = static_cast<int32_t>(q_heads);
        a.b_group = static_cast<int32_t>(q_heads / kv_heads);
        a.a_so = S * qw;
        a.a_si = head_dim;
        a.b_so = S * kw;
        a.b_si = head_dim;
        a.c_so = q_heads * S * S;
        a.c_si = S * S;
        a.causal = moe::CAUSAL_SCORES;
        a.window = static_cast<int32_t>(w);
        ctx->launch("attn_scores", s,
                    [&] { moe::launch_gemm_batched(a, false, static_cast<int>(zb), s); });
        ctx->launch("attn_softmax", s,
                    [&] { moe::launch_attn_softmax(scores, zb, S, head_dim, w, s); });
        // out[b, :, h] = P[b, h] V[b, :, h / group]   (queries x head_dim)
        moe::GemmArgs b{};
        b.A = scores;
        b.lda = S;
        b.B0 = b.B1 = v;
        b.ldb = kw;
        b.C = out;
        b.ldc = qw;
        b.M = S;
        b.N = head_dim;
        b.K = S;
        b.batch_inner = static_cast<int32_t>(q_heads);
        b.b_group = static_cast<int32_t>(q_heads / kv_heads);
        b.a_so = q_heads * S * S;
        b.a_si = S * S;
        b.b_so = S * kw;
        b.b_si = head_dim;
        b.c_so = S * qw;
        b.c_si = head_dim;
        b.causal = moe::CAUSAL_PV;
        b.window = static_cast<int32_t>(w);
        ctx->launch("attn_pv", s,
                    [&] { moe::launch_gemm_batched(b, true, static_cast<int>(zb), s); });
    });
}

int moe_attention_last(moe_ctx* ctx, const float* q, const float* k, const float* v, float* out,
                       int64_t batch, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                       int64_t head_dim, int64_t window, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(batch, "batch");
        check_dims(seq_len, "seq_len");
        moe::require(kv_heads >= 1 && q_heads >= kv_heads && q_heads % kv_heads == 0,
                     "q_heads must be a positive multiple of kv_heads");
        moe::require(head_dim > 0, "head_dim must be > 0");
        moe::require(window >= 0, "window must be >= 0 (0 = unlimited)");
        if (batch == 0 || seq_len == 0) return;
        check_ptr(q, "q");
        check_ptr(k, "k");
        check_ptr(v, "v");
        check_ptr(out, "out");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        float* scores =
            static_cast<float*>(ctx->workspace(size_t(batch * q_heads * seq_len) * sizeof(float)));
        ctx->launch("attn_last", s, [&] {
            moe::launch_attn_last(q, k, v, out, scores, batch, seq_len, q_heads, kv_heads,
                                  head_dim, window, s);
        });
    });
}

int moe_rope_rows(moe_ctx* ctx, float* q, float* k, const float* table, int64_t table_positions,
                  const int32_t* positions, int64_t rows, int64_t q_heads, int64_t kv_heads,
                  int64_t head_dim, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(rows, "rows");
        moe::require(q_heads >= 0 && kv_heads >= 0, "heads must be >= 0");
        moe::require(head_dim > 0 && head_dim % 2 == 0, "head_dim must be even and > 0");
        if (rows == 0 || q_heads + kv_heads == 0) return;
        moe::require(table_positions >= 1, "the rope table needs at least one position");
        check_ptr(table, "table");
        check_ptr(positions, "positions");
        if (q_heads > 0) check_ptr(q, "q");
        if (kv_heads > 0) check_ptr(k, "k");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("rope", s, [&] {
            moe::launch_rope_rows(q, k, table, table_positions, positions, rows, q_heads,
                                  kv_heads, head_dim, s);
        });
    });
}

int moe_attention_paths(moe_ctx* ctx, const float* q, const float* k, const float* v, float* out,
                        int64_t nq, int64_t kv_rows, const int32_t* key_rows,
                        const int32_t* key_beg, const int32_t* key_end, int64_t max_len,
                        int64_t key_total, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                        int64_t window, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(nq, "nq");
        check_dims(kv_rows, "kv_rows");
        moe::require(kv_heads >= 1 && q_heads >= kv_heads && q_heads % kv_heads == 0,
                     "q_heads must be a positive multiple of kv_heads");
        moe::require(head_dim > 0, "head_dim must be > 0");
        moe::require(window >= 0, "window must be >= 0 (0 = unlimited)");
        moe::require(max_len >= 0 && key_total >= 0, "max_len and key_total must be >= 0");
        if (nq == 0) return;
        moe::require(kv_rows >= 1, "kv_rows must be >= 1");
        check_ptr(q, "q");
        check_ptr(k, "k");
        check_ptr(v, "v");
        check_ptr(out, "out");
        check_ptr(key_rows, "key_rows");
        check_ptr(key_beg, "key_beg");
        check_ptr(key_end, "key_end");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        float* scores = nullptr;
        int64_t scores_floats = 0;
        if (max_len > 8192) {
            scores_floats = std::max<int64_t>(key_total, 1) * q_heads;
            scores = static_cast<float*>(ctx->workspace(size_t(scores_floats) * sizeof(float)));
        }
        ctx->launch("attn_paths", s, [&] {
            moe::launch_attn_paths(q, k, v, out, scores, key_rows, key_beg, key_end, nq, kv_rows,
                                   max_len, key_total, scores_floats, q_heads, kv_heads,
                                   head_dim, window, s);
        });
    });
}

int moe_add(moe_ctx* ctx, float* a, const float* b, int64_t n, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        moe::require(n >= 0, "n must be >= 0");
        if (n == 0) return;
        check_ptr(a, "a");
        check_ptr(b, "b");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("add", s, [&] { moe::launch_add(a, b, n, s); });
    });
}

int moe_add_bias(moe_ctx* ctx, float* a, const float* bias, int64_t rows, int64_t cols,
                 void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(rows, "rows");
        check_dims(cols, "cols");
        if (rows == 0 || cols == 0) return;
        check_ptr(a, "a");
        check_ptr(bias, "bias");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("add_bias", s, [&] { moe::launch_add_bias(a, bias, rows, cols, s); });
    });
}

int moe_embed(moe_ctx* ctx, const float* table, const int32_t* tokens, int64_t n, int64_t d,
              int64_t vocab, float* out, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(n, "n");
        check_dims(d, "d");
        check_dims(vocab, "vocab");
        if (n == 0 || d == 0) return;
        check_ptr(table, "table");
        check_ptr(tokens, "tokens");
        check_ptr(out, "out");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("embed", s, [&] { moe::launch_embed(table, tokens, n, d, vocab, out, s); });
    });
}

int moe_rms_norm(moe_ctx* ctx, const float* x, const float* weight, float eps, int64_t rows,
                 int64_t h, int contract, float* y, float* row_inv, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(rows, "rows");
        check_dims(h, "h");
        moe::require(contract == MOE_CONTRACT_NONE || contract == MOE_CONTRACT_FMA,
                     "unknown contract mode");
        if (rows == 0) return;
        moe::require(h > 0, "rms norm: h must be > 0");
        check_ptr(x, "x");
        if (y != nullptr) check_ptr(weight, "weight");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        if (row_inv == nullptr) {
            Carve c(ctx->workspace(size_t(rows) * sizeof(float) + 256));
            row_inv = c.take<float>(rows);
        }
        ctx->launch("rms_norm", s, [&] {
            moe::launch_layer_norm(x, weight, nullptr, rows, h, eps, contract, true, nullptr,
                                   row_inv, y, ctx->cus, s);
        });
    });
}

int moe_route(moe_ctx* ctx, const float* logits, const float* expert_bias, int64_t T,
              int64_t E, int64_t k, int mode, float quantum, float tie_eps,
              int32_t* topk_idx, float* topk_w, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_routing(T, E, k);
        moe::require(mode == MOE_ROUTER_PHI_QUANT || mode == MOE_ROUTER_SOFTMAX_TOPK,
                     "unknown router mode");
        if (T == 0) return;
        check_ptr(logits, "logits");
        check_ptr(topk_idx, "topk_idx");
        check_ptr(topk_w, "topk_w");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch(mode == MOE_ROUTER_PHI_QUANT ? "route_phi" : "route_softmax", s, [&] {
            moe::launch_route(logits, expert_bias, T, E, k, mode, quantum, tie_eps, topk_idx,
                              topk_w, s);
        });
    });
}

int moe_permute(moe_ctx* ctx, const int32_t* topk_idx, int64_t T, int64_t k, int64_t E,
                int32_t* expert_offsets, int32_t* perm, int32_t* inv, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_routing(T, E, k);
        check_ptr(expert_offsets, "expert_offsets");
        if (T > 0) {
            check_ptr(topk_idx, "topk_idx");
            check_ptr(perm, "perm");
            check_ptr(inv, "inv");
        }
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        const int64_t nb = moe::ceil_div(T, moe::kPermTokens);
        auto* counts = static_cast<int32_t*>(ctx->workspace(static_cast<size_t>(E * nb + 1) * 4));
        ctx->launch("perm_count", s, [&] { moe::launch_perm_count(topk_idx, T, k, E, counts, s); });
        ctx->launch("perm_scan", s,
                    [&] { moe::launch_perm_scan(counts, nb, E, expert_offsets, s); });
        ctx->launch("perm_place", s,
                    [&] { moe::launch_perm_place(topk_idx, T, k, E, counts, perm, inv, s); });
    });
}

int moe_expert_ffn_grouped(moe_ctx* ctx, const float* x, const int32_t* perm,
                           const int32_t* expert_offsets, const float* w1, const float* w3,
                           const float* w2, int act, int64_t T, int64_t k, int64_t d,
                           int64_t d_ff, int64_t E, float* h, float* out_rows, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_routing(T, E, k);
        check_dims(d, "d");
        check_dims(d_ff, "d_ff");
        moe::require(act == MOE_ACT_SWIGLU || act == MOE_ACT_SILU_MLP, "unknown act");
        if (T == 0 || d == 0) return;
        check_ptr(x, "x");
        check_ptr(perm, "perm");
        check_ptr(expert_offsets, "expert_offsets");
        check_ptr(out_rows, "out_rows");
        if (d_ff > 0) {
            check_ptr(w1, "w1");
            check_ptr(w2, "w2");
            check_ptr(h, "h");
            if (act == MOE_ACT_SWIGLU) check_ptr(w3, "w3");
        }
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        // one K range for w2 (out_rows holds one row per pair); stream-K
        // where the planner takes it, its partial tiles in the workspace
        FfnPlan plan = choose_ffn_plan(ctx, T * k, d, d_ff, E);
        if (plan.splits > 1) plan.splits = 1;
        float* sk_part = nullptr;
        if (plan.sk_floats > 0)
            sk_part = static_cast<float*>(ctx->workspace(size_t(plan.sk_floats) * sizeof(float)));
        expert_ffn(ctx, x, perm, expert_offsets, w1, w3, w2, act, T, k, d, d_ff, E, h, out_rows,
                   s, plan, sk_part);
    });
}

int moe_combine(moe_ctx* ctx, const float* out_rows, const int32_t* topk_idx,
                const float* topk_w, const int32_t* inv, const float* resid, float* y,
                int64_t T, int64_t k, int64_t d, int contract, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_dims(T, "T");
        check_dims(d, "d");
        moe::require(k >= 1 && k <= moe::kMaxTopK, "k must be in [1, 32]");
        moe::require(contract == MOE_CONTRACT_NONE || contract == MOE_CONTRACT_FMA,
                     "unknown contract mode");
        if (T == 0 || d == 0) return;
        check_ptr(out_rows, "out_rows");
        check_ptr(topk_idx, "topk_idx");
        check_ptr(topk_w, "topk_w");
        check_ptr(inv, "inv");
        check_ptr(y, "y");
        moe::require(d % 4 != 0 || (aligned16(out_rows) && aligned16(y) &&
                                    (resid == nullptr || aligned16(resid))),
                     "combine: rows of width d % 4 == 0 must be 16-byte aligned");
        DeviceScope dev(ctx->device);
        hipStream_t s = as_stream(stream);
        ctx->launch("combine", s, [&] {
            moe::launch_combine(out_rows, topk_idx, topk_w, inv, resid, y, T, k, d, T * k,
                                contract, 1, 0, s);
        });
    });
}

int moe_layer_forward(moe_ctx* ctx, const moe_layer_desc* desc,
                      const moe_layer_weights* weights, const float* x, float* y,
                      int32_t* topk_idx_out, float* topk_w_out, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_desc(desc);
        check_ptr(weights, "weights");
        if (desc->T == 0) return;
        DeviceScope dev(ctx->device);
        const FfnPlan plan =
            choose_ffn_plan(ctx, desc->T * desc->k, desc->d, desc->d_ff, desc->E);
        void* base = ctx->workspace(carve_layer(nullptr, *desc, plan).bytes);
        layer_forward(ctx, *desc, *weights, x, y, topk_idx_out, topk_w_out, as_stream(stream),
                      base, plan);
    });
}

int moe_layer_forward_noalloc(moe_ctx* ctx, const moe_layer_desc* desc,
                              const moe_layer_weights* weights, const float* x, float* y,
                              int32_t* topk_idx_out, float* topk_w_out, void* stream) {
    return guarded([&] {
        check_ctx(ctx);
        check_desc(desc);
        check_ptr(weights, "weights");
        if (desc->T == 0) return;
        moe::require(ctx->scratch != nullptr, "no-alloc scratch not bound to this context");
        DeviceScope dev(ctx->device);
        const FfnPlan plan =
            choose_ffn_plan(ctx, desc->T * desc->k, desc->d, desc->d_ff, desc->E);
        const size_t need = carve_layer(nullptr, *desc, plan).bytes;
        if (need > kNoAllocScratchBytes)
            throw moe::InvalidArg("moe_layer_forward_noalloc: this layer needs " +
                                  std::to_string(need) + " bytes of scratch, more than the " +
                                  std::to_string(kNoAllocScratchBytes) +
                                  " the library holds per GPU; use moe_layer_forward");
        // no events either: timing records them, and this entry point
        // creates nothing
        TimingPause pause(ctx);
        layer_forward(ctx, *desc, *weights, x, y, topk_idx_out, topk_w_out, as_stream(stream),
                      ctx->scratch, plan);
    });
}

int moe_layer_w2_splits(moe_ctx* ctx, const moe_layer_desc* desc, int32_t* splits) {
    return guarded([&] {
        check_ctx(ctx);
        check_desc(desc);
        check_ptr(splits, "splits");
        DeviceScope dev(ctx->device);
        *splits = choose_ffn_plan(ctx, desc->T * desc->k, desc->d, desc->d_ff, desc->E).splits;
    });
}

}  // extern "C"
