// Shared definitions of the gfx950 MoE library: the context, error
// propagation to the C ABI, and the launch wrapper that can bracket every
// kernel with HIP events.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/moe_amd.h"

namespace moe {

// A shape or argument the caller got wrong (MOE_ERR_INVALID).
struct InvalidArg : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
// An argument the kernels do not support (MOE_ERR_UNSUPPORTED).
struct Unsupported : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

inline void require(bool ok, const std::string& what) {
    if (!ok) throw InvalidArg(what);
}

constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, workgroups dealt round-robin

// Default GEMM raster group (m-tiles per n-sweep; 0 = every m-tile, i.e.
// m-fastest): 8, so each XCD's ~64 resident workgroups cover about 8
// m-tiles x 8 n-tiles and share every A and B panel 8 ways in its L2.
// Measured best on MI355X for the grouped expert GEMMs at config 3, config
// 5's w2 and the reference's layer shape (config 4 is 1 % faster m-fastest), and
// for the large dense shapes (8192^3 NT 128 -> 136 TFLOP/s).
constexpr int kGemmGroupM = 8;
// ... and for the grouped w1/w3 launches with at most 1024 K columns: 4 (same box, three
// runs each, config 5's layer 1.172 -> 1.164 ms, its K = 1024 w1/w3 1 % faster; the
// reference's w2 at K = 448, tried with it, was level or 0.2 % slower and keeps 8)
constexpr int kGemmGroupMShortK = 4;

// The GEMM uses whose tile shape the host needs for grid sizing.
// W2Narrow: the w2 GEMM on the 128x128 tile (GemmArgs::tile = 1 on the
// grouped EPI_STORE path), for widths d whose wide tile leaves few n-tiles.
// W13Tall: w1/w3 on the 256 x 64 tile (GemmArgs::tile = 1 on the grouped
// SwiGLU / SiLU path), for d_ff % 128 == 64.
enum class GemmUse { Dense, W13, W13Tall, W2, W2Narrow };
struct GemmTile {
    int bm, bn;
};
GemmTile gemm_tile(GemmUse use);
// Workgroups of the grouped kernel of `use` one CU holds at once.
int gemm_blocks_per_cu(GemmUse use);
// ... of its stream-K kernel (GemmArgs::sk_grid > 0).
int gemm_sk_blocks_per_cu(GemmUse use);
// Floats of GemmArgs::sk_part a stream-K launch of `use` on `grid`
// workgroups needs.
int64_t gemm_sk_part_floats(GemmUse use, int grid);
constexpr int kMaxW2Splits = 4;  // split-K of the layer's w2 (partials summed by the combine)

// Dense SGEMM tile shapes, GemmArgs::tile: 0 = 128x128 (any shape), 1 =
// 64x128 and 2 = 32x128 (direct-load path only: 16-byte aligned rows,
// K % 16 == 0, and for NN N % 4 == 0), 3 = 256x128 (direct path),
// 5 = 32x128 with K groups (direct ring path, K a multiple of 16 x groups,
// no K split, operands under 2 GiB).  Ids below kDenseTiles; 4 is the skinny
// kernel.
constexpr int kDenseTiles = 6;
// GemmArgs::tile of the skinny dense kernel (M <= 64, direct rows only; not
// one of the tile shapes the planner's tile loop weighs).
constexpr int kSkinnyTile = 4;
constexpr int kDenseKwTile = 5;
GemmTile dense_tile(int tile);
// Workgroups of dense tile shape `tile` (direct-load kernel) one CU holds at once.
int dense_blocks_per_cu(int tile, bool nn);
// K groups of a dense tile shape (1, or the K-group tiles' count).
int dense_tile_groups(int tile);
constexpr int kMaxDenseSplits = 16;  // split-K of a dense SGEMM (partials in the workspace)
// GemmArgs::tile of the grouped (expert) launches for layers whose experts
// hold few rows each: the grouped skinny kernel, w1/w3 and w2 alike.
constexpr int kGroupedSkinnyTile = 2;

// Routing constants.
constexpr int kPermTokens = 256;    // tokens per permutation block
constexpr int kMaxExperts = 1024;   // bitmap in LDS: E * 4 * 8 B = 32 KiB
constexpr int kMaxTopK = 32;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Kernel launch arguments of the GEMM engine (one struct, passed by value).
struct GemmArgs {
    const float* A;          // [rows, K] row-major, leading dim lda
    int64_t lda;
    const int32_t* gather;   // grouped: packed row -> token of A, or nullptr
    int64_t gather_rows;     // rows of A the gather may address (clamp)
    const float* B0;         // NT: [N, K]; NN: [K, N]
    const float* B1;         // second operand of the dual (SwiGLU) kernel
    int64_t ldb;
    int64_t b_expert_stride; // grouped: elements between experts' matrices
    const float* bias;       // [N] or nullptr
    float* C;                // output, leading dim ldc
    int64_t ldc;
    int64_t M, N, K;         // dense: M rows; grouped: per-expert N, K
    const int32_t* offsets;  // grouped: expert_offsets[E+1]
    int64_t rows_limit;      // grouped: packed rows of A / C (T*k); bounds every tile
    int32_t E;
    int32_t m_tiles;         // m-tiles covered by the grid (upper bound)
    int32_t n_tiles;
    int32_t group_m;         // raster: m-tiles that sweep the n-tiles together
    int32_t k_splits;        // K ranges computed by separate tiles (>= 1)
    int64_t k_split_len;     // K per split (a multiple of 16)
    int64_t c_split_stride;  // elements between the outputs of consecutive splits
    int32_t tile;            // dense: tile shape (kDenseTiles); grouped w2: 1 = 128x128;
                             // grouped w1/w3: 1 = 256x64
    // Batched dense GEMMs (attention; grid.y = batches): batch z splits into
    // zo = z / batch_inner, zi = z % batch_inner, and the operands start at
    // A + zo*a_so + zi*a_si, B + zo*b_so + (zi / b_group)*b_si,
    // C + zo*c_so + zi*c_si.  Zero-initialised arguments mean one batch.
    int32_t batch_inner, b_group;
    int64_t a_so, a_si, b_so, b_si, c_so, c_si;
    // Causal attention (rows are query positions): CAUSAL_SCORES skips tiles
    // whose keys (columns) all lie after every query row or, with window > 0,
    // all before it; CAUSAL_PV limits K (keys) to the causal window of the
    // tile's rows -- the probabilities outside it are zero.
    int32_t causal;
    int32_t window;
    // Stream-K grouped launch (sk_grid > 0): sk_grid workgroups share the
    // tiles' K steps evenly; sk_part holds 2 * sk_grid partial tiles of
    // NB * BM * BN floats for the tiles their range boundaries cut.
    int32_t sk_grid;
    float* sk_part;
    // Dense, one batch, no K split: a residual [M, N] with C's leading dim,
    // added after the bias, C = (A B + bias) + resid (it may be C itself);
    // nullptr for none.
    const float* resid;
};

enum Causal : int { CAUSAL_NONE = 0, CAUSAL_SCORES = 1, CAUSAL_PV = 2 };

enum Epilogue : int { EPI_STORE = 0, EPI_BIAS = 1, EPI_SILU = 2, EPI_SWIGLU = 3 };

// Launchers implemented in the .hip files.
void launch_gemm(const GemmArgs& a, bool nn, bool grouped, int epi, bool vec,
                 hipStream_t s);
// Dense batched GEMM over grid.y (the batch fields of GemmArgs; M, N, K,
// lda/ldb/ldc, causal, window as for one batch; direct-load path only).
void launch_gemm_batched(const GemmArgs& a, bool nn, int batches, hipStream_t s);
// Attention pieces: RoPE in place on q [rows, q_heads*hd] and k [rows,
// kv_heads*hd] (row r at position r % seq_len, cos/sin from table[pos][hd/2][2]);
// the masked softmax of a [batches, S, S] score block in place (scores scaled
// by 1/sqrt(hd), keys ki <= qi and qi - ki < window visible, the rest set to 0).
void launch_rope(float* q, float* k, const float* table, int64_t rows, int64_t seq_len,
                 int64_t first_pos, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                 hipStream_t s);
// Attention of the last position of each sequence: q [batch, q_heads*hd]
// (one row per sequence) against k, v [batch*seq_len, kv_heads*hd];
// scores: batch*q_heads*seq_len floats of workspace.
void launch_attn_last(const float* q, const float* k, const float* v, float* out, float* scores,
                      int64_t batch, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                      int64_t head_dim, int64_t window, hipStream_t s);
// RoPE with row r at positions[r]; attention of nq query rows over explicit
// key lists key_rows[key_beg[i] .. key_end[i]) (max_len: the longest list;
// scores: workspace of (last key_end) * q_heads floats when a list exceeds LDS).
void launch_rope_rows(float* q, float* k, const float* table, int64_t table_positions,
                      const int32_t* positions, int64_t rows, int64_t q_heads, int64_t kv_heads,
                      int64_t head_dim, hipStream_t s);
void launch_attn_paths(const float* q, const float* k, const float* v, float* out,
                       float* scores, const int32_t* key_rows, const int32_t* key_beg,
                       const int32_t* key_end, int64_t nq, int64_t kv_rows, int64_t max_len,
                       int64_t key_total, int64_t scores_floats, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, int64_t window, hipStream_t s);
// Causal attention in one pass, scores on chip (head_dim 64 or 128; false:
// another head_dim, nothing launched).  16-byte aligned q, k, v, out.
bool launch_flash_attention(const float* q, const float* k, const float* v, float* out,
                            int64_t batch, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                            int64_t head_dim, int64_t window, hipStream_t s);
void launch_attn_softmax(float* scores, int64_t batches, int64_t seq_len, int64_t head_dim,
                         int64_t window, hipStream_t s);
// a[i] += b[i];  a[r, c] += bias[c];  out[i, :] = table[tokens[i], :]
void launch_add(float* a, const float* b, int64_t n, hipStream_t s);
void launch_add_bias(float* a, const float* bias, int64_t rows, int64_t cols, hipStream_t s);
void launch_embed(const float* table, const int32_t* tokens, int64_t n, int64_t d,
                  int64_t vocab, float* out, hipStream_t s);
// zero / nzero: words the launch also sets to 0 (the routing counters of
// the launch that follows), or null / 0.
void launch_gate_logits(const float* x, const float* w, float* logits,
                        int64_t T, int64_t d, int64_t E, int contract,
                        hipStream_t s, uint32_t* zero = nullptr, int64_t nzero = 0);
void launch_route(const float* logits, const float* bias, int64_t T, int64_t E,
                  int64_t k, int mode, float quantum, float tie_eps,
                  int32_t* idx, float* w, hipStream_t s);
// The layer's routing and permutation in two launches.  route_count: the
// routing and the per-block expert counts, added into counts[E *
// ceil(T / kPermTokens)], which must be 0 when it starts (the gate's zero
// region).  perm_place_scan: perm and inv from those raw counts (each block
// scans them itself) and the expert offsets; for E * blocks up to
// kPlaceScanMax (past it: perm_scan, then perm_place).
constexpr int64_t kPlaceScanMax = 16384;
void launch_route_count(const float* logits, const float* bias, int64_t T, int64_t E,
                        int64_t k, int mode, float quantum, float tie_eps, int32_t* idx,
                        float* w, int32_t* counts, hipStream_t s);
void launch_perm_place_scan(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                            const int32_t* counts, int32_t* perm, int32_t* inv,
                            int32_t* offsets, hipStream_t s);
// A layer of one permutation block (T <= kPermTokens): the two launches
// above as one (routing, offsets, perm and inv; no counts), where
// route_place_one_fits says so.
bool route_place_one_fits(int64_t T, int64_t E, int64_t k, int mode);
void launch_route_place_one(const float* logits, const float* bias, int64_t T, int64_t E,
                            int64_t k, int mode, float quantum, float tie_eps, int32_t* idx,
                            float* w, int32_t* perm, int32_t* inv, int32_t* offsets,
                            hipStream_t s);
void launch_perm_count(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                       int32_t* counts, hipStream_t s);
void launch_perm_scan(int32_t* counts, int64_t nblocks, int64_t E,
                      int32_t* offsets, hipStream_t s);
void launch_perm_place(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                       const int32_t* base, int32_t* perm, int32_t* inv,
                       hipStream_t s);
void launch_empty(hipStream_t s);
void launch_silu(const float* x, float* y, int64_t n, hipStream_t s);
void launch_mul(const float* a, const float* b, float* c, int64_t n, hipStream_t s);
// c[rows, cols] (contiguous) = sum over `splits` partials part_stride apart,
// in order, + bias[cols] (nullable), + resid[rows, cols] (nullable; may be c).
void launch_split_sum(const float* parts, int splits, int64_t part_stride, const float* bias,
                      const float* resid, float* c, int64_t rows, int64_t cols, hipStream_t s);
// Layer norm (rms: RMS norm, no mean, no bias) over rows of h: per-row mean
// and 1/sqrt(var + eps) from the CPU loop's sequential chains, and
// (y != nullptr) the normalised rows.  row_inv (and row_mean for the layer
// norm) must be valid [rows] buffers; cus sizes the grid.
void launch_layer_norm(const float* x, const float* w, const float* b, int64_t rows, int64_t h,
                       float eps, int contract, bool rms, float* row_mean, float* row_inv,
                       float* y, int cus, hipStream_t s);

// out_rows holds `parts` partial row buffers of rows_total x d, part_stride
// elements apart; a row's value is their sum in part order.
void launch_combine(const float* out_rows, const int32_t* idx, const float* w,
                    const int32_t* inv, const float* resid, float* y,
                    int64_t T, int64_t k, int64_t d, int64_t rows_total,
                    int contract, int parts, int64_t part_stride, hipStream_t s);

}  // namespace moe

// The context: the device it is bound to, a grow-only workspace (so frees
// never land inside a timed region), and the optional per-kernel timers.
struct moe_ctx {
    int device = 0;
    int cus = 0;               // compute units of the device
    int w2_blocks_per_cu = 0;  // occupancy of the grouped w2 kernel (lazily queried)
    int w2n_blocks_per_cu = 0;  // ... of its 128x128-tile variant
    int w13_blocks_per_cu[2] = {};  // ... of the w1/w3 kernel, per tile (GemmArgs::tile)
    int sk_blocks_per_cu[5] = {};   // ... of the stream-K kernels, per GemmUse
    int sk_mode = -1;  // moe_ctx_set_stream_k: -1 planner (or MOE_SK), 0 off, 1 on
    int dense_blocks_per_cu[2][moe::kDenseTiles] = {};  // [nn][tile], lazily queried
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* scratch = nullptr;   // this device's no-alloc scratch (moe_layer_forward_noalloc)
    bool timing = false;
    struct Pending {
        const char* name;
        hipEvent_t start, stop;
    };
    std::vector<Pending> pending;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> event_pool;
    std::map<std::string, std::pair<double, int64_t>> totals;
    std::vector<std::string> name_store;  // keeps returned names alive

    void* workspace(size_t bytes);

    template <class F>
    void launch(const char* name, hipStream_t s, F&& f) {
        if (!timing) {
            f();
            moe::hip_check(hipGetLastError(), name);
            return;
        }
        std::pair<hipEvent_t, hipEvent_t> ev;
        if (!event_pool.empty()) {
            ev = event_pool.back();
            event_pool.pop_back();
        } else {
            moe::hip_check(hipEventCreate(&ev.first), "hipEventCreate");
            moe::hip_check(hipEventCreate(&ev.second), "hipEventCreate");
        }
        moe::hip_check(hipEventRecord(ev.first, s), "hipEventRecord");
        f();
        moe::hip_check(hipGetLastError(), name);
        moe::hip_check(hipEventRecord(ev.second, s), "hipEventRecord");
        pending.push_back({name, ev.first, ev.second});
    }
    void collect();
};
