// fp32 GEMM engine for gfx950 on the matrix cores (v_mfma_f32_32x32x2_f32).
//
// One kernel template serves every contraction of the MoE path:
//   dense NT  C = A B^T (+bias)       tensor_ops::matmul_transposed / Linear
//   dense NN  C = A B (+bias)         tensor_ops::matmul (declared only in the
//                                     reference, include/tensor.h:61)
//   grouped   per-expert tiles over ragged packed rows, A rows gathered
//             through the permutation, one launch for all experts:
//             w1/w3 with the SwiGLU (or SiLU) epilogue, then w2.
//
// A workgroup of WM x WN wave64s computes a BM x BN output tile (per B
// operand); each wave holds its (BM/WM) x (BN/WN) quadrant as 32x32 MFMA
// blocks in accumulator registers.  K advances BK at a time through
// double-buffered LDS tiles ([rows][BK+4] floats: the 4-float pad makes the
// 16-byte fragment reads conflict-free), with the next tile's global loads
// in flight in registers while the matrix cores work on the current one:
// one barrier per K step.
//
// Within each 16-column slice of a K step, lane half h (lanes 32h..32h+31)
// feeds columns 8h..8h+7, so one 16-byte LDS read gives a lane its A (or B)
// operand for 4 MFMAs; both operands use the same column order, so every
// product pairs the same k.  Products are accumulated in fp32 by the MFMA
// unit; the order differs from the reference's single sequential
// accumulator, within the 1e-4 relative-error budget of the activations.
//
// The dual-B variant keeps two accumulator sets (w1 and w3 tiles of the
// same d_ff columns) so the SwiGLU epilogue silu(g) * u happens in registers
// and w1/w3 need no interleaved copy (the reference interleaves rows at
// load, src/model.cu:1340-1365).
#include "common.hpp"

#include <cstdlib>
#include <type_traits>
#include <utility>

// Tile configurations (index into CFG_TABLE below) chosen per use; the
// defaults are the measured best on MI355X and can be overridden at build
// time for tuning (-DMOE_W13_CFG=n ...).
#ifndef MOE_W13_CFG
#define MOE_W13_CFG 0
#endif
#ifndef MOE_W2_CFG
#define MOE_W2_CFG 4
#endif
#ifndef MOE_DENSE_CFG
#define MOE_DENSE_CFG 0
#endif
// Main-loop schedule per use, a bit mask of SCHED_* (below).  Defaults are
// the measured best on MI355X: direct loads issued as buffer loads, fragment
// reads in burst order, the three-stage ring, for every use.  Raised wave
// priority around the MFMAs once helped w1/w3 by a little, but its
// instructions fence the scheduler, so a step's loads cannot spread among
// its MFMAs: without it, spread, w1/w3 run 2.5 % faster (configs 3-5, the
// reference's layer shape).  The 128 x 128 dense tile once kept two stages
// (four workgroups per CU against the ring's three); with the loads spread,
// the ring is 1 % faster on the large NT squares.
#ifndef MOE_W13_SCHED
#define MOE_W13_SCHED 62
#endif
#ifndef MOE_W2_SCHED
#define MOE_W2_SCHED 62
#endif
#ifndef MOE_DENSE_SCHED
#define MOE_DENSE_SCHED 62
#endif
// The 256 x 128 tile takes the three-stage ring, like the expert GEMMs
// whose per-wave work it shares.
#ifndef MOE_DENSE_TALL_SCHED
#define MOE_DENSE_TALL_SCHED 62
#endif
// The small dense tiles (64 x 128, 32 x 128) serve short and skinny
// products whose few workgroups per CU cannot hide HBM latency with two
// stages: they take the ring too, for a second step of loads in flight.
#ifndef MOE_DENSE_SMALL_SCHED
#define MOE_DENSE_SMALL_SCHED 62
#endif

namespace moe {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Schedule bits: SCHED_PRIO raises the wave's issue priority during its
// matrix-core burst; SCHED_MIDSTORE (register-staged path) stores the next
// tile to LDS halfway through the burst instead of after it; SCHED_DIRECT
// takes the direct global->LDS path where it applies.
// SCHED_QSPLIT (direct path) reads a K step's fragments in the order the
// burst consumes them -- lane-half k columns 0-3 of every operand first, then
// 4-7 -- and runs the burst operand by operand, so the first MFMAs wait only
// for the reads they use instead of all of them.
// SCHED_BUFLDS (direct path) issues the global->LDS loads as buffer loads
// (a resource per operand, fixed 32-bit lane offsets, the K step in the
// scalar offset); the compiler counts those on the vector-memory counter
// only, so the fragment reads of a K step get partial waits.
// SCHED_RING3 (direct path, with SCHED_BUFLDS) keeps three LDS stages, one
// __shared__ array each, and loads two K steps ahead: the wait before each
// barrier leaves the newest stage's loads in flight (SCHED_RING(n): n
// stages, n - 1 steps ahead).
constexpr int SCHED_PRIO = 1, SCHED_MIDSTORE = 2, SCHED_DIRECT = 4, SCHED_QSPLIT = 8,
              SCHED_BUFLDS = 16, SCHED_RING3 = 32;
// With SCHED_RING3, bits 8-11 may give the ring a depth other than three
// (4-8 stages, loads that many steps minus one ahead): SCHED_RING(n).
constexpr int SCHED_RING(int n) { return SCHED_RING3 | (n << 8); }
constexpr int ring_stages(int sched) {
    return (sched & SCHED_RING3) == 0 ? 0 : (((sched >> 8) & 15) != 0 ? (sched >> 8) & 15 : 3);
}

// KW_ > 1 (direct ring path, dense, no stream-K): KW groups of WM x WN
// waves share the tile and split its K steps evenly (group g takes the g-th
// run of K steps, each group with its own ring stages); at the end the other
// groups' accumulators are added, through LDS, to group 0's, which writes the
// tile.  A workgroup alone on its CU then still has KW waves per SIMD.
template <int BM_, int BN_, int BK_, int WM_, int WN_, int KW_ = 1>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, KW = KW_;
    static constexpr int THREADS = 64 * WM * WN * KW;
    static constexpr int FM = BM / WM / 32;   // 32x32 blocks per wave along m
    static constexpr int FN = BN / WN / 32;   // ... along n (per B operand)
    static constexpr int LDS = BK + 4;        // LDS row stride in floats
    static constexpr int KQ = BK / 4;         // 16-byte chunks per row and K step
    static constexpr int A_LD = BM * KQ / THREADS;  // A chunks per thread
    static constexpr int B_LD = BN * KQ / THREADS;  // B chunks per thread (per operand)
    static_assert(FM >= 1 && FN >= 1 && BM % (32 * WM) == 0 && BN % (32 * WN) == 0, "tile");
    static_assert(BK % 16 == 0, "K step is a multiple of 16");
    // the register-staged kernel deals whole 16-byte chunks to every thread
    static constexpr bool STAGED = KW == 1 && A_LD * THREADS == BM * KQ &&
                                   B_LD * THREADS == BN * KQ && A_LD >= 1 && B_LD >= 1;
};

template <int ID> struct CfgOf;
template <> struct CfgOf<0> { using T = Cfg<128, 128, 16, 2, 2>; };
template <> struct CfgOf<1> { using T = Cfg<128, 128, 32, 2, 2>; };
template <> struct CfgOf<2> { using T = Cfg<256, 128, 16, 4, 2>; };
template <> struct CfgOf<3> { using T = Cfg<128, 64, 16, 2, 2>; };
template <> struct CfgOf<4> { using T = Cfg<128, 256, 16, 2, 2>; };
template <> struct CfgOf<5> { using T = Cfg<256, 128, 32, 4, 2>; };
template <> struct CfgOf<6> { using T = Cfg<256, 256, 16, 4, 2>; };
template <> struct CfgOf<7> { using T = Cfg<64, 128, 16, 1, 2>; };
template <> struct CfgOf<8> { using T = Cfg<64, 128, 16, 2, 2>; };  // direct only
template <> struct CfgOf<9> { using T = Cfg<32, 128, 16, 1, 4>; };  // direct only
// w1/w3 on 256 rows x 64 columns per operand: the same per-wave work as the
// 128 x 128 dual tile (64 rows x 64 columns of each operand), for d_ff that
// is a multiple of 64 but not of 128 (448: exactly 7 n-tiles instead of 4,
// the last of them half empty)
template <> struct CfgOf<10> { using T = Cfg<256, 64, 16, 4, 1>; };
// Dense 256 rows x 128 columns, each wave 64 rows x all 128 columns (2 x 4
// blocks of 32 x 32: the most MFMA work per fragment read of the dense
// tiles); NN reads its B fragments column-strided (below).
template <> struct CfgOf<11> { using T = Cfg<256, 128, 16, 4, 1>; };
// Dense 32 x 128 with four K groups: 8 waves, each 32 rows x 64 columns (two
// column blocks, so NN reads its B pairs 8 bytes at a time) over a quarter of
// K -- for products whose 32 x 128 tiles give each CU one workgroup.
// Measured on MI355X at 1024^3 (same box, NN / NT, the clock spun up first):
// 26.3-26.4 / 25.0-25.1 us against 32.0 / 31.2-31.7 for the best tile and
// split plan; at 1024 x 1024 x 512 17.7 / 16.9 against 23.0 / 22.3, at K =
// 2048 43.3 / 41.4 against 47.3 / 46.8.  Timed without the spin-up (this
// layout 29.8-30.2 / 27.7-27.9 us at 1024^3), the other layouts of 32 x 128
// were slower: two groups of four 32 x 32 waves 32.2 /
// 29.2-29.6, two groups of two 32 x 64 waves 29.9-30.7 / 27.4-27.7, four
// groups of one 32 x 128 wave 30.6-31.0 / 29.2-30.4, four groups of four
// 32 x 32 waves slower on every larger shape; two groups on the 64 x 128
// tile no faster than that tile's plans.
#ifndef MOE_DENSE_KW
#define MOE_DENSE_KW 4
#endif
#ifndef MOE_DENSE_KW_WN
#define MOE_DENSE_KW_WN 2
#endif
template <> struct CfgOf<12> { using T = Cfg<32, 128, 16, 1, MOE_DENSE_KW_WN, MOE_DENSE_KW>; };

// Workgroup ids are dealt round-robin over the XCDs.  Renumber them so each
// XCD works through a contiguous run of logical tiles: tiles that share an
// operand panel then share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
    const int xcd = bid % kNumXcd, slot = bid / kNumXcd;
    const int per = nb / kNumXcd, rem = nb % kNumXcd;
    return xcd < rem ? xcd * (per + 1) + slot
                     : rem * (per + 1) + (xcd - rem) * per + slot;
}

// Logical tile order: groups of `group` consecutive m-tiles sweep the
// n-tiles together, `group` m-tiles per n-tile.  With group = 8 the ~64
// workgroups an XCD runs at once cover about 8 m-tiles x 8 n-tiles, so each
// A panel and each B panel in flight is shared by 8 of them; group = m_tiles
// is the m-fastest order (every m-tile of one n-tile, then the next n-tile).
__device__ __forceinline__ void tile_of(int logical, int m_tiles, int n_tiles, int group,
                                        int& mt, int& nt) {
    const int per_group = group * n_tiles;
    const int g = logical / per_group, r = logical % per_group;
    const int rows = m_tiles - g * group < group ? m_tiles - g * group : group;
    nt = r / rows;
    mt = g * group + r % rows;
}

// Grouped GEMMs: the expert owning m-tile `mt` when each expert e is split
// into ceil(n_e / BM) tiles in expert order.  Every wave computes it with a
// wave-wide scan of the per-expert tile counts (64 experts per step), so no
// tile table is needed and each kernel may use its own BM.  Returns false
// for the surplus tiles of the worst-case grid.
template <int BM>
__device__ __forceinline__ bool find_expert(const int32_t* __restrict__ offsets, int E, int mt,
                                            int& expert, int& first_tile) {
    const int lane = threadIdx.x & 63;
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        int cnt = 0;
        if (e < E) {
            const int n = offsets[e + 1] - offsets[e];
            cnt = n > 0 ? (n + BM - 1) / BM : 0;
        }
        int incl = cnt;
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        const int start = carry + incl - cnt;
        const bool hit = cnt > 0 && mt >= start && mt < start + cnt;
        const unsigned long long m = __ballot(hit);
        if (m != 0ull) {
            const int l = __ffsll(static_cast<long long>(m)) - 1;
            expert = e0 + l;
            first_tile = __builtin_amdgcn_readfirstlane(__shfl(start, l, 64));
            return true;
        }
        carry += __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));
    }
    return false;
}

// Real m-tiles of a grouped launch: the sum over experts of ceil(n_e / BM),
// read from the offsets with a wave-wide sum (every lane gets the total).
template <int BM>
__device__ __forceinline__ int grouped_real_m_tiles(const int32_t* __restrict__ offsets, int E) {
    const int lane = threadIdx.x & 63;
    int cnt = 0;
    for (int e = lane; e < E; e += 64) {
        const int n = offsets[e + 1] - offsets[e];
        cnt += n > 0 ? (n + BM - 1) / BM : 0;
    }
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    // every lane holds the total; reading it from the first lane tells the
    // compiler so, and the tile indices derived from it stay scalar
    return __builtin_amdgcn_readfirstlane(cnt);
}

// The tile of this workgroup: (mt, nt) and its K split.  A grouped launch
// sizes its grid for the worst case (ceil(pairs / BM) + E m-tiles, every
// expert's last tile partial); here the real tiles are counted, workgroups
// past them exit at once, and only the real tiles are dealt to the XCDs --
// so each XCD gets an even share of real work whatever the raster group
// (the surplus ids are spread over the XCDs by the round-robin dispatch).
template <int BM, bool GROUPED>
__device__ __forceinline__ bool launch_tile(const GemmArgs& p, int& mt, int& nt, int& split) {
    int m_tiles = p.m_tiles;
    if (GROUPED) {
        const int real = grouped_real_m_tiles<BM>(p.offsets, p.E);
        m_tiles = real < m_tiles ? real : m_tiles;
    }
    const int tiles_mn = m_tiles * p.n_tiles;
    const int total = GROUPED ? tiles_mn * p.k_splits : static_cast<int>(gridDim.x);
    if (static_cast<int>(blockIdx.x) >= total) return false;
    const int logical = xcd_remap(blockIdx.x, total);
    split = logical / tiles_mn;
    tile_of(logical % tiles_mn, m_tiles, p.n_tiles, p.group_m < m_tiles ? p.group_m : m_tiles, mt,
            nt);
    return true;
}

// SiLU of the w1/w3 epilogue: x / (1 + exp(-x)) (src/tensor.cu:132-134,
// 169-173).  The reference rounds float(exp(double(-x))); with
// MOE_EPI_FAST_EXP the epilogue takes the single-precision hardware exp2 of
// -x * log2(e) instead (relative error about |x| * 6e-8 + 1 ulp; the GEMM
// sum before it already differs from the reference's loop by rounding).
#ifndef MOE_EPI_FAST_EXP
#define MOE_EPI_FAST_EXP 1
#endif
__device__ __forceinline__ float silu_ref(float g) {
#if MOE_EPI_FAST_EXP
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896340736f);
#else
    const float e = static_cast<float>(exp(-static_cast<double>(g)));
#endif
    return g / (1.0f + e);
}

// The store of one output element (row `row` of the launch, column n) under
// epilogue EPI; v0, v1: the accumulators of the first and the second B
// operand.
template <int EPI>
__device__ __forceinline__ void epi_store(const GemmArgs& p, float* Cb, int split, int64_t row,
                                          int64_t n, float v0, float v1) {
    float v = v0;
    if (EPI == EPI_BIAS) {
        if (p.bias != nullptr) v = v + p.bias[n];
        if (p.resid != nullptr) v = v + p.resid[row * p.ldc + n];
    } else if (EPI == EPI_SILU) {
        v = silu_ref(v);
    } else if (EPI == EPI_SWIGLU) {
        v = silu_ref(v) * v1;
    }
    Cb[split * p.c_split_stride + row * p.ldc + n] = v;
}

template <bool VEC>
__device__ __forceinline__ f32x4 load_k4(const float* row, int64_t k, int64_t K) {
    if (VEC) {
        // K % 4 == 0 and 16-byte aligned rows: the 4 columns are all in or out.
        if (k < K) return *reinterpret_cast<const f32x4*>(row + k);
        return f32x4{0.f, 0.f, 0.f, 0.f};
    }
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (k + j < K) ? row[k + j] : 0.0f;
    return v;
}

template <class C, int SCHED, bool NN, bool VEC, bool GROUPED, int NB, int EPI>
__global__ __launch_bounds__(C::THREADS, 2) void gemm_kernel(const GemmArgs p) {
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, LDS = C::LDS, KQ = C::KQ;
    constexpr int FM = C::FM, FN = C::FN;
    static_assert(C::STAGED, "staging divides evenly");
    __shared__ __align__(16) float As[2][BM * LDS];
    __shared__ __align__(16) float Bs[2][NB][BN * LDS];

    const int tid = threadIdx.x;
    int mt, nt, split;  // split: K range of this tile (split-K)
    if (!launch_tile<BM, GROUPED>(p, mt, nt, split)) return;  // surplus workgroup

    // ---- which rows / which expert this workgroup owns
    int64_t row0;
    int rows;
    const float* B[NB];
    if (GROUPED) {
        int e, first;
        if (!find_expert<BM>(p.offsets, p.E, mt, e, first)) return;  // surplus tile
        int64_t e_end = p.offsets[e + 1];
        e_end = e_end < p.rows_limit ? e_end : p.rows_limit;
        row0 = p.offsets[e] + static_cast<int64_t>(mt - first) * BM;
        if (row0 < 0 || row0 >= e_end) return;  // only reachable with inconsistent offsets
        rows = static_cast<int>(e_end - row0 < BM ? e_end - row0 : BM);
        B[0] = p.B0 + e * p.b_expert_stride;
        if (NB == 2) B[NB - 1] = p.B1 + e * p.b_expert_stride;
    } else {
        row0 = static_cast<int64_t>(mt) * BM;
        rows = static_cast<int>(p.M - row0 < BM ? p.M - row0 : BM);
        B[0] = p.B0;
        if (NB == 2) B[NB - 1] = p.B1;
    }
    const int64_t n0 = static_cast<int64_t>(nt) * BN;
    const int64_t N = p.N;
    // K columns [kbeg, K) of this split; loads are bounded by K
    const int64_t kbeg = split * p.k_split_len;
    const int64_t K = p.K - kbeg < p.k_split_len ? p.K : kbeg + p.k_split_len;

    // ---- global -> register staging.  Chunk c = tid + THREADS*i of a tile:
    // A and NT B rows are c / KQ, the 4 columns (c % KQ) * 4; consecutive
    // threads read consecutive 16 bytes of a row.
    const float* arow[C::A_LD];
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
        const int c = tid + C::THREADS * i;
        int r = c / KQ;
        r = r < rows ? r : rows - 1;  // rows past the edge: any valid row, masked at the store
        int64_t src = row0 + r;
        if (GROUPED && p.gather != nullptr) {
            int64_t tok = p.gather[row0 + r];
            tok = tok < 0 ? 0 : (tok >= p.gather_rows ? p.gather_rows - 1 : tok);
            src = tok;
        }
        arow[i] = p.A + src * p.lda;
    }
    // B, NT ([N, K]): like A.  NN ([K, N]): chunk c is 4 consecutive k rows of
    // column c % BN, k quad c / BN, transposed into LDS.
    const float* bptr[NB][C::B_LD];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < C::B_LD; ++i) {
            const int c = tid + C::THREADS * i;
            int64_t n = NN ? n0 + c % BN : n0 + c / KQ;
            n = n < N ? n : N - 1;
            bptr[nb][i] = NN ? B[nb] + n : B[nb] + n * p.ldb;
        }

    f32x4 ra[C::A_LD], rb[NB][C::B_LD];
    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i)
            ra[i] = load_k4<VEC>(arow[i], k0 + ((tid + C::THREADS * i) % KQ) * 4, K);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < C::B_LD; ++i) {
                const int c = tid + C::THREADS * i;
                if (!NN) {
                    rb[nb][i] = load_k4<VEC>(bptr[nb][i], k0 + (c % KQ) * 4, K);
                } else {
                    const int64_t kb = k0 + (c / BN) * 4;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        rb[nb][i][j] = kb + j < K ? bptr[nb][i][(kb + j) * p.ldb] : 0.0f;
                }
            }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i) {
            const int c = tid + C::THREADS * i;
            *reinterpret_cast<f32x4*>(&As[buf][(c / KQ) * LDS + (c % KQ) * 4]) = ra[i];
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < C::B_LD; ++i) {
                const int c = tid + C::THREADS * i;
                const int at = NN ? (c % BN) * LDS + (c / BN) * 4 : (c / KQ) * LDS + (c % KQ) * 4;
                *reinterpret_cast<f32x4*>(&Bs[buf][nb][at]) = rb[nb][i];
            }
    };

    // ---- matrix-core main loop
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % C::WM, wn = wave / C::WM;
    const int lr = lane & 31, lh = lane >> 5;
    const int arow0 = wm * (BM / C::WM), bcol0 = wn * (BN / C::WN);

    f32x16 acc[NB][FM][FN];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int bi = 0; bi < FM; ++bi)
#pragma unroll
            for (int bj = 0; bj < FN; ++bj)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[nb][bi][bj][r] = 0.0f;

    // One K step on LDS buffer `buf`.  `mid` runs between the two halves of
    // the matrix-core burst (the schedule may place the next tile's LDS
    // stores there, SCHED_MIDSTORE); SCHED_PRIO raises the burst's priority.
    auto compute = [&](int buf, auto&& mid) {
        if (SCHED & SCHED_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int sl = 0; sl < BK / 16; ++sl) {  // 16-column slices of the K step
            f32x4 a[FM][2], b[NB][FN][2];
#pragma unroll
            for (int bi = 0; bi < FM; ++bi) {
                const float* src = &As[buf][(arow0 + bi * 32 + lr) * LDS + sl * 16 + 8 * lh];
                a[bi][0] = *reinterpret_cast<const f32x4*>(src);
                a[bi][1] = *reinterpret_cast<const f32x4*>(src + 4);
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int bj = 0; bj < FN; ++bj) {
                    const float* src =
                        &Bs[buf][nb][(bcol0 + bj * 32 + lr) * LDS + sl * 16 + 8 * lh];
                    b[nb][bj][0] = *reinterpret_cast<const f32x4*>(src);
                    b[nb][bj][1] = *reinterpret_cast<const f32x4*>(src + 4);
                }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if (sl == BK / 16 - 1 && q == 1) mid();
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                        for (int bi = 0; bi < FM; ++bi)
#pragma unroll
                            for (int bj = 0; bj < FN; ++bj)
                                acc[nb][bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                    a[bi][q][s], b[nb][bj][q][s], acc[nb][bi][bj], 0, 0, 0);
            }
        }
        if (SCHED & SCHED_PRIO) __builtin_amdgcn_s_setprio(0);
    };

    const int64_t nk = (K - kbeg + BK - 1) / BK;
    if (nk > 0) {
        gload(kbeg);
        lstore(0);
        __syncthreads();
        for (int64_t kt = 0; kt < nk; ++kt) {
            const int cur = static_cast<int>(kt & 1);
            const bool more = kt + 1 < nk;
            if (more) gload(kbeg + (kt + 1) * BK);
            if (SCHED & SCHED_MIDSTORE) {
                compute(cur, [&] {
                    if (more) lstore(cur ^ 1);
                });
            } else {
                compute(cur, [] {});
                if (more) lstore(cur ^ 1);
            }
            __syncthreads();
        }
    }

    // ---- epilogue.  32x32 accumulator layout: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32 of its block.
#pragma unroll
    for (int bi = 0; bi < FM; ++bi)
#pragma unroll
        for (int bj = 0; bj < FN; ++bj)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                const int64_t n = n0 + bcol0 + bj * 32 + lr;
                if (i < rows && n < N)
                    epi_store<EPI>(p, p.C, split, row0 + i, n, acc[0][bi][bj][r],
                                   acc[NB - 1][bi][bj][r]);
            }
}

// ---------------------------------------------------------------------------
// GEMM with direct global->LDS loads (gfx950 buffer_load_dwordx4 ... lds,
// or global_load_lds_dwordx4 where an operand's byte offsets pass 2^31).
//
// Lane L of a load instruction writes its 16 bytes at LDS base + 16*L, from
// any global address it chooses, so each lane fetches the chunk that belongs
// at its slot: A (and NT B) tiles are stored unpadded, 4 chunks of 16 bytes
// per row of the 16-wide K step, chunk c of row r at slot c ^ ((r >> 2) & 3).
// The swizzle keeps the 16-byte fragment reads conflict-free.  The data goes
// from L2 straight to LDS -- no staging registers, no LDS store
// instructions -- and lands while the matrix cores run: each K step reads
// all fragments of the current stage, issues the next stage's loads, runs
// the MFMA burst, then waits for its loads and meets the other waves at the
// barrier.  Requires K % 16 == 0 and 16-byte aligned rows.
//
// The buffer form (SCHED_BUFLDS) keeps each lane's source as a fixed 32-bit
// offset from a wave-uniform base and advances K through the scalar offset,
// so a K step spends no vector instructions on 64-bit addresses.  The
// compiler also counts the global form against the LDS counter (it is a
// FLAT instruction that writes LDS), which forces a wait for every fragment
// read before the first MFMA; the buffer form leaves that counter to the
// fragment reads, and the first MFMAs wait only for their own operands.
// Measured on MI355X: dense NT 8192^3 119 -> 138 TFLOP/s, config-3 w2
// 8.03 -> 7.72 ms, config-5 w2 0.51 -> 0.47 ms, w1/w3 unchanged.
//
// NN B ([K, N] row-major) stays k-major in LDS: one load instruction moves
// 256 consecutive floats of the tile, 256 / BN k-rows of BN columns, and
// instructions sit NN_PAD floats apart so that k-rows 8 apart (the two lane
// halves of a fragment read) fall on opposite halves of the 64 banks.  A
// lane then gathers its column's 8 k values with 4-byte reads.  Requires
// N % 4 == 0 as well.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void glb_void;

// Raw buffer resource over [p, p + 4 GiB): no stride, no range clamp.  `p`
// must be wave-uniform; it is read from the first lane so the resource
// lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const float* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v))));
    const uint64_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v >> 32))));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((hi << 32) | lo),
                                             static_cast<short>(0), -1, 0x00020000);
}

template <int... I, class F>
__device__ __forceinline__ void static_for_int(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}), ...);
}

// One 16-byte-per-lane buffer load into LDS at `dst` + 16 * lane, from
// `base` + `voff` (per lane) + `soff` (uniform) bytes.
__device__ __forceinline__ void buffer_load_lds16(const float* base, lds_void* dst, uint32_t voff,
                                                  uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(raw_rsrc(base), dst, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }

// The K-step barrier of the three-stage ring.  __syncthreads() carries a
// workgroup fence, and a fence must wait for every load that writes LDS --
// the stage two steps ahead included (the compiler emits vmcnt(0) before each
// barrier), which leaves only one step for those loads to land.  The ring
// orders its stages itself: before the barrier each wave has waited for its
// loads of the next stage (vmcnt(loads per stage)) and for its own LDS reads
// (lgkmcnt(0); the matrix cores have consumed them), so after it every wave's
// next stage has landed and no wave still reads the stage the following step
// overwrites.  The empty asm statements keep the compiler from moving memory
// operations across the barrier.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int BN>
struct NnB {
    static constexpr int RPI = 256 / BN;        // k-rows per load instruction
    static constexpr int PAD = 4 * RPI;         // floats between instructions' rows
    static constexpr int STRIDE = 256 + PAD;    // LDS floats per load instruction
    static_assert(BN <= 256 && 256 % BN == 0, "NN direct tiles: BN divides 256");
    // LDS index of element (k, n) of the 16 x BN tile
    static __device__ __forceinline__ int at(int k, int n) {
        return (k / RPI) * STRIDE + (k % RPI) * BN + n;
    }
};

// Grouped GEMMs: rows [row0, row0 + rows) of m-tile `mt` and its expert e.
// False for a surplus tile of the worst-case grid (or inconsistent offsets).
template <int BM>
__device__ __forceinline__ bool grouped_tile_rows(const GemmArgs& p, int mt, int& e,
                                                  int64_t& row0, int& rows) {
    int first;
    if (!find_expert<BM>(p.offsets, p.E, mt, e, first)) return false;
    int64_t e_end = p.offsets[e + 1];
    e_end = e_end < p.rows_limit ? e_end : p.rows_limit;
    row0 = p.offsets[e] + static_cast<int64_t>(mt - first) * BM;
    if (row0 < 0 || row0 >= e_end) return false;
    rows = static_cast<int>(e_end - row0 < BM ? e_end - row0 : BM);
    return true;
}

// The epilogue of one output tile: every accumulator of this lane that lies
// inside [rows, N) goes through epi_store.  32x32 accumulator layout: lane l,
// register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32 of its block.
// One 32x32 block (bi, bj) of this lane's accumulators, a0 and a1 its
// values for the first and the last B operand.
template <class C, int EPI>
__device__ __forceinline__ void store_block(const GemmArgs& p, float* Cb, int split, int64_t row0,
                                            int rows, int64_t n0, int bi, int bj, const f32x16& a0,
                                            const f32x16& a1, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % C::WM, wn = wave / C::WM;
    const int lr = lane & 31, lh = lane >> 5;
    const int arow0 = wm * (C::BM / C::WM), bcol0 = wn * (C::BN / C::WN);
    if constexpr (EPI == EPI_BIAS) {
        // the lane's column is the same for all 16 values: its bias is
        // loaded once (C may alias it as far as the compiler knows, so a
        // load per store would wait behind each store)
        const int64_t n = n0 + bcol0 + bj * 32 + lr;
        if (n >= p.N) return;
        const bool hb = p.bias != nullptr;
        const float bn = hb ? p.bias[n] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (i >= rows) continue;
            float v = a0[r];
            if (hb) v = v + bn;
            if (p.resid != nullptr) v = v + p.resid[(row0 + i) * p.ldc + n];
            Cb[split * p.c_split_stride + (row0 + i) * p.ldc + n] = v;
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        const int64_t n = n0 + bcol0 + bj * 32 + lr;
        if (i < rows && n < p.N) epi_store<EPI>(p, Cb, split, row0 + i, n, a0[r], a1[r]);
    }
}

template <class C, int NB, int EPI>
__device__ __forceinline__ void store_tile(const GemmArgs& p, float* Cb, int split, int64_t row0,
                                           int rows, int64_t n0,
                                           const f32x16 (&acc)[NB][C::FM][C::FN], int tid) {
    if constexpr (EPI == EPI_BIAS) {
        if (p.resid != nullptr) {
            // A row of blocks at a time, all of its residual values loaded
            // before any of its stores: resid may alias C, so the compiler
            // would otherwise wait for each load before the next store.
            const int lane = tid & 63, wave = tid >> 6;
            const int wm = wave % C::WM, wn = wave / C::WM;
            const int lr = lane & 31, lh = lane >> 5;
            const int arow0 = wm * (C::BM / C::WM), bcol0 = wn * (C::BN / C::WN);
            const bool hb = p.bias != nullptr;
            float bn[C::FN];
#pragma unroll
            for (int bj = 0; bj < C::FN; ++bj) {
                const int64_t n = n0 + bcol0 + bj * 32 + lr;
                bn[bj] = hb && n < p.N ? p.bias[n] : 0.0f;
            }
#pragma unroll
            for (int bi = 0; bi < C::FM; ++bi) {
                float rv[C::FN][16];
#pragma unroll
                for (int bj = 0; bj < C::FN; ++bj)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                        const int64_t n = n0 + bcol0 + bj * 32 + lr;
                        rv[bj][r] = i < rows && n < p.N ? p.resid[(row0 + i) * p.ldc + n] : 0.0f;
                    }
#pragma unroll
                for (int bj = 0; bj < C::FN; ++bj)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                        const int64_t n = n0 + bcol0 + bj * 32 + lr;
                        if (i < rows && n < p.N) {
                            float v = acc[0][bi][bj][r];
                            if (hb) v = v + bn[bj];
                            Cb[split * p.c_split_stride + (row0 + i) * p.ldc + n] = v + rv[bj][r];
                        }
                    }
            }
            return;
        }
    }
#pragma unroll
    for (int bi = 0; bi < C::FM; ++bi)
#pragma unroll
        for (int bj = 0; bj < C::FN; ++bj)
            store_block<C, EPI>(p, Cb, split, row0, rows, n0, bi, bj, acc[0][bi][bj],
                                acc[NB - 1][bi][bj], tid);
}

// Stream-K partial tiles: the accumulators of one K segment of a tile, stored
// lane by lane (16 bytes per lane and instruction, coalesced) in slot `part`
// of NB * BM * BN floats; the fix-up kernel reads them back in the same
// order with the same lanes.
template <class C, int NB>
__device__ __forceinline__ int sk_part_index(int nb, int bi, int bj, int r4, int tid) {
    return (((nb * C::FM + bi) * C::FN + bj) * 4 + r4) * C::THREADS + tid;
}

// One output tile (mt, nt) of the direct-load GEMM, over K split `split`
// or, with seg_lo >= 0, over K steps [seg_lo, seg_hi) of it (a stream-K
// segment).  part == nullptr: the epilogue writes the tile; otherwise the
// raw accumulators go to the partial slot `part`.  LOOPED: called once per
// segment in a loop; the lane index is then hidden from the optimiser, so
// the per-lane LDS and store addresses are recomputed in each segment
// instead of being hoisted out of the loop and held in registers across it
// (they cost 60-90 more VGPRs, past the budget of two workgroups per CU).
template <class C, int SCHED, bool NN, bool GROUPED, int NB, int EPI, bool LOOPED = false>
__device__ __forceinline__ void direct_tile(const GemmArgs& p, int mt, int nt, int split,
                                            int64_t seg_lo, int64_t seg_hi, float* part) {
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK;
    constexpr int FM = C::FM, FN = C::FN;
    constexpr int KW = C::KW;
    constexpr int NW = C::THREADS / 64 / KW;  // waves per K group
    // 1 KiB load instructions per tile (16 rows x 16 k, or 256 floats of an
    // NN B tile), dealt to the waves: INS per wave, the last ones idle when
    // the tile has fewer instructions than waves.
    constexpr int A_TOT = BM / 16, B_TOT = BN / 16;
    constexpr int A_INS = (A_TOT + NW - 1) / NW;
    constexpr int B_INS = (B_TOT + NW - 1) / NW;
    static_assert(BK == 16, "direct path: 16-wide K steps");
    static_assert(A_TOT * 16 == BM && B_TOT * 16 == BN, "load split");
    static_assert(A_INS * NW == A_TOT || A_TOT < NW, "A load split");
    static_assert(B_INS * NW == B_TOT || B_TOT < NW, "B load split");
    constexpr int B_SIZE = NN ? B_TOT * NnB<BN>::STRIDE : BN * BK;
    // NN with 4 (or 2) column blocks per wave: block bj holds the columns
    // FN c + bj (c = lane % 32), so one 16-byte (8-byte) LDS read of a k-row
    // gives a lane its B value for all FN blocks (NN B sits k-major in LDS;
    // with 32-column blocks each value would be a separate 4-byte read), and
    // the epilogue writes FN adjacent columns per lane.
#ifndef MOE_NN_STRIDE2
#define MOE_NN_STRIDE2 1
#endif
    constexpr bool NSTRIDE = NN && (FN == 4 || (FN == 2 && MOE_NN_STRIDE2));
    __shared__ __align__(16) float As[2][BM * BK];
    __shared__ __align__(16) float Bs[2][NB][B_SIZE];

    int tid = threadIdx.x;
    if constexpr (LOOPED) asm volatile("" : "+v"(tid));
    // wave: this wave's index in its K group wk (the load dealing, the
    // quadrant and the epilogue are per group)
    const int lane = tid & 63, wk = (tid >> 6) / NW, wave = (tid >> 6) % NW;
    static_assert(KW == 1 || (!GROUPED && !LOOPED), "K groups: dense, one tile per workgroup");

    int64_t row0;
    int rows;
    const float* B[NB];
    const float* Ab = p.A;
    float* Cb = p.C;
    if (GROUPED) {
        int e;
        // surplus tile, or (only with inconsistent offsets) no rows
        if (!grouped_tile_rows<BM>(p, mt, e, row0, rows)) return;
        B[0] = p.B0 + e * p.b_expert_stride;
        if (NB == 2) B[NB - 1] = p.B1 + e * p.b_expert_stride;
    } else {
        row0 = static_cast<int64_t>(mt) * BM;
        rows = static_cast<int>(p.M - row0 < BM ? p.M - row0 : BM);
        // batch of a batched launch (grid.y); one batch otherwise
        const int64_t z = blockIdx.y;
        const int64_t inner = p.batch_inner > 0 ? p.batch_inner : 1;
        const int64_t zo = z / inner, zi = z % inner;
        const int64_t bz = zi / (p.b_group > 0 ? p.b_group : 1);
        Ab = p.A + zo * p.a_so + zi * p.a_si;
        Cb = p.C + zo * p.c_so + zi * p.c_si;
        B[0] = p.B0 + zo * p.b_so + bz * p.b_si;
        if (NB == 2) B[NB - 1] = p.B1 + zo * p.b_so + bz * p.b_si;
    }
    const int64_t n0 = static_cast<int64_t>(nt) * BN;
    const int64_t N = p.N;
    // K columns [kbeg, K) of this split; loads are bounded by K
    int64_t kbeg = split * p.k_split_len;
    int64_t K = p.K - kbeg < p.k_split_len ? p.K : kbeg + p.k_split_len;
    if (seg_lo >= 0) {
        // a stream-K segment: K steps [seg_lo, seg_hi) of the split
        K = kbeg + seg_hi * BK;
        kbeg += seg_lo * BK;
    }
    if (!GROUPED && p.causal == CAUSAL_SCORES) {
        // keys n0.. all after the last query row, or (window) all too old for
        // the first: nothing of this tile is ever read
        if (n0 > row0 + rows - 1) return;
        if (p.window > 0 && n0 + BN - 1 < row0 - (p.window - 1)) return;
    } else if (!GROUPED && p.causal == CAUSAL_PV) {
        // probabilities of keys past the last row (or before the first row's
        // window) are zero: leave them out of the K loop (multiples of 16)
        const int64_t hi = ((row0 + rows + 15) / 16) * 16;
        K = K < hi ? K : hi;
        if (p.window > 0) {
            int64_t lo = row0 - (p.window - 1);
            lo = lo > 0 ? (lo / 16) * 16 : 0;
            kbeg = kbeg > lo ? kbeg : lo;
        }
    }
    if constexpr (KW > 1) {
        // group wk: the wk-th of KW equal runs of the K steps (the host keeps
        // the step count a multiple of KW, so every group meets the same
        // barriers)
        const int64_t per = (K - kbeg) / BK / KW;
        kbeg += wk * per * BK;
        K = kbeg + per * BK;
    }

    // Per-lane source of each load instruction: instruction j of this wave
    // fills rows 16*J .. 16*J+15 (J = wave*INS + j); lane L writes slot L%4
    // of row 16*J + L/4, i.e. global chunk (L%4) ^ swz(row).
    const int lrow = lane >> 2, lslot = lane & 3;
    const float* asrc[A_INS];
#pragma unroll
    for (int j = 0; j < A_INS; ++j) {
        int r = 16 * (wave * A_INS + j) + lrow;
        r = r < BM ? r : BM - 1;  // an idle wave's instruction (never issued)
        const int rr = r < rows ? r : rows - 1;  // past the edge: a valid row, masked at the store
        int64_t src = row0 + rr;
        if (GROUPED && p.gather != nullptr) {
            int64_t tok = p.gather[row0 + rr];
            tok = tok < 0 ? 0 : (tok >= p.gather_rows ? p.gather_rows - 1 : tok);
            src = tok;
        }
        asrc[j] = Ab + src * p.lda + 4 * (lslot ^ swz(r));
    }
    // B: NT rows n like A's rows.  NN: instruction J's lane L holds floats
    // 256 J + 4 L .. +3 of the k-major tile, i.e. k-row (256 J + 4 L) / BN,
    // columns n0 + (256 J + 4 L) % BN (past N: the last 4 columns, masked at
    // the store); its source advances by k0 rows.
    const float* bsrc[NB][B_INS];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < B_INS; ++j) {
            int J = wave * B_INS + j;
            J = J < B_TOT ? J : B_TOT - 1;
            if (NN) {
                const int flat = 256 * J + 4 * lane;
                int64_t n = n0 + flat % BN;
                n = n < N ? n : N - 4;
                bsrc[nb][j] = B[nb] + static_cast<int64_t>(flat / BN) * p.ldb + n;
            } else {
                const int r = 16 * J + lrow;
                int64_t n = n0 + r;
                n = n < N ? n : N - 1;
                bsrc[nb][j] = B[nb] + n * p.ldb + 4 * (lslot ^ swz(r));
            }
        }
    // SCHED_BUFLDS: byte offsets of the same sources from wave-uniform bases
    // (A: the matrix when rows are gathered, else the tile's first row; B:
    // the tile's first row (NT) or column (NN)).  The host takes this path
    // only when every offset stays below 2^31.
    const float* abase = (GROUPED && p.gather != nullptr) ? Ab : Ab + row0 * p.lda;
    const float* bbase[NB];
    uint32_t aoff[A_INS], boff32[NB][B_INS];
    if (SCHED & SCHED_BUFLDS) {
#pragma unroll
        for (int j = 0; j < A_INS; ++j) aoff[j] = static_cast<uint32_t>((asrc[j] - abase) * 4);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            bbase[nb] = NN ? B[nb] + n0 : B[nb] + n0 * p.ldb;
#pragma unroll
            for (int j = 0; j < B_INS; ++j)
                boff32[nb][j] = static_cast<uint32_t>((bsrc[nb][j] - bbase[nb]) * 4);
        }
    }
    // loads of the K step at k0 into the stage at (adst, bdst): A tile, then
    // the NB B tiles B_SIZE floats apart
    auto issue_to = [&](float* adst, float* bdst, int64_t k0) {
        const int64_t boff = NN ? k0 * p.ldb : k0;
        constexpr int BSTEP = NN ? NnB<BN>::STRIDE : 256;
        if (SCHED & SCHED_BUFLDS) {
            // wave-uniform byte offsets of the K step (scalar operands of
            // the loads; read from the first lane so that the compiler never
            // treats them as per-lane values)
            const uint32_t ak = static_cast<uint32_t>(
                __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(k0 * 4))));
            const uint32_t bk = static_cast<uint32_t>(
                __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(boff * 4))));
#pragma unroll
            for (int j = 0; j < A_INS; ++j)
                if (A_INS * NW == A_TOT || wave * A_INS + j < A_TOT)
                    buffer_load_lds16(abase, (lds_void*)&adst[(wave * A_INS + j) * 256], aoff[j],
                                      ak);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int j = 0; j < B_INS; ++j)
                    if (B_INS * NW == B_TOT || wave * B_INS + j < B_TOT)
                        buffer_load_lds16(bbase[nb],
                                          (lds_void*)&bdst[nb * B_SIZE + (wave * B_INS + j) * BSTEP],
                                          boff32[nb][j], bk);
            return;
        }
#pragma unroll
        for (int j = 0; j < A_INS; ++j)
            if (A_INS * NW == A_TOT || wave * A_INS + j < A_TOT)
                __builtin_amdgcn_global_load_lds((glb_void*)(asrc[j] + k0),
                                                 (lds_void*)&adst[(wave * A_INS + j) * 256], 16, 0,
                                                 0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int j = 0; j < B_INS; ++j)
                if (B_INS * NW == B_TOT || wave * B_INS + j < B_TOT)
                    __builtin_amdgcn_global_load_lds(
                        (glb_void*)(bsrc[nb][j] + boff),
                        (lds_void*)&bdst[nb * B_SIZE + (wave * B_INS + j) * BSTEP], 16, 0, 0);
    };
    auto issue = [&](int buf, int64_t k0) { issue_to(As[buf], &Bs[buf][0][0], k0); };

    const int wm = wave % C::WM, wn = wave / C::WM;
    const int lr = lane & 31, lh = lane >> 5;
    const int arow0 = wm * (BM / C::WM), bcol0 = wn * (BN / C::WN);

    f32x16 acc[NB][FM][FN];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int bi = 0; bi < FM; ++bi)
#pragma unroll
            for (int bj = 0; bj < FN; ++bj)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[nb][bi][bj][r] = 0.0f;

    // 32-row blocks of this wave that hold at least one real row
    // A wave whose columns all lie past N (the last n-tile of an N that is
    // not a multiple of BN) has no real output either: it skips its bursts.
    const int live_rows = n0 + bcol0 < N ? rows - arow0 : 0;
    const int live = live_rows <= 0 ? 0 : (live_rows >= FM * 32 ? FM : (live_rows + 31) / 32);

    // K steps of this tile (wave-uniform; fits 31 bits: the host bounds K)
    const int64_t nk = __builtin_amdgcn_readfirstlane(static_cast<int>((K - kbeg) / BK));
    f32x4 a[FM][2], b[NB][FN][2];
    // the fragments of one K step that a burst over the first NBLK 32-row
    // blocks uses, from the stage at (Acur, Bcur) (no LDS read may follow the
    // next stage's loads: they would have to wait)
    auto read_frags = [&](auto nblk, const float* Acur, const float* Bcur) {
        constexpr int NBLK = decltype(nblk)::value < 0 ? FM : decltype(nblk)::value;
        if constexpr (NBLK == 0) return;
        auto read_a = [&](int q) {
#pragma unroll
            for (int bi = 0; bi < NBLK; ++bi) {
                const int r = arow0 + bi * 32 + lr;
                a[bi][q] = *reinterpret_cast<const f32x4*>(&Acur[r * BK] +
                                                           4 * ((2 * lh + q) ^ swz(r)));
            }
        };
        auto read_b = [&](int nb, int q) {
            if constexpr (NSTRIDE && FN == 4) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(
                        &Bcur[nb * B_SIZE + NnB<BN>::at(8 * lh + 4 * q + s, bcol0 + 4 * lr)]);
#pragma unroll
                    for (int bj = 0; bj < 4; ++bj) b[nb][bj][q][s] = v[bj];
                }
                return;
            } else if constexpr (NSTRIDE) {
                typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const f32x2 v = *reinterpret_cast<const f32x2*>(
                        &Bcur[nb * B_SIZE + NnB<BN>::at(8 * lh + 4 * q + s, bcol0 + 2 * lr)]);
#pragma unroll
                    for (int bj = 0; bj < 2; ++bj) b[nb][bj][q][s] = v[bj];
                }
                return;
            }
#pragma unroll
            for (int bj = 0; bj < FN; ++bj) {
                const int r = bcol0 + bj * 32 + lr;
                if (NN) {
                    // the same k order as A: slot s of half q is k = 8 lh + 4 q + s
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        b[nb][bj][q][s] = Bcur[nb * B_SIZE + NnB<BN>::at(8 * lh + 4 * q + s, r)];
                } else {
                    b[nb][bj][q] = *reinterpret_cast<const f32x4*>(&Bcur[nb * B_SIZE + r * BK] +
                                                                   4 * ((2 * lh + q) ^ swz(r)));
                }
            }
        };
        if (SCHED & SCHED_QSPLIT) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                read_a(q);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) read_b(nb, q);
            }
        } else {
            read_a(0);
            read_a(1);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                read_b(nb, 0);
                read_b(nb, 1);
            }
        }
    };
    // the MFMA burst of one K step over the first NBLK 32-row blocks of this
    // wave
    auto mfma_burst = [&](auto nblk) {
        constexpr int NBLK = decltype(nblk)::value;
        if constexpr (NBLK == 0) return;
        if (SCHED & SCHED_PRIO) __builtin_amdgcn_s_setprio(1);
        {
            auto step = [&](int q, int s, int nb) {
#pragma unroll
                for (int bi = 0; bi < NBLK; ++bi)
#pragma unroll
                    for (int bj = 0; bj < FN; ++bj)
                        acc[nb][bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            a[bi][q][s], b[nb][bj][q][s], acc[nb][bi][bj], 0, 0, 0);
            };
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if (SCHED & SCHED_QSPLIT) {
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                        for (int s = 0; s < 4; ++s) step(q, s, nb);
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) step(q, s, nb);
                }
            }
        }
        if (SCHED & SCHED_PRIO) __builtin_amdgcn_s_setprio(0);
    };
    // NBLK < 0: this wave's live blocks chosen in every K step (wave-uniform
    // branches)
    auto mfma_step = [&](auto nblk) {
        if constexpr (decltype(nblk)::value >= 0) {
            mfma_burst(nblk);
        } else {
            if (live == FM) mfma_burst(std::integral_constant<int, FM>{});
            else if (FM > 1 && live == 1) mfma_burst(std::integral_constant<int, 1>{});
            else if (live > 0) mfma_burst(std::integral_constant<int, FM>{});
        }
    };

    constexpr int LPS_MAX = A_INS + NB * B_INS;
    // every wave issues LPS_MAX loads per stage (the tile has at least as
    // many load instructions as waves, in whole multiples)
    constexpr bool LPS_ALL = A_INS * NW == A_TOT && B_INS * NW == B_TOT;
    // The ring's RS stage arrays (unused ones shrink to one float; kernels
    // without the ring reference none of them, so none is allocated)
    constexpr bool RING = (SCHED & SCHED_RING3) != 0;
    constexpr int RS = ring_stages(SCHED);
    static_assert(!RING || (RS >= 3 && RS <= 8), "ring stages");
    static_assert(!RING || (RS - 2) * LPS_MAX <= 63, "vmcnt range");
    // each stage array holds the KW groups' stages side by side
    constexpr int SA = BM * BK, SB = NB * B_SIZE, KSA = KW * SA, KSB = KW * SB;
    __shared__ __align__(16) float RA0[KSA], RA1[KSA], RA2[KSA], RA3[RS > 3 ? KSA : 1],
        RA4[RS > 4 ? KSA : 1], RA5[RS > 5 ? KSA : 1], RA6[RS > 6 ? KSA : 1], RA7[RS > 7 ? KSA : 1];
    __shared__ __align__(16) float RB0[KSB], RB1[KSB], RB2[KSB], RB3[RS > 3 ? KSB : 1],
        RB4[RS > 4 ? KSB : 1], RB5[RS > 5 ? KSB : 1], RB6[RS > 6 ? KSB : 1], RB7[RS > 7 ? KSB : 1];
    const int ga = KW > 1 ? wk * SA : 0, gb = KW > 1 ? wk * SB : 0;
    auto ra = [&](auto u) -> float* {
        constexpr int U = decltype(u)::value;
        if constexpr (U == 0) return RA0 + ga;
        else if constexpr (U == 1) return RA1 + ga;
        else if constexpr (U == 2) return RA2 + ga;
        else if constexpr (U == 3) return RA3 + ga;
        else if constexpr (U == 4) return RA4 + ga;
        else if constexpr (U == 5) return RA5 + ga;
        else if constexpr (U == 6) return RA6 + ga;
        else return RA7 + ga;
    };
    auto rb = [&](auto u) -> float* {
        constexpr int U = decltype(u)::value;
        if constexpr (U == 0) return RB0 + gb;
        else if constexpr (U == 1) return RB1 + gb;
        else if constexpr (U == 2) return RB2 + gb;
        else if constexpr (U == 3) return RB3 + gb;
        else if constexpr (U == 4) return RB4 + gb;
        else if constexpr (U == 5) return RB5 + gb;
        else if constexpr (U == 6) return RB6 + gb;
        else return RB7 + gb;
    };
    // The K loop for a burst over NBLK blocks (NBLK < 0: over the live ones,
    // chosen per step).  Blocks whose 32 rows all lie past the tile's last
    // real row (the ragged end of an expert) are skipped.  The ring kernels
    // instantiate the loop per burst width and each wave picks one per tile:
    // the wave-uniform branch in every K step cost 2-3 % of the MFMA time
    // (measured on MI355X at configs 3-5; the reference's layer shape, whose
    // w2 tiles are 28 K steps long, gains 1 % per layer); the two-stage
    // kernels measured 1-3 % slower so and keep one loop.
    // The order of one ring step (scheduling groups, in turn): its fragment
    // reads, then its MFMAs with its loads spread among them, one after every
    // PER MFMAs.  Issued in a burst ahead of the MFMAs, the loads (each a
    // scalar LDS address move and a buffer load) held back the step's first
    // MFMA; spread, they issue while the matrix cores run (measured on
    // MI355X: 2-6 % less time per GEMM at configs 3-5 and the reference's
    // layer shape).
    auto schedule_step = [&](auto nblk) {
        constexpr int NBLK = decltype(nblk)::value;
        if constexpr (LPS_ALL && NBLK > 0) {
            constexpr int MF = NBLK * FN * NB * 8;
            constexpr int DSR =
                NBLK * 2 + (NSTRIDE ? NB * 8 : (NN ? NB * FN * 8 : NB * FN * 2));
            constexpr int PER = MF / (LPS_MAX + 2);
            __builtin_amdgcn_sched_group_barrier(0x100, DSR, 0);  // LDS reads
            static_for_int(std::make_integer_sequence<int, LPS_MAX>{}, [&](auto) {
                __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);  // MFMAs
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // a load
            });
            __builtin_amdgcn_sched_group_barrier(0x008, MF - PER * LPS_MAX, 0);
        }
    };
    auto k_loop = [&](auto nblk) {
        if constexpr (RING) {
            // RS stages (three by default), one __shared__ array each (the
            // compiler then waits only for the loads landing in the stage it
            // reads), the K loop unrolled by RS so every step names its arrays.
            static_assert((SCHED & SCHED_BUFLDS) != 0, "the ring uses buffer loads");
            // this wave's loads per stage (tiles with fewer load instructions
            // than waves leave some waves without an A or B load)
            int lps = 0;
#pragma unroll
            for (int j = 0; j < A_INS; ++j)
                lps += (A_INS * NW == A_TOT || wave * A_INS + j < A_TOT);
#pragma unroll
            for (int j = 0; j < B_INS; ++j)
                lps += NB * (B_INS * NW == B_TOT || wave * B_INS + j < B_TOT);
            // s_waitcnt vmcnt(m * lps): at most m newer stages' loads may stay in
            // flight (m <= RS - 2; the count is wave-uniform, the wait needs an
            // immediate, so dispatch over the possible values: the RS - 1 values
            // of m when every wave issues LPS_MAX loads, else those of m * lps)
            auto wait_stages = [&](int64_t m) {
                if constexpr (LPS_ALL) {
                    static_for_int(std::make_integer_sequence<int, RS - 1>{}, [&](auto c) {
                        constexpr int M = decltype(c)::value, V = M * LPS_MAX;
                        if (m == M || (M == 0 && m < 0))
                            __builtin_amdgcn_s_waitcnt(0x3f70 | (V & 15) | ((V >> 4) << 14));
                    });
                    return;
                }
                const int v = m <= 0 ? 0 : static_cast<int>(m) * lps;
                constexpr int VMAX = (RS - 2) * LPS_MAX;
                static_for_int(std::make_integer_sequence<int, VMAX + 1>{}, [&](auto c) {
                    constexpr int V = decltype(c)::value;
                    if (v == V) __builtin_amdgcn_s_waitcnt(0x3f70 | (V & 15) | ((V >> 4) << 14));
                });
            };
            if (nk > 0) {
                // the first RS - 1 stages, then wait for the first of them
                static_for_int(std::make_integer_sequence<int, RS - 1>{}, [&](auto u) {
                    constexpr int U = decltype(u)::value;
                    if (U < nk) issue_to(ra(u), rb(u), kbeg + U * BK);
                });
                wait_stages(nk - 1 < RS - 2 ? nk - 1 : RS - 2);
                ring_barrier();
            }
            for (int64_t kt0 = 0; kt0 < nk; kt0 += RS) {
                // Step kt reads stage kt % RS, issues the loads of step kt + RS - 1
                // into the stage step kt - 1 read (every wave passed the barrier
                // after reading it), runs its burst, and before the barrier waits
                // for step kt + 1's loads: the later steps' may still be in flight.
                auto one = [&](auto off) {
                    constexpr int OFF = decltype(off)::value;
                    using U = std::integral_constant<int, OFF>;
                    const int64_t kt = kt0 + OFF;
                    if (kt >= nk) return;
                    read_frags(nblk, ra(U{}), rb(U{}));
                    using NX = std::integral_constant<int, (OFF + RS - 1) % RS>;
                    // Every step issues loads, so a step is one block whose
                    // loads the scheduler can spread among its MFMAs, and
                    // every step leaves the RS - 2 newest stages in flight:
                    // the last RS - 1 steps load step nk - 1 again, into
                    // stages that no later step reads.
                    const int64_t kn = kt + RS - 1 < nk ? kt + RS - 1 : nk - 1;
                    issue_to(ra(NX{}), rb(NX{}), kbeg + kn * BK);
                    mfma_step(nblk);
                    schedule_step(nblk);
                    wait_stages(RS - 2);
                    ring_barrier();
                };
                static_for_int(std::make_integer_sequence<int, RS>{}, [&](auto off) { one(off); });
            }
            // the repeated loads of the last steps land before the
            // workgroup's LDS is used again (or released)
            __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
        } else {
            if (nk > 0) {
                issue(0, kbeg);
                __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): this wave's loads landed
                __syncthreads();                      // ... and every other wave's
            }
            for (int64_t kt = 0; kt < nk; ++kt) {
                const int cur = static_cast<int>(kt & 1);
                read_frags(nblk, As[cur], &Bs[cur][0][0]);
                if (kt + 1 < nk) issue(cur ^ 1, kbeg + (kt + 1) * BK);
                mfma_step(nblk);
                __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
                __syncthreads();
            }
        }
    };
    if constexpr (RING) {
        if (live > 1 || (FM == 1 && live == 1)) k_loop(std::integral_constant<int, FM>{});
        else if (live == 1) k_loop(std::integral_constant<int, 1>{});
        else k_loop(std::integral_constant<int, 0>{});
    } else {
        k_loop(std::integral_constant<int, -1>{});
    }
    if constexpr (KW > 1) {
        static_assert(RING, "K groups run on the ring path");
        // Groups 1 .. KW - 1 put their accumulators in LDS, in the stage
        // arrays RB0 and RB1 (every wave's loads have landed and every
        // fragment read has ended at the barrier below), then group 0 adds
        // them to its own in group order -- K's first run, then the next --
        // and writes the tile.  Slot (g - 1) * NW + wave of PER_WAVE floats:
        // the first SLOTS in RB0, the rest in RB1.
        constexpr int PER_WAVE = NB * FM * FN * 16 * 64;  // floats
        constexpr int SLOTS = KSB / PER_WAVE;
        static_assert(2 * SLOTS >= (KW - 1) * NW, "reduction space");
        auto slot = [&](int g) -> float* {
            const int L = (g - 1) * NW + wave;
            return L < SLOTS ? RB0 + L * PER_WAVE : RB1 + (L - SLOTS) * PER_WAVE;
        };
        __syncthreads();
        if (wk > 0) {
            float* red = slot(wk);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int bi = 0; bi < FM; ++bi)
#pragma unroll
                    for (int bj = 0; bj < FN; ++bj)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4)
                            reinterpret_cast<f32x4*>(red)[(((nb * FM + bi) * FN + bj) * 4 + r4) * 64 + lane] =
                                f32x4{acc[nb][bi][bj][4 * r4], acc[nb][bi][bj][4 * r4 + 1],
                                      acc[nb][bi][bj][4 * r4 + 2], acc[nb][bi][bj][4 * r4 + 3]};
        }
        __syncthreads();
        if (wk > 0) return;  // no barrier follows
        for (int g = 1; g < KW; ++g) {
            const float* red = slot(g);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int bi = 0; bi < FM; ++bi)
#pragma unroll
                    for (int bj = 0; bj < FN; ++bj)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            const f32x4 v = reinterpret_cast<const f32x4*>(
                                red)[(((nb * FM + bi) * FN + bj) * 4 + r4) * 64 + lane];
#pragma unroll
                            for (int c = 0; c < 4; ++c) acc[nb][bi][bj][4 * r4 + c] += v[c];
                        }
        }
    }
    if constexpr (NSTRIDE) {
        // FN adjacent columns per lane and row: one 4 FN-byte store when they
        // all lie inside N and the row start is aligned to it
        typedef float f32xw __attribute__((ext_vector_type(FN)));
        const int64_t nc = n0 + bcol0 + FN * lr;
        const bool vecw = nc + FN - 1 < N && p.ldc % FN == 0 && p.c_split_stride % FN == 0 &&
                          (reinterpret_cast<uintptr_t>(Cb) & (4 * FN - 1)) == 0;
        // the lane's FN columns' bias, loaded once (see store_block)
        const bool hb = EPI == EPI_BIAS && p.bias != nullptr;
        f32xw bv;
#pragma unroll
        for (int bj = 0; bj < FN; ++bj) bv[bj] = hb && vecw ? p.bias[nc + bj] : 0.0f;
#pragma unroll
        for (int bi = 0; bi < FM; ++bi) {
            // the residual of this row of blocks, loaded before its stores
            // (resid may alias C: see store_tile)
            f32xw rv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
                for (int bj = 0; bj < FN; ++bj)
                    rv[r][bj] = EPI == EPI_BIAS && p.resid != nullptr && vecw && i < rows
                                    ? p.resid[(row0 + i) * p.ldc + nc + bj]
                                    : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = arow0 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (i >= rows) continue;
                if (vecw) {
                    f32xw v;
#pragma unroll
                    for (int bj = 0; bj < FN; ++bj) {
                        v[bj] = acc[0][bi][bj][r];
                        if (hb) v[bj] = v[bj] + bv[bj];
                        if (EPI == EPI_BIAS && p.resid != nullptr) v[bj] = v[bj] + rv[r][bj];
                    }
                    *reinterpret_cast<f32xw*>(&Cb[split * p.c_split_stride + (row0 + i) * p.ldc + nc]) = v;
                } else {
#pragma unroll
                    for (int bj = 0; bj < FN; ++bj)
                        if (nc + bj < N)
                            epi_store<EPI>(p, Cb, split, row0 + i, nc + bj, acc[0][bi][bj][r],
                                           acc[NB - 1][bi][bj][r]);
                }
            }
        }
        return;
    }
    if (part != nullptr) {
        f32x4* dst = reinterpret_cast<f32x4*>(part);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int bi = 0; bi < FM; ++bi)
#pragma unroll
                for (int bj = 0; bj < FN; ++bj)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4)
                        dst[sk_part_index<C, NB>(nb, bi, bj, r4, tid)] =
                            f32x4{acc[nb][bi][bj][4 * r4], acc[nb][bi][bj][4 * r4 + 1],
                                  acc[nb][bi][bj][4 * r4 + 2], acc[nb][bi][bj][4 * r4 + 3]};
        return;
    }
    store_tile<C, NB, EPI>(p, Cb, split, row0, rows, n0, acc, tid);
}

template <class C, int SCHED, bool NN, bool GROUPED, int NB, int EPI>
__global__ __launch_bounds__(C::THREADS, 2) void gemm_direct_kernel(const GemmArgs p) {
    int mt, nt, split;  // split: K range of this tile (split-K)
    if (!launch_tile<C::BM, GROUPED>(p, mt, nt, split)) return;  // surplus workgroup
    direct_tile<C, SCHED, NN, GROUPED, NB, EPI>(p, mt, nt, split, -1, -1, nullptr);
}

// ---------------------------------------------------------------------------
// Stream-K grouped GEMM.  The grid holds as many workgroups G as the GPU
// runs at once.  The real tiles of the launch (counted from the offsets), in
// raster order, first go out whole, G at a time, for as many full rounds as
// they fill (tiles / G); the tiles left over, fewer than G, are laid end to
// end, K steps within a tile, and their I = tiles x K-steps iterations are
// dealt in contiguous ranges, q = I / G to each logical workgroup and one
// more to the first I % G: every workgroup does the same number of K steps
// (within one), so the launch has no partly filled last round of whole
// tiles.  (Dealing every tile that way puts the workgroups of an XCD at
// unrelated K offsets, so tiles that share an operand panel no longer read
// it from L2 together: measured 7-10 % slower per K step.)  A tile that lies
// within one workgroup's range is written by its epilogue as usual; a tile
// cut by range boundaries leaves one partial accumulator set per piece, the
// piece at the start of a workgroup's range in slot 2w, the piece at its end
// in slot 2w + 1, and the fix-up kernel (a second launch on the same stream)
// adds the pieces in K order and runs the epilogue.  No workgroup waits for
// another.  Logical workgroups are dealt to the XCDs in contiguous runs, so
// each XCD works through a contiguous run of tiles.
struct SkSched {
    int m_tiles, tiles, group, nk;
    int rounds;  // whole-tile rounds before the stream-K part: tiles / G
    int base;    // first iteration of the stream-K part: rounds * G * nk
    int q, r;    // its iterations per workgroup: q + 1 for the first r workgroups, q after
};

// The schedule of a stream-K launch on G workgroups (every count fits 31
// bits: the host checks tiles x K steps).
template <int BM, int BK>
__device__ __forceinline__ SkSched sk_sched(const GemmArgs& p, int G) {
    SkSched s;
    const int real = grouped_real_m_tiles<BM>(p.offsets, p.E);
    s.m_tiles = real < p.m_tiles ? real : p.m_tiles;
    s.tiles = s.m_tiles * p.n_tiles;
    s.group = p.group_m < s.m_tiles ? p.group_m : s.m_tiles;
    s.nk = static_cast<int>(p.K / BK);
    s.rounds = s.tiles / G;
    s.base = s.rounds * G * s.nk;
    const int iters = (s.tiles - s.rounds * G) * s.nk;
    s.q = iters / G;
    s.r = iters - s.q * G;
    return s;
}

// First iteration of logical workgroup w in the stream-K part (w = G: the
// end of the launch).
__device__ __forceinline__ int sk_begin(const SkSched& s, int w) {
    return s.base + w * s.q + (w < s.r ? w : s.r);
}

template <class C, int SCHED, int NB, int EPI>
__global__ __launch_bounds__(C::THREADS, 2) void gemm_sk_kernel(const GemmArgs p) {
    const int G = static_cast<int>(gridDim.x);
    const SkSched s = sk_sched<C::BM, C::BK>(p, G);
    const int w = xcd_remap(blockIdx.x, G);
    // whole tiles first, round by round (the workgroups of an XCD run a
    // contiguous run of tiles in step, as the one-tile kernel does), then
    // this workgroup's range of the rest; one call site, so the tile code is
    // inlined once
    const int beg = sk_begin(s, w), end = sk_begin(s, w + 1);
    constexpr int64_t SLOT = int64_t(NB) * C::BM * C::BN;
    int round = 0, it = beg;
    for (;;) {
        int t, ks, ke;
        float* part = nullptr;
        if (round < s.rounds) {
            t = round * G + w;
            ks = 0;
            ke = s.nk;
            ++round;
        } else if (it < end) {
            t = it / s.nk;
            ks = it - t * s.nk;
            ke = s.nk - ks < end - it ? s.nk : ks + (end - it);
            if (ks != 0 || ke != s.nk)
                part = p.sk_part + (2 * int64_t(w) + (it == beg ? 0 : 1)) * SLOT;
            it += ke - ks;
        } else {
            break;
        }
        int mt, nt;
        tile_of(t, s.m_tiles, p.n_tiles, s.group, mt, nt);
        direct_tile<C, SCHED, false, true, NB, EPI, true>(p, mt, nt, 0, ks, ke, part);
    }
}

// The fix-up of the stream-K launch with the same arguments: block (b, q)
// looks at the boundary between logical workgroups b and b + 1.  When it
// cuts a tile and workgroup b's range holds that tile's first K step (so no
// earlier boundary cuts it), the block adds the pieces of the tile's
// accumulator block q (one 32x32 block per wave, for every B operand) in K
// order -- the piece of workgroup b, then those of b + 1, b + 2, ... up to
// the tile's end -- and writes it through the epilogue.  FM x FN blocks per
// tile keep each block's chain of dependent loads short (one block per tile
// took 0.16 ms at config 3's w2, whose 64 cut tiles have 8 pieces each).
template <class C, int NB, int EPI>
__global__ __launch_bounds__(C::THREADS, 2) void gemm_sk_fixup_kernel(const GemmArgs p) {
    const int G = p.sk_grid;
    const SkSched s = sk_sched<C::BM, C::BK>(p, G);
    const int w = static_cast<int>(blockIdx.x) + 1;
    const int b = sk_begin(s, w);
    if (b >= sk_begin(s, G)) return;
    const int t = b / s.nk, t0 = t * s.nk, t1 = t0 + s.nk;
    if (b == t0) return;                       // the boundary falls between tiles
    const int prev = sk_begin(s, w - 1);
    if (prev > t0) return;                     // an earlier boundary cuts this tile
    constexpr int64_t SLOT = int64_t(NB) * C::BM * C::BN;
    const int bi = static_cast<int>(blockIdx.y) / C::FN, bj = static_cast<int>(blockIdx.y) % C::FN;
    const int tid = threadIdx.x;
    f32x16 acc[NB];
    auto add_slot = [&](int64_t slot, bool first) {
        const f32x4* src = reinterpret_cast<const f32x4*>(p.sk_part + slot * SLOT);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const f32x4 v = src[sk_part_index<C, NB>(nb, bi, bj, r4, tid)];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[nb][4 * r4 + j] = first ? v[j] : acc[nb][4 * r4 + j] + v[j];
            }
    };
    // workgroup w - 1 holds the tile's first piece: in its start slot when
    // its range begins at the tile's start, else in its end slot
    add_slot(2 * int64_t(w - 1) + (prev == t0 ? 0 : 1), true);
    // The later pieces (the start slots of workgroups w, w + 1, ... while
    // their ranges begin inside the tile), up to 4 at a time: every load of
    // a batch is issued before its adds, which keep the K order, so a tile
    // cut into many short pieces costs one memory round trip per 4 pieces,
    // not per piece.
    constexpr int PB = 4;
    bool more = true;
    for (int u = w; more;) {
        int64_t slot[PB];
        int n = 0;
        while (n < PB) {
            if (u >= G) { more = false; break; }
            const int bu = sk_begin(s, u);
            if (bu >= t1) { more = false; break; }
            if (sk_begin(s, u + 1) != bu) slot[n++] = 2 * int64_t(u);  // skip empty ranges
            ++u;
        }
        f32x4 v[PB][NB * 4];
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            if (i >= n) break;
            const f32x4* src = reinterpret_cast<const f32x4*>(p.sk_part + slot[i] * SLOT);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    v[i][nb * 4 + r4] = src[sk_part_index<C, NB>(nb, bi, bj, r4, tid)];
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            if (i >= n) break;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[nb][4 * r4 + j] = acc[nb][4 * r4 + j] + v[i][nb * 4 + r4][j];
        }
    }
    int mt, nt;
    tile_of(t, s.m_tiles, p.n_tiles, s.group, mt, nt);
    int e, rows;
    int64_t row0;
    if (!grouped_tile_rows<C::BM>(p, mt, e, row0, rows)) return;
    store_block<C, EPI>(p, p.C, 0, row0, rows, static_cast<int64_t>(nt) * C::BN, bi, bj, acc[0],
                        acc[NB - 1], tid);
}

// ---------------------------------------------------------------------------
// Skinny dense GEMM (M <= 64): B streams once from HBM straight into
// registers, no LDS and no barriers.  Each wave owns 64 columns and all
// 16 * MB rows of the product over its K range (K splits: grid.y), on
// v_mfma_f32_16x16x4_f32 -- 16 rows per MFMA, so M = 16 wastes no matrix-core
// work (the 32 x 32 tiles compute twice the rows).  In a 16-wide K chunk lane
// (j, g) = (lane % 16, lane / 16) holds k = k0 + 4g .. k0 + 4g + 3, one per
// MFMA step s, for A (one 16-byte load per 16-row block: row 16 mb + j) and
// B, so the four steps cover the chunk's 16 k exactly once:
//   NN ([K, N]): B row k0 + 4g + s, columns n0 + 4j .. 4j + 3 (16 bytes; the
//     four column blocks c are the columns 4j + c, so a lane ends up with 4
//     adjacent columns of each output row: one 16-byte store);
//   NT ([N, K]): B rows n0 + 16c + j, k0 + 4g .. 4g + 3 (16 bytes per block c).
// 16x16 accumulator layout: lane l, register r holds row 4 (l / 16) + r,
// column block entry l % 16.  Chunks are loaded PF ahead into a register
// ring (the K loop unrolled over it).  Rows past M and columns past N load a
// valid row or column and are masked at the store.  Requires K % 16 == 0,
// 16-byte aligned rows, and for NN N % 4 == 0.
typedef float f32x4s __attribute__((ext_vector_type(4)));

template <bool NN, int MB, int EPI>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(const GemmArgs p) {
    constexpr int PF = MB >= 4 ? 3 : 4;  // chunks in flight besides the one computed
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int64_t N = p.N, M = p.M;
    const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * 64;
    if (n0 >= N) return;  // a wave past the last column block (no barrier in this kernel)
    const int split = blockIdx.y;
    const int64_t kbeg = split * p.k_split_len;
    const int64_t kend = p.K - kbeg < p.k_split_len ? p.K : kbeg + p.k_split_len;
    const int64_t nch = (kend - kbeg) / 16;

    const float* arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        int64_t r = 16 * mb + j;
        r = r < M ? r : M - 1;
        arow[mb] = p.A + r * p.lda + 4 * g;
    }
    const float* bptr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (NN) {
            int64_t c = n0 + 4 * j;
            c = c < N ? c : N - 4;
            bptr[q] = p.B0 + (4 * g + q) * p.ldb + c;  // step q's k-row
        } else {
            int64_t n = n0 + 16 * q + j;
            n = n < N ? n : N - 1;
            bptr[q] = p.B0 + n * p.ldb + 4 * g;        // block q's column
        }
    }
    struct Chunk {
        f32x4s a[MB], b[4];
    };
    auto load = [&](Chunk& c, int64_t k0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) c.a[mb] = *reinterpret_cast<const f32x4s*>(arow[mb] + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            c.b[q] = *reinterpret_cast<const f32x4s*>(bptr[q] + (NN ? k0 * p.ldb : k0));
    };
    f32x4s acc[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[mb][c] = f32x4s{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Chunk& c) {
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[mb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        c.a[mb][st], NN ? c.b[st][cb] : c.b[cb][st], acc[mb][cb], 0, 0, 0);
    };
    Chunk ring[PF + 1];
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (u < nch) load(ring[u], kbeg + 16 * u);
    for (int64_t c0 = 0; c0 < nch; c0 += PF + 1) {
#pragma unroll
        for (int u = 0; u <= PF; ++u) {
            const int64_t ci = c0 + u;
            if (ci < nch) {
                if (ci + PF < nch) load(ring[(u + PF) % (PF + 1)], kbeg + 16 * (ci + PF));
                compute(ring[u]);
            }
        }
    }

    // epilogue: split partials (no bias) or the output with bias; the bias
    // of the lane's columns is loaded once (see store_block)
    float* Cb = p.C + split * p.c_split_stride;
    const bool hb = EPI == EPI_BIAS && p.bias != nullptr;
    float bcol[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int64_t col = NN ? n0 + 4 * j + c : n0 + 16 * c + j;
        bcol[c] = hb && col < N ? p.bias[col] : 0.0f;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = 16 * mb + 4 * g + r;
            if (row >= M) continue;
            if (NN) {
                const int64_t col = n0 + 4 * j;
                if (col >= N) continue;
                f32x4s v{acc[mb][0][r], acc[mb][1][r], acc[mb][2][r], acc[mb][3][r]};
                if (hb)
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] = v[c] + bcol[c];
                if (EPI == EPI_BIAS && p.resid != nullptr)
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] = v[c] + p.resid[row * p.ldc + col + c];
                *reinterpret_cast<f32x4s*>(Cb + row * p.ldc + col) = v;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int64_t col = n0 + 16 * c + j;
                    if (col >= N) continue;
                    float v = acc[mb][c][r];
                    if (hb) v = v + bcol[c];
                    if (EPI == EPI_BIAS && p.resid != nullptr) v = v + p.resid[row * p.ldc + col];
                    Cb[row * p.ldc + col] = v;
                }
            }
        }
}

template <bool NN>
void launch_skinny(const GemmArgs& a, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(ceil_div(a.N, 256)), static_cast<unsigned>(a.k_splits));
    const int mb = static_cast<int>(ceil_div(a.M, 16));
    if (mb <= 1) hipLaunchKernelGGL((gemm_skinny_kernel<NN, 1, EPI_BIAS>), grid, dim3(256), 0, s, a);
    else if (mb <= 2) hipLaunchKernelGGL((gemm_skinny_kernel<NN, 2, EPI_BIAS>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((gemm_skinny_kernel<NN, 4, EPI_BIAS>), grid, dim3(256), 0, s, a);
}

// ---------------------------------------------------------------------------
// Grouped skinny expert GEMM (NT, w1/w3 or w2) for layers whose experts hold
// few rows each -- a batch of 64 tokens over 4 experts, a decoder's last rows
// -- where the tiled kernels' 128-row tiles are mostly empty and the run is a
// few K steps of load latency per tile.  A workgroup owns one expert's block
// of 16 * MB packed rows and 64 columns; its four waves take four consecutive
// quarters of the K range (grid.z: the w2 K splits, each its own partial
// rows) and stream A and B straight into registers as the skinny dense
// kernel does (v_mfma_f32_16x16x4_f32, the same lane layout), then meet in
// LDS: every output is the waves' partials added in wave order, then the
// epilogue.  grid.y = E * rb, rb the row blocks of the largest expert the
// launch allows for (rows_limit / (16 * MB), rounded up); blocks past an
// expert's rows exit at once.  With K splits, an activation launch (SiLU,
// SwiGLU) stores each split's raw sums of its B operands instead,
// sk_part[split][row][o * N + n], and skinny_act_fixup_kernel adds them in
// split order and applies the activation.  Requires K % 16 == 0 per split
// and 16-byte aligned rows.
template <int MB, int NBO, int EPI>
__global__ __launch_bounds__(256) void gemm_skinny_grouped_kernel(const GemmArgs p, int rb) {
    // chunks in flight besides the one computed (3 and 5, or 4 and 6, measured
    // 1-7 % slower on the planner's shapes)
    constexpr int PF = NBO == 2 ? 2 : 3;
    constexpr int RW = 16 * MB;           // rows of the workgroup
    constexpr int LDR = 65;               // LDS row stride of a partial (64 columns + 1)
    __shared__ float red[4][NBO][RW * LDR];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int j = lane & 15, g = lane >> 4;
    const int e = static_cast<int>(blockIdx.y) / rb, b = static_cast<int>(blockIdx.y) % rb;
    const int64_t end = p.offsets[e + 1];
    const int64_t row0 = p.offsets[e] + static_cast<int64_t>(b) * RW;
    if (row0 >= end) return;  // the whole workgroup (no barrier reached yet)
    const int64_t N = p.N, n0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int split = blockIdx.z;
    const int64_t kbeg = split * p.k_split_len;
    const int64_t kend = p.K - kbeg < p.k_split_len ? p.K : kbeg + p.k_split_len;
    const int64_t nch = (kend - kbeg) / 16;
    const int64_t c0 = nch * wave / 4, c1 = nch * (wave + 1) / 4;  // this wave's chunks

    const float* arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        int64_t r = row0 + 16 * mb + j;
        r = r < end ? r : end - 1;
        int64_t t = r;
        if (p.gather != nullptr) {  // a token row of A, clamped to the rows it has
            t = p.gather[r];
            t = t < 0 ? 0 : (t >= p.gather_rows ? p.gather_rows - 1 : t);
        }
        arow[mb] = p.A + t * p.lda + 4 * g;
    }
    const float* bptr[NBO][4];
#pragma unroll
    for (int o = 0; o < NBO; ++o)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int64_t n = n0 + 16 * q + j;
            n = n < N ? n : N - 1;
            bptr[o][q] = (o == 0 ? p.B0 : p.B1) + e * p.b_expert_stride + n * p.ldb + 4 * g;
        }
    struct Chunk {
        f32x4s a[MB], b[NBO][4];
    };
    auto load = [&](Chunk& c, int64_t k0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) c.a[mb] = *reinterpret_cast<const f32x4s*>(arow[mb] + k0);
#pragma unroll
        for (int o = 0; o < NBO; ++o)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                c.b[o][q] = *reinterpret_cast<const f32x4s*>(bptr[o][q] + k0);
    };
    f32x4s acc[NBO][MB][4];
#pragma unroll
    for (int o = 0; o < NBO; ++o)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[o][mb][c] = f32x4s{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Chunk& c) {
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int o = 0; o < NBO; ++o)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
                        acc[o][mb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            c.a[mb][st], c.b[o][cb][st], acc[o][mb][cb], 0, 0, 0);
    };
    const int64_t n_my = c1 - c0;
    Chunk ring[PF + 1];
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (u < n_my) load(ring[u], kbeg + 16 * (c0 + u));
    for (int64_t i0 = 0; i0 < n_my; i0 += PF + 1) {
#pragma unroll
        for (int u = 0; u <= PF; ++u) {
            const int64_t ci = i0 + u;
            if (ci < n_my) {
                if (ci + PF < n_my) load(ring[(u + PF) % (PF + 1)], kbeg + 16 * (c0 + ci + PF));
                compute(ring[u]);
            }
        }
    }

    // partials to LDS: lane (j, g), register i of block (mb, cb) is row
    // 16 mb + 4 g + i, column 16 cb + j
#pragma unroll
    for (int o = 0; o < NBO; ++o)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    red[wave][o][(16 * mb + 4 * g + i) * LDR + 16 * cb + j] = acc[o][mb][cb][i];
    __syncthreads();
    // every output: the four waves' partials in wave order, then the epilogue
    // (or, for an activation split over K, the split's raw sums)
    float* Cb = p.C;
    const bool raw = EPI != EPI_STORE && p.k_splits > 1;
    for (int idx = threadIdx.x; idx < RW * 64; idx += 256) {
        const int r = idx >> 6, c = idx & 63;
        const int64_t row = row0 + r, n = n0 + c;
        if (row >= end || n >= N) continue;
        float v[NBO];
#pragma unroll
        for (int o = 0; o < NBO; ++o) {
            float sum = red[0][o][r * LDR + c];
#pragma unroll
            for (int w = 1; w < 4; ++w) sum += red[w][o][r * LDR + c];
            v[o] = sum;
        }
        if (raw) {
#pragma unroll
            for (int o = 0; o < NBO; ++o)
                p.sk_part[(split * p.rows_limit + row) * (NBO * N) + o * N + n] = v[o];
        } else {
            epi_store<EPI>(p, Cb, split, row, n, v[0], v[NBO - 1]);
        }
    }
}

// The activation of a K-split grouped skinny launch: h[row][n] = act of the
// splits' sums of each B operand, added in split order.
template <int NBO, int EPI>
__global__ __launch_bounds__(256) void skinny_act_fixup_kernel(const float* __restrict__ part,
                                                               float* __restrict__ h,
                                                               int64_t rows, int64_t N,
                                                               int64_t ldh, int splits) {
    const int64_t total = rows * N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const int64_t row = i / N, n = i % N;
        float v[NBO];
#pragma unroll
        for (int o = 0; o < NBO; ++o) {
            float sum = part[row * (NBO * N) + o * N + n];
            for (int sp = 1; sp < splits; ++sp)
                sum += part[(sp * rows + row) * (NBO * N) + o * N + n];
            v[o] = sum;
        }
        h[row * ldh + n] = EPI == EPI_SWIGLU ? silu_ref(v[0]) * v[NBO - 1] : silu_ref(v[0]);
    }
}

template <int MB>
void launch_skinny_grouped_mb(const GemmArgs& a, int epi, hipStream_t s) {
    const int rb = static_cast<int>(ceil_div(a.rows_limit, 16 * MB));
    const dim3 grid(static_cast<unsigned>(ceil_div(a.N, 64)), static_cast<unsigned>(a.E * rb),
                    static_cast<unsigned>(a.k_splits));
    switch (epi) {
        case EPI_SWIGLU:
            hipLaunchKernelGGL((gemm_skinny_grouped_kernel<MB, 2, EPI_SWIGLU>), grid, dim3(256), 0,
                               s, a, rb);
            break;
        case EPI_SILU:
            hipLaunchKernelGGL((gemm_skinny_grouped_kernel<MB, 1, EPI_SILU>), grid, dim3(256), 0,
                               s, a, rb);
            break;
        case EPI_STORE:
            hipLaunchKernelGGL((gemm_skinny_grouped_kernel<MB, 1, EPI_STORE>), grid, dim3(256), 0,
                               s, a, rb);
            break;
        default: throw Unsupported("grouped skinny epilogue");
    }
}

// Whether every byte offset of a SCHED_BUFLDS launch (lane offset from the
// operand's base plus the K step's scalar offset) stays below 2^31.
bool buf_offsets_fit(const GemmArgs& a, int bm, int bn, bool nn, bool grouped) {
    constexpr int64_t lim = int64_t(1) << 31;
    const int64_t a_rows = grouped && a.gather != nullptr ? a.gather_rows : bm;
    const int64_t a_bytes = (a_rows + 1) * a.lda * 4;
    const int64_t b_bytes = nn ? (a.K + 16) * a.ldb * 4 + int64_t(bn) * 4 : (int64_t(bn) + 1) * a.ldb * 4;
    return a_bytes < lim && b_bytes < lim;
}

template <class C, int SCHED, bool NN, bool GROUPED, int NB, int EPI>
void launch_cfg(const GemmArgs& a, bool vec, hipStream_t s) {
    // direct global->LDS path: 16-byte aligned rows, K a multiple of 16 (NN:
    // B's rows, of N floats, 16-byte aligned too)
    if constexpr ((SCHED & SCHED_DIRECT) != 0 && C::BK == 16) {
        const bool b_ok = !NN || (a.ldb % 4 == 0 && a.N % 4 == 0 &&
                                  reinterpret_cast<uintptr_t>(a.B0) % 16 == 0);
        if (vec && b_ok && a.K % 16 == 0 && a.k_split_len % 16 == 0) {
            const dim3 grid(static_cast<unsigned>(a.m_tiles) * static_cast<unsigned>(a.n_tiles) *
                            static_cast<unsigned>(a.k_splits));
            const bool fits = buf_offsets_fit(a, C::BM, C::BN, NN, GROUPED);
            if constexpr (C::KW > 1) {
                // K groups: the ring path only, every group the same K steps
                static_assert((SCHED & SCHED_BUFLDS) && (SCHED & SCHED_RING3), "K groups need the ring");
                if (!fits || a.k_splits != 1 || (a.K / 16) % C::KW != 0)
                    throw Unsupported("K-group GEMM tile: operands past 2 GiB or K steps not a "
                                      "multiple of the groups");
                hipLaunchKernelGGL((gemm_direct_kernel<C, SCHED, NN, GROUPED, NB, EPI>), grid,
                                   dim3(C::THREADS), 0, s, a);
                return;
            } else {
                if (!(SCHED & SCHED_BUFLDS) || fits)
                    hipLaunchKernelGGL((gemm_direct_kernel<C, SCHED, NN, GROUPED, NB, EPI>), grid,
                                       dim3(C::THREADS), 0, s, a);
                else
                    hipLaunchKernelGGL(
                        (gemm_direct_kernel<C, (SCHED & ~(SCHED_BUFLDS | SCHED_RING3)), NN, GROUPED, NB, EPI>), grid,
                        dim3(C::THREADS), 0, s, a);
                return;
            }
        }
    }
    if constexpr (C::STAGED) {
        const dim3 grid(static_cast<unsigned>(a.m_tiles) * static_cast<unsigned>(a.n_tiles) *
                        static_cast<unsigned>(a.k_splits));
        if (vec)
            hipLaunchKernelGGL((gemm_kernel<C, SCHED, NN, true, GROUPED, NB, EPI>), grid,
                               dim3(C::THREADS), 0, s, a);
        else
            hipLaunchKernelGGL((gemm_kernel<C, SCHED, NN, false, GROUPED, NB, EPI>), grid,
                               dim3(C::THREADS), 0, s, a);
    } else {
        throw Unsupported("GEMM tile shape needs aligned rows and K % 16 == 0");
    }
}

// The stream-K launch of a grouped GEMM and its fix-up (grid sk_grid - 1:
// one block per range boundary).  It needs the direct buffer-load path:
// where that does not apply (unaligned rows, K % 16 != 0, operands past
// 2 GiB), the one-tile-per-workgroup launch runs instead.
template <class C, int SCHED, int NB, int EPI>
void launch_sk(const GemmArgs& a, bool vec, hipStream_t s) {
    static_assert((SCHED & SCHED_BUFLDS) != 0 && (SCHED & SCHED_DIRECT) != 0, "stream-K path");
    if (!vec || a.K % 16 != 0 || !buf_offsets_fit(a, C::BM, C::BN, false, true)) {
        GemmArgs d = a;
        d.sk_grid = 0;
        launch_cfg<C, SCHED, false, true, NB, EPI>(d, vec, s);
        return;
    }
    hipLaunchKernelGGL((gemm_sk_kernel<C, SCHED, NB, EPI>), dim3(a.sk_grid), dim3(C::THREADS), 0,
                       s, a);
    if (a.sk_grid > 1)
        hipLaunchKernelGGL((gemm_sk_fixup_kernel<C, NB, EPI>),
                           dim3(a.sk_grid - 1, C::FM * C::FN), dim3(C::THREADS), 0, s, a);
}

using DenseCfg = CfgOf<MOE_DENSE_CFG>::T;
using DenseMidCfg = CfgOf<8>::T;
using DenseSmallCfg = CfgOf<9>::T;
using DenseTallCfg = CfgOf<11>::T;  // 256 x 128, each wave 64 rows x 128 columns
using DenseKwCfg = CfgOf<12>::T;  // 32 x 128, four K groups
using W13Cfg = CfgOf<MOE_W13_CFG>::T;
using W2Cfg = CfgOf<MOE_W2_CFG>::T;
using W2NarrowCfg = CfgOf<0>::T;  // w2 with d too narrow for the wide tile's n-tiles
using W13TallCfg = CfgOf<10>::T;  // w1/w3 with d_ff % 128 == 64

template <class C, bool NN>
void launch_dense(const GemmArgs& a, bool vec, hipStream_t s) {
    launch_cfg<C, MOE_DENSE_SMALL_SCHED | SCHED_DIRECT, NN, false, 1, EPI_BIAS>(a, vec, s);
}

template <class C, int SCHED>
int dense_occupancy(bool nn) {
    int n = 0;
    const hipError_t e =
        nn ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                 &n, gemm_direct_kernel<C, SCHED, true, false, 1, EPI_BIAS>, C::THREADS, 0)
           : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                 &n, gemm_direct_kernel<C, SCHED, false, false, 1, EPI_BIAS>, C::THREADS, 0);
    hip_check(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    return n > 0 ? n : 1;
}

}  // namespace

namespace {
template <class C, bool NN>
void launch_batched_cfg(const GemmArgs& args, int batches, hipStream_t s) {
    GemmArgs a = args;
    a.m_tiles = static_cast<int32_t>(ceil_div(a.M, C::BM));
    a.n_tiles = static_cast<int32_t>(ceil_div(a.N, C::BN));
    a.group_m = a.m_tiles;
    a.k_splits = 1;
    a.k_split_len = a.K;
    a.c_split_stride = 0;
    constexpr int SCHED = MOE_DENSE_SCHED | SCHED_DIRECT;
    const dim3 grid(static_cast<unsigned>(a.m_tiles) * static_cast<unsigned>(a.n_tiles),
                    static_cast<unsigned>(batches));
    if (!(SCHED & SCHED_BUFLDS) || buf_offsets_fit(a, C::BM, C::BN, NN, false))
        hipLaunchKernelGGL((gemm_direct_kernel<C, SCHED, NN, false, 1, EPI_BIAS>), grid,
                           dim3(C::THREADS), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_direct_kernel<C, (SCHED & ~(SCHED_BUFLDS | SCHED_RING3)), NN, false, 1, EPI_BIAS>),
                           grid, dim3(C::THREADS), 0, s, a);
}
}  // namespace

void launch_gemm_batched(const GemmArgs& a, bool nn, int batches, hipStream_t s) {
    if (batches <= 0 || a.M <= 0 || a.N <= 0) return;
    if (a.resid != nullptr) throw Unsupported("batched GEMM with a residual");
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool ok = a.K % 16 == 0 && a.lda % 4 == 0 && a.ldb % 4 == 0 && al(a.A) && al(a.B0) &&
                    (!nn || a.N % 4 == 0) && a.a_so % 4 == 0 && a.a_si % 4 == 0 &&
                    a.b_so % 4 == 0 && a.b_si % 4 == 0;
    if (!ok) throw Unsupported("batched GEMM needs 16-byte aligned rows and K % 16 == 0");
    // narrow outputs (an attention head's 64 values) take the 128 x 64 tile
    if (a.N <= 64) {
        if (nn) launch_batched_cfg<CfgOf<3>::T, true>(a, batches, s);
        else launch_batched_cfg<CfgOf<3>::T, false>(a, batches, s);
    } else {
        if (nn) launch_batched_cfg<DenseCfg, true>(a, batches, s);
        else launch_batched_cfg<DenseCfg, false>(a, batches, s);
    }
}

GemmTile dense_tile(int tile) {
    switch (tile) {
        case kDenseKwTile: return {DenseKwCfg::BM, DenseKwCfg::BN};
        case 1: return {DenseMidCfg::BM, DenseMidCfg::BN};
        case 2: return {DenseSmallCfg::BM, DenseSmallCfg::BN};
        case 3: return {DenseTallCfg::BM, DenseTallCfg::BN};
        default: return {DenseCfg::BM, DenseCfg::BN};
    }
}

int dense_tile_groups(int tile) { return tile == kDenseKwTile ? DenseKwCfg::KW : 1; }

int dense_blocks_per_cu(int tile, bool nn) {
    switch (tile) {
        case kDenseKwTile: return dense_occupancy<DenseKwCfg, MOE_DENSE_SMALL_SCHED | SCHED_DIRECT>(nn);
        case 1: return dense_occupancy<DenseMidCfg, MOE_DENSE_SMALL_SCHED | SCHED_DIRECT>(nn);
        case 2: return dense_occupancy<DenseSmallCfg, MOE_DENSE_SMALL_SCHED | SCHED_DIRECT>(nn);
        case 3: return dense_occupancy<DenseTallCfg, MOE_DENSE_TALL_SCHED | SCHED_DIRECT>(nn);
        default: return dense_occupancy<DenseCfg, MOE_DENSE_SCHED | SCHED_DIRECT>(nn);
    }
}

int gemm_blocks_per_cu(GemmUse use) {
    int n = 0;
    hipError_t e = hipSuccess;
    auto query = [&](auto kernel, int threads) {
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0);
    };
    switch (use) {
        case GemmUse::W2Narrow:
            query(gemm_direct_kernel<W2NarrowCfg, MOE_W2_SCHED | SCHED_DIRECT, false, true, 1,
                                     EPI_STORE>,
                  W2NarrowCfg::THREADS);
            break;
        case GemmUse::W2:
            if constexpr ((MOE_W2_SCHED & SCHED_DIRECT) != 0 && W2Cfg::BK == 16)
                query(gemm_direct_kernel<W2Cfg, MOE_W2_SCHED, false, true, 1, EPI_STORE>,
                      W2Cfg::THREADS);
            else
                query(gemm_kernel<W2Cfg, MOE_W2_SCHED, false, true, true, 1, EPI_STORE>,
                      W2Cfg::THREADS);
            break;
        case GemmUse::W13Tall:
            query(gemm_direct_kernel<W13TallCfg, MOE_W13_SCHED, false, true, 2, EPI_SWIGLU>,
                  W13TallCfg::THREADS);
            break;
        default:
            if constexpr ((MOE_W13_SCHED & SCHED_DIRECT) != 0 && W13Cfg::BK == 16)
                query(gemm_direct_kernel<W13Cfg, MOE_W13_SCHED, false, true, 2, EPI_SWIGLU>,
                      W13Cfg::THREADS);
            else
                query(gemm_kernel<W13Cfg, MOE_W13_SCHED, false, true, true, 2, EPI_SWIGLU>,
                      W13Cfg::THREADS);
            break;
    }
    hip_check(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    return n > 0 ? n : 1;
}

int gemm_sk_blocks_per_cu(GemmUse use) {
    int n = 0;
    hipError_t e = hipSuccess;
    auto query = [&](auto kernel, int threads) {
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0);
    };
    switch (use) {
        case GemmUse::W2Narrow:
            query(gemm_sk_kernel<W2NarrowCfg, MOE_W2_SCHED | SCHED_DIRECT, 1, EPI_STORE>,
                  W2NarrowCfg::THREADS);
            break;
        case GemmUse::W2:
            query(gemm_sk_kernel<W2Cfg, MOE_W2_SCHED | SCHED_DIRECT, 1, EPI_STORE>,
                  W2Cfg::THREADS);
            break;
        case GemmUse::W13Tall:
            query(gemm_sk_kernel<W13TallCfg, MOE_W13_SCHED | SCHED_DIRECT, 2, EPI_SWIGLU>,
                  W13TallCfg::THREADS);
            break;
        default:
            query(gemm_sk_kernel<W13Cfg, MOE_W13_SCHED | SCHED_DIRECT, 2, EPI_SWIGLU>,
                  W13Cfg::THREADS);
            break;
    }
    hip_check(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    return n > 0 ? n : 1;
}

int64_t gemm_sk_part_floats(GemmUse use, int grid) {
    const GemmTile t = gemm_tile(use);
    const int nb = (use == GemmUse::W13 || use == GemmUse::W13Tall) ? 2 : 1;
    return 2 * int64_t(grid) * nb * t.bm * t.bn;
}

GemmTile gemm_tile(GemmUse use) {
    switch (use) {
        case GemmUse::Dense: return {DenseCfg::BM, DenseCfg::BN};
        case GemmUse::W13: return {W13Cfg::BM, W13Cfg::BN};
        case GemmUse::W2Narrow: return {W2NarrowCfg::BM, W2NarrowCfg::BN};
        case GemmUse::W13Tall: return {W13TallCfg::BM, W13TallCfg::BN};
        default: return {W2Cfg::BM, W2Cfg::BN};
    }
}

void launch_gemm(const GemmArgs& args, bool nn, bool grouped, int epi, bool vec,
                 hipStream_t s) {
    if (args.m_tiles <= 0 || args.n_tiles <= 0) return;
    GemmArgs a = args;
    // Raster group (m-tiles per n-sweep).  MOE_GEMM_GROUP_M overrides the
    // default for tuning; values outside [1, m_tiles] mean m_tiles.
    static const int env_group = [] {
        const char* v = std::getenv("MOE_GEMM_GROUP_M");
        return v != nullptr ? std::atoi(v) : 0;
    }();
    int group = env_group != 0
                    ? env_group
                    : (grouped && epi != EPI_STORE && a.K <= 1024 ? kGemmGroupMShortK : kGemmGroupM);
    // the grouped w2 over many experts: m-fastest (config 4's 64 experts, same box, w2
    // per launch 5.57 -> 5.46 ms at 16,384 tokens, 1.61 -> 1.51 ms at 4,096, 0.59 -> 0.52 ms
    // at 1,024, 0.38 -> 0.22 ms at 256; bit-identical; its w1/w3 measured level or slower)
    if (env_group == 0 && grouped && epi == EPI_STORE && a.E >= 32) group = 0;
    // ... and so does the w1/w3 over many experts while they average at most 32 rows (config
    // 4, same box, ms per layer: 64 / 128 / 256 tokens 0.558 / 0.783 / 0.862 -> 0.503 / 0.672 /
    // 0.817; at 64 rows per expert, 512 tokens, it was 15 % slower)
    if (env_group == 0 && grouped && epi != EPI_STORE && a.E >= 32 && a.rows_limit <= 32 * int64_t(a.E))
        group = 0;
    if (group < 1 || group > a.m_tiles) group = a.m_tiles;
    a.group_m = group;
    if (a.k_splits <= 1) {
        a.k_splits = 1;
        a.k_split_len = a.K;
        a.c_split_stride = 0;
    }
    if (a.resid != nullptr && (grouped || a.k_splits > 1))
        throw Unsupported("a residual needs a dense GEMM without K splits");
    if (!grouped) {
        if (epi != EPI_BIAS) throw Unsupported("dense GEMM epilogue");
        switch (a.tile) {
            case 0:
                if (nn) launch_cfg<DenseCfg, MOE_DENSE_SCHED, true, false, 1, EPI_BIAS>(a, vec, s);
                else launch_cfg<DenseCfg, MOE_DENSE_SCHED, false, false, 1, EPI_BIAS>(a, vec, s);
                break;
            case 1:
                if (nn) launch_dense<DenseMidCfg, true>(a, vec, s);
                else launch_dense<DenseMidCfg, false>(a, vec, s);
                break;
            case 2:
                if (nn) launch_dense<DenseSmallCfg, true>(a, vec, s);
                else launch_dense<DenseSmallCfg, false>(a, vec, s);
                break;
            case kDenseKwTile:
                if (nn) launch_dense<DenseKwCfg, true>(a, vec, s);
                else launch_dense<DenseKwCfg, false>(a, vec, s);
                break;
            case 3:
                if (nn)
                    launch_cfg<DenseTallCfg, MOE_DENSE_TALL_SCHED | SCHED_DIRECT, true, false, 1, EPI_BIAS>(
                        a, vec, s);
                else
                    launch_cfg<DenseTallCfg, MOE_DENSE_TALL_SCHED | SCHED_DIRECT, false, false, 1, EPI_BIAS>(
                        a, vec, s);
                break;
            case kSkinnyTile:
                // the planner checked M <= 64, K % 16 == 0 (per split), aligned rows
                if (a.M > 64 || a.K % 16 != 0 || a.k_split_len % 16 != 0 || !vec ||
                    (nn && a.N % 4 != 0))
                    throw Unsupported("skinny GEMM shape");
                if (nn) launch_skinny<true>(a, s);
                else launch_skinny<false>(a, s);
                break;
            default: throw Unsupported("dense GEMM tile shape");
        }
        return;
    }
    if (nn) throw Unsupported("grouped NN GEMM");
    if (a.tile == kGroupedSkinnyTile) {
        // the planner took it for few rows per expert; it checked the shape
        const int64_t splits = std::max<int64_t>(a.k_splits, 1);
        if (!vec || a.K % 16 != 0 || a.sk_grid > 0 ||
            (splits > 1 && a.k_split_len % 16 != 0) ||
            a.E * ceil_div(a.rows_limit, 16) > 65535 || ceil_div(a.N, 64) > INT32_MAX)
            throw Unsupported("grouped skinny GEMM shape");
        const bool act_split = splits > 1 && epi != EPI_STORE;
        if (act_split && a.sk_part == nullptr) throw Unsupported("grouped skinny split partials");
        GemmArgs g = a;
        g.k_splits = static_cast<int32_t>(splits);
        if (splits == 1) g.k_split_len = a.K;
        // 16 rows per workgroup while the experts average at most 16 rows, else 32
        if (a.rows_limit <= 16 * int64_t(a.E)) launch_skinny_grouped_mb<1>(g, epi, s);
        else launch_skinny_grouped_mb<2>(g, epi, s);
        if (act_split) {
            const int64_t total = a.rows_limit * a.N;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 4096));
            const int sp = static_cast<int>(splits);
            if (epi == EPI_SWIGLU)
                hipLaunchKernelGGL((skinny_act_fixup_kernel<2, EPI_SWIGLU>), dim3(blocks), dim3(256), 0,
                                   s, a.sk_part, a.C, a.rows_limit, a.N, a.ldc, sp);
            else
                hipLaunchKernelGGL((skinny_act_fixup_kernel<1, EPI_SILU>), dim3(blocks), dim3(256), 0,
                                   s, a.sk_part, a.C, a.rows_limit, a.N, a.ldc, sp);
        }
        return;
    }
    if (a.sk_grid > 0) {
        // stream-K: the host checked the direct path's requirements
        if (a.k_splits != 1 || a.sk_part == nullptr) throw Unsupported("stream-K arguments");
        switch (epi) {
            case EPI_SWIGLU:
                if (a.tile == 1) launch_sk<W13TallCfg, MOE_W13_SCHED | SCHED_DIRECT, 2, EPI_SWIGLU>(a, vec, s);
                else launch_sk<W13Cfg, MOE_W13_SCHED | SCHED_DIRECT, 2, EPI_SWIGLU>(a, vec, s);
                break;
            case EPI_SILU:
                if (a.tile == 1) launch_sk<W13TallCfg, MOE_W13_SCHED | SCHED_DIRECT, 1, EPI_SILU>(a, vec, s);
                else launch_sk<W13Cfg, MOE_W13_SCHED | SCHED_DIRECT, 1, EPI_SILU>(a, vec, s);
                break;
            case EPI_STORE:
                if (a.tile == 1) launch_sk<W2NarrowCfg, MOE_W2_SCHED | SCHED_DIRECT, 1, EPI_STORE>(a, vec, s);
                else launch_sk<W2Cfg, MOE_W2_SCHED | SCHED_DIRECT, 1, EPI_STORE>(a, vec, s);
                break;
            default: throw Unsupported("grouped GEMM epilogue");
        }
        return;
    }
    switch (epi) {
        case EPI_SWIGLU:
            if (a.tile == 1)
                launch_cfg<W13TallCfg, MOE_W13_SCHED, false, true, 2, EPI_SWIGLU>(a, vec, s);
            else
                launch_cfg<W13Cfg, MOE_W13_SCHED, false, true, 2, EPI_SWIGLU>(a, vec, s);
            break;
        case EPI_SILU:
            if (a.tile == 1)
                launch_cfg<W13TallCfg, MOE_W13_SCHED, false, true, 1, EPI_SILU>(a, vec, s);
            else
                launch_cfg<W13Cfg, MOE_W13_SCHED, false, true, 1, EPI_SILU>(a, vec, s);
            break;
        case EPI_STORE:
            if (a.tile == 1)
                launch_cfg<W2NarrowCfg, MOE_W2_SCHED | SCHED_DIRECT, false, true, 1, EPI_STORE>(
                    a, vec, s);
            else
                launch_cfg<W2Cfg, MOE_W2_SCHED, false, true, 1, EPI_STORE>(a, vec, s);
            break;
        default: throw Unsupported("grouped GEMM epilogue");
    }
}

}  // namespace moe
