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
// Workgroup: 256 threads = 4 wave64s in a 2x2 arrangement, 128x128 output
// tile, each wave a 64x64 quadrant held as 2x2 MFMA blocks of 32x32 in
// accumulator registers.  K advances 16 at a time through double-buffered
// LDS tiles ([rows][16+4] floats: the 4-float pad makes the 16-byte fragment
// reads and writes bank-conflict free), with the next tile's global loads in
// flight while the matrix cores work on the current one: one barrier per
// K step.
//
// Within a 16-wide K step, lane half h (lanes 32h..32h+31) feeds K columns
// 8h..8h+7, so each lane fetches its A and B fragments for 4 MFMAs with one
// 16-byte LDS read; both operands use the same column order, so every
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

namespace moe {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = kGemmBM;
constexpr int BN = kGemmBN;
constexpr int BK = kGemmBK;
constexpr int LDS = BK + 4;

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

// The reference's SiLU: x / (1 + float(exp(double(-x)))) (src/tensor.cu:
// 132-134,169-173); exp in double, one rounding to float.
__device__ __forceinline__ float silu_ref(float g) {
    const float e = static_cast<float>(exp(-static_cast<double>(g)));
    return g / (1.0f + e);
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

template <bool NN, bool VEC, bool GROUPED, int NB, int EPI>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_kernel(const GemmArgs p) {
    __shared__ __align__(16) float As[2][BM * LDS];
    __shared__ __align__(16) float Bs[2][NB][BN * LDS];

    const int tid = threadIdx.x;
    int mt, nt;
    tile_of(xcd_remap(blockIdx.x, gridDim.x), p.m_tiles, p.n_tiles, p.group_m, mt, nt);

    // ---- which rows / which expert this workgroup owns
    int64_t row0;
    int rows;
    const float* B[NB];
    if (GROUPED) {
        if (mt >= p.tile_start[p.E]) return;  // surplus tile of the worst-case grid
        int lo = 0, hi = p.E;                 // last expert whose first tile <= mt
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (p.tile_start[mid] <= mt) lo = mid; else hi = mid;
        }
        int64_t e_end = p.offsets[lo + 1];
        e_end = e_end < p.rows_limit ? e_end : p.rows_limit;
        row0 = p.offsets[lo] + static_cast<int64_t>(mt - p.tile_start[lo]) * BM;
        if (row0 < 0 || row0 >= e_end) return;  // only reachable with inconsistent offsets
        rows = static_cast<int>(e_end - row0 < BM ? e_end - row0 : BM);
        B[0] = p.B0 + lo * p.b_expert_stride;
        if (NB == 2) B[NB - 1] = p.B1 + lo * p.b_expert_stride;
    } else {
        row0 = static_cast<int64_t>(mt) * BM;
        rows = static_cast<int>(p.M - row0 < BM ? p.M - row0 : BM);
        B[0] = p.B0;
        if (NB == 2) B[NB - 1] = p.B1;
    }
    const int64_t n0 = static_cast<int64_t>(nt) * BN;
    const int64_t N = p.N, K = p.K;

    // ---- global -> register staging assignment
    // A (always [rows, K]): thread covers rows lrow and lrow + 64, 4 columns.
    const int lrow = tid >> 2;
    const int lk = (tid & 3) * 4;
    const float* arow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int r = lrow + 64 * i;
        r = r < rows ? r : rows - 1;  // rows past the edge: any valid row, masked at the store
        int64_t src = row0 + r;
        if (GROUPED && p.gather != nullptr) {
            int64_t tok = p.gather[row0 + r];
            tok = tok < 0 ? 0 : (tok >= p.gather_rows ? p.gather_rows - 1 : tok);
            src = tok;
        }
        arow[i] = p.A + src * p.lda;
    }
    // B, NT ([N, K]): like A.  NN ([K, N]): thread owns one column and 8 of
    // the 16 k rows (kq..kq+3 and 8+kq..8+kq+3), transposed into LDS.
    const float* bptr[NB][2];
    const int ncol = tid & (BN - 1);
    const int kq = (tid >> 7) * 4;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (!NN) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                int64_t n = n0 + lrow + 64 * i;
                n = n < N ? n : N - 1;
                bptr[nb][i] = B[nb] + n * p.ldb;
            }
        } else {
            int64_t n = n0 + ncol;
            n = n < N ? n : N - 1;
            bptr[nb][0] = B[nb] + n;
            bptr[nb][1] = B[nb] + n;
        }
    }

    f32x4 ra[2], rb[NB][2];
    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) ra[i] = load_k4<VEC>(arow[i], k0 + lk, K);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (!NN) {
#pragma unroll
                for (int i = 0; i < 2; ++i) rb[nb][i] = load_k4<VEC>(bptr[nb][i], k0 + lk, K);
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int64_t k = k0 + 8 * h + kq + j;
                        rb[nb][h][j] = k < K ? bptr[nb][h][k * p.ldb] : 0.0f;
                    }
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<f32x4*>(&As[buf][(lrow + 64 * i) * LDS + lk]) = ra[i];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (!NN) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    *reinterpret_cast<f32x4*>(&Bs[buf][nb][(lrow + 64 * i) * LDS + lk]) = rb[nb][i];
            } else {
                *reinterpret_cast<f32x4*>(&Bs[buf][nb][ncol * LDS + kq]) = rb[nb][0];
                *reinterpret_cast<f32x4*>(&Bs[buf][nb][ncol * LDS + 8 + kq]) = rb[nb][1];
            }
        }
    };

    // ---- matrix-core main loop
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int lr = lane & 31, lh = lane >> 5;

    f32x16 acc[NB][2][2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int bj = 0; bj < 2; ++bj)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[nb][bi][bj][r] = 0.0f;

    auto compute = [&](int buf) {
        f32x4 a[2][2], b[NB][2][2];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            const float* src = &As[buf][(wm * 64 + bi * 32 + lr) * LDS + 8 * lh];
            a[bi][0] = *reinterpret_cast<const f32x4*>(src);
            a[bi][1] = *reinterpret_cast<const f32x4*>(src + 4);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
                const float* src = &Bs[buf][nb][(wn * 64 + bj * 32 + lr) * LDS + 8 * lh];
                b[nb][bj][0] = *reinterpret_cast<const f32x4*>(src);
                b[nb][bj][1] = *reinterpret_cast<const f32x4*>(src + 4);
            }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                        for (int bj = 0; bj < 2; ++bj)
                            acc[nb][bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                a[bi][q][s], b[nb][bj][q][s], acc[nb][bi][bj], 0, 0, 0);
    };

    const int64_t nk = (K + BK - 1) / BK;
    if (nk > 0) {
        gload(0);
        lstore(0);
        __syncthreads();
        for (int64_t kt = 0; kt < nk; ++kt) {
            const int cur = static_cast<int>(kt & 1);
            if (kt + 1 < nk) gload((kt + 1) * BK);
            compute(cur);
            if (kt + 1 < nk) lstore(cur ^ 1);
            __syncthreads();
        }
    }

    // ---- epilogue.  32x32 accumulator layout: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32 of its block.
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = wm * 64 + bi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                const int64_t n = n0 + wn * 64 + bj * 32 + lr;
                if (i < rows && n < N) {
                    float v = acc[0][bi][bj][r];
                    if (EPI == EPI_BIAS) {
                        if (p.bias != nullptr) v = v + p.bias[n];
                    } else if (EPI == EPI_SILU) {
                        v = silu_ref(v);
                    } else if (EPI == EPI_SWIGLU) {
                        v = silu_ref(v) * acc[NB - 1][bi][bj][r];
                    }
                    p.C[(row0 + i) * p.ldc + n] = v;
                }
            }
}

template <bool NN, bool GROUPED, int NB, int EPI>
void launch_vec(const GemmArgs& a, bool vec, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(a.m_tiles) * static_cast<unsigned>(a.n_tiles));
    if (vec)
        hipLaunchKernelGGL((gemm_kernel<NN, true, GROUPED, NB, EPI>), grid,
                           dim3(kGemmThreads), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_kernel<NN, false, GROUPED, NB, EPI>), grid,
                           dim3(kGemmThreads), 0, s, a);
}

}  // namespace

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
    int group = env_group != 0 ? env_group : kGemmGroupM;
    if (group < 1 || group > a.m_tiles) group = a.m_tiles;
    a.group_m = group;
    if (!grouped) {
        if (epi != EPI_BIAS) throw Unsupported("dense GEMM epilogue");
        if (nn) launch_vec<true, false, 1, EPI_BIAS>(a, vec, s);
        else launch_vec<false, false, 1, EPI_BIAS>(a, vec, s);
        return;
    }
    if (nn) throw Unsupported("grouped NN GEMM");
    switch (epi) {
        case EPI_SWIGLU: launch_vec<false, true, 2, EPI_SWIGLU>(a, vec, s); break;
        case EPI_SILU: launch_vec<false, true, 1, EPI_SILU>(a, vec, s); break;
        case EPI_STORE: launch_vec<false, true, 1, EPI_STORE>(a, vec, s); break;
        default: throw Unsupported("grouped GEMM epilogue");
    }
}

}  // namespace moe
