// Routing on gfx950: router gate logits, top-k selection, the stable bucket
// sort of (token, slot) pairs by expert, and the gate-weighted combine.
//
// All of it is integer or HBM-bound work.  Bit-exactness with the CPU path
// is the contract here: logits keep one k-ascending fp32 accumulator per
// output (the reference's matmul_transposed loop, src/tensor.cu:136-148),
// the routers replay the reference's comparisons in the same order, and the
// permutation is a stable sort, so indices, offsets and packed order are
// bit-identical to the CPU path.  Floating-point contraction is explicit:
// this file is compiled with -ffp-contract=off and fuses only where
// __builtin_fmaf is written.
#include "common.hpp"

#include <climits>
#include <cmath>

namespace moe {
namespace {

// ---------------------------------------------------------------- gate
// Workgroup: 32 token rows x a chunk of up to 64 experts.  Thread (r, g)
// owns row r and experts g, g+8, ..., g+56 of the chunk: up to 8 independent
// accumulator chains.  K streams through LDS 64 columns at a time with
// coalesced loads; x rows are read once per expert chunk.
constexpr int GATE_ROWS = 32;
constexpr int GATE_EXPERTS = 64;
constexpr int GATE_KC = 64;

template <int CONTRACT>
__device__ __forceinline__ float mac(float acc, float a, float b) {
    if (CONTRACT) return __builtin_fmaf(a, b, acc);
    const float prod = a * b;
    return acc + prod;
}

template <int CONTRACT>
__global__ __launch_bounds__(256) void gate_logits_kernel(
        const float* __restrict__ x, const float* __restrict__ w,
        float* __restrict__ logits, int64_t T, int64_t d, int64_t E) {
    __shared__ float xs[GATE_ROWS][GATE_KC + 1];
    __shared__ float ws[GATE_EXPERTS][GATE_KC + 1];
    const int tid = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * GATE_ROWS;
    const int64_t e0 = static_cast<int64_t>(blockIdx.y) * GATE_EXPERTS;
    const int r = tid & (GATE_ROWS - 1);
    const int g = tid >> 5;  // 0..7
    float acc[GATE_EXPERTS / 8];
#pragma unroll
    for (int j = 0; j < GATE_EXPERTS / 8; ++j) acc[j] = 0.0f;

    for (int64_t k0 = 0; k0 < d; k0 += GATE_KC) {
        const int kn = static_cast<int>(d - k0 < GATE_KC ? d - k0 : GATE_KC);
        // stage x[t0.., k0..] and w[e0.., k0..]: 64 consecutive floats per row
#pragma unroll
        for (int i = 0; i < GATE_ROWS * GATE_KC / 256; ++i) {
            const int idx = tid + 256 * i;
            const int rr = idx / GATE_KC, cc = idx % GATE_KC;
            const int64_t t = t0 + rr;
            xs[rr][cc] = (t < T && cc < kn) ? x[t * d + k0 + cc] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < GATE_EXPERTS * GATE_KC / 256; ++i) {
            const int idx = tid + 256 * i;
            const int ee = idx / GATE_KC, cc = idx % GATE_KC;
            const int64_t e = e0 + ee;
            ws[ee][cc] = (e < E && cc < kn) ? w[e * d + k0 + cc] : 0.0f;
        }
        __syncthreads();
        // Only the kn real columns are accumulated: no padding term ever
        // enters a sum, so the chain is exactly the CPU's.
        for (int kk = 0; kk < kn; ++kk) {
            const float xv = xs[r][kk];
#pragma unroll
            for (int j = 0; j < GATE_EXPERTS / 8; ++j)
                acc[j] = mac<CONTRACT>(acc[j], xv, ws[g + 8 * j][kk]);
        }
        __syncthreads();
    }
    const int64_t t = t0 + r;
    if (t < T) {
#pragma unroll
        for (int j = 0; j < GATE_EXPERTS / 8; ++j) {
            const int64_t e = e0 + g + 8 * j;
            if (e < E) logits[t * E + e] = acc[j];
        }
    }
}

// -------------------------------------------------------------- routers
// PhiMoE::route score canonicalisation (src/layer.cu:50-55).
__device__ __forceinline__ float quantise(float score, float quantum) {
    if (!(quantum > 0.0f)) return score;
    const float rounded = floorf(fabsf(score) / quantum + 0.5f) * quantum;
    return score < 0.0f ? -rounded : rounded;
}

// PHI_QUANT: one thread per token replays the reference's sequential select
// (src/layer.cu:56-69): ascending scan, take e when nothing is held or when
// it beats the held score by more than tie_eps; repeat excluding the picks.
// The rule is order-dependent (not a reduction), so it stays sequential.
__global__ __launch_bounds__(256) void route_phi_kernel(
        const float* __restrict__ logits, const float* __restrict__ bias,
        int64_t T, int64_t E, int64_t k, float quantum, float tie_eps,
        int32_t* __restrict__ idx, float* __restrict__ w) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const float* row = logits + t * E;
    const float weight = 1.0f / static_cast<float>(k);
    int32_t picks[kMaxTopK];
    for (int s = 0; s < k; ++s) {
        int best = -1;
        float best_value = -INFINITY;
        for (int e = 0; e < E; ++e) {
            bool taken = false;
            for (int c = 0; c < s; ++c) taken |= (picks[c] == e);
            if (taken) continue;
            const float raw = bias != nullptr ? row[e] + bias[e] : row[e];
            const float v = quantise(raw, quantum);
            if (best < 0 || v > best_value + tie_eps) {
                best = e;
                best_value = v;
            }
        }
        picks[s] = best;
        idx[t * k + s] = best;
        w[t * k + s] = weight;
    }
}

// SOFTMAX_TOPK: a group of G lanes (a power of two, <= 64) per token; lane j
// holds experts j, j+G, ...  Each of the k rounds takes every lane's best
// unpicked expert and reduces over the group with xor-shuffles under the
// total order (value descending, index ascending), NaN ranking as -inf.
// The group's first lane then forms the weights in double, as the oracle.
__device__ __forceinline__ bool beats(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

__global__ __launch_bounds__(256) void route_softmax_kernel(
        const float* __restrict__ logits, const float* __restrict__ bias,
        int64_t T, int64_t E, int64_t k, int G,
        int32_t* __restrict__ idx, float* __restrict__ w) {
    const int lane = threadIdx.x & 63;
    const int sub = lane & (G - 1);
    const int64_t t = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / G;
    const bool live = t < T;
    const float* row = logits + (live ? t : 0) * E;
    // experts of this lane: sub + G*j, j < per_lane (<= kMaxExperts / G)
    const int per_lane = static_cast<int>((E + G - 1) / G);
    uint32_t picked = 0;  // bit j: expert sub + G*j already selected (per_lane <= 32)
    double top = 0.0;
    double sum = 0.0;
    for (int s = 0; s < k; ++s) {
        float bv = -INFINITY;
        int bi = INT_MAX;
        if (live) {
            for (int j = 0; j < per_lane; ++j) {
                const int e = sub + G * j;
                if (e >= E || ((picked >> j) & 1u)) continue;
                float v = bias != nullptr ? row[e] + bias[e] : row[e];
                if (isnan(v)) v = -INFINITY;
                if (beats(v, e, bv, bi)) { bv = v; bi = e; }
            }
        }
        for (int off = G >> 1; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, G);
            const int oi = __shfl_xor(bi, off, G);
            if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (live && bi != INT_MAX && (bi % G) == sub) picked |= 1u << (bi / G);
        if (live && sub == 0) {
            idx[t * k + s] = bi;
            if (s == 0) top = static_cast<double>(bv);
            sum += exp(static_cast<double>(bv) - top);
            w[t * k + s] = bv;  // the selected value, turned into a weight below
        }
    }
    if (live && sub == 0) {
        for (int s = 0; s < k; ++s) {
            const double ex = exp(static_cast<double>(w[t * k + s]) - top);
            w[t * k + s] = static_cast<float>(ex / sum);
        }
    }
}

// ---------------------------------------------------------- permutation
// Stable bucket sort in three passes over blocks of kPermTokens tokens.
// A block records which of its tokens chose expert e as a 256-bit mask per
// expert in LDS (atomicOr: order-free), so a pair's rank inside its block is
// a popcount of the bits below it -- ascending token order, as the
// reference's assignments[e] (src/layer.cu:86-92), without any
// order-dependent atomics.
__device__ void build_masks(const int32_t* __restrict__ idx, int64_t T,
                            int64_t k, int64_t E, int64_t tb,
                            unsigned long long* masks) {
    const int tid = threadIdx.x;
    for (int i = tid; i < E * 4; i += blockDim.x) masks[i] = 0ull;
    __syncthreads();
    const int64_t t = tb + tid;
    if (tid < kPermTokens && t < T) {
        for (int s = 0; s < k; ++s) {
            const int e = idx[t * k + s];
            if (e >= 0 && e < E)
                atomicOr(&masks[e * 4 + (tid >> 6)], 1ull << (tid & 63));
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void perm_count_kernel(
        const int32_t* __restrict__ idx, int64_t T, int64_t k, int64_t E,
        int32_t* __restrict__ counts) {
    __shared__ unsigned long long masks[kMaxExperts * 4];
    const int64_t b = blockIdx.x, nb = gridDim.x;
    build_masks(idx, T, k, E, b * kPermTokens, masks);
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        const int c = __popcll(masks[e * 4]) + __popcll(masks[e * 4 + 1]) +
                      __popcll(masks[e * 4 + 2]) + __popcll(masks[e * 4 + 3]);
        counts[e * nb + b] = c;  // expert-major: the scan below is a plain scan
    }
}

// Exclusive scan of counts[E * nb] in place (one workgroup of 1024 threads),
// then the per-expert offsets and the per-expert first GEMM m-tile.
__global__ __launch_bounds__(1024) void perm_scan_kernel(
        int32_t* __restrict__ counts, int64_t nb, int64_t E,
        int32_t* __restrict__ offsets, int32_t* __restrict__ tile_start) {
    __shared__ int32_t wave_sums[16];
    __shared__ int32_t carry;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid == 0) carry = 0;
    __syncthreads();
    const int64_t n = E * nb;
    for (int64_t base = 0; base < n; base += 1024) {
        const int64_t i = base + tid;
        const int32_t v = i < n ? counts[i] : 0;
        int32_t incl = v;  // inclusive scan within the wave
        for (int off = 1; off < 64; off <<= 1) {
            const int32_t o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        if (lane == 63) wave_sums[wv] = incl;
        __syncthreads();
        int32_t before = carry;
        for (int j = 0; j < wv; ++j) before += wave_sums[j];
        if (i < n) counts[i] = before + incl - v;
        __syncthreads();
        if (tid == 1023) carry = before + incl;
        __syncthreads();
    }
    // offsets[e] = base of (e, block 0); offsets[E] = total pairs
    for (int64_t e = tid; e < E; e += 1024) offsets[e] = nb > 0 ? counts[e * nb] : 0;
    if (tid == 0) offsets[E] = carry;
    __syncthreads();
    if (tile_start != nullptr && tid == 0) {
        int32_t acc = 0;
        for (int64_t e = 0; e < E; ++e) {
            tile_start[e] = acc;
            acc += (offsets[e + 1] - offsets[e] + kGemmBM - 1) / kGemmBM;
        }
        tile_start[E] = acc;
    }
}

__global__ __launch_bounds__(256) void perm_place_kernel(
        const int32_t* __restrict__ idx, int64_t T, int64_t k, int64_t E,
        const int32_t* __restrict__ base, int32_t* __restrict__ perm,
        int32_t* __restrict__ inv) {
    __shared__ unsigned long long masks[kMaxExperts * 4];
    const int64_t b = blockIdx.x, nb = gridDim.x;
    const int tid = threadIdx.x;
    build_masks(idx, T, k, E, b * kPermTokens, masks);
    const int64_t t = b * kPermTokens + tid;
    if (tid < kPermTokens && t < T) {
        const int word = tid >> 6;
        const unsigned long long below = (1ull << (tid & 63)) - 1ull;
        for (int s = 0; s < k; ++s) {
            const int e = idx[t * k + s];
            if (e < 0 || e >= E) { inv[t * k + s] = -1; continue; }
            int rank = __popcll(masks[e * 4 + word] & below);
            for (int q = 0; q < word; ++q) rank += __popcll(masks[e * 4 + q]);
            const int32_t pos = base[e * nb + b] + rank;
            perm[pos] = static_cast<int32_t>(t);
            inv[t * k + s] = pos;
        }
    }
}

// First GEMM m-tile of each expert from the offsets (for callers that
// bring their own offsets to the grouped FFN).
__global__ void tile_start_kernel(const int32_t* __restrict__ offsets, int64_t E,
                                  int32_t* __restrict__ tile_start) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int32_t acc = 0;
    for (int64_t e = 0; e < E; ++e) {
        tile_start[e] = acc;
        acc += (offsets[e + 1] - offsets[e] + kGemmBM - 1) / kGemmBM;
    }
    tile_start[E] = acc;
}

// -------------------------------------------------------------- combine
// One workgroup per token.  The token's slots are ordered by ascending
// expert (ties by slot), then y = 0 + w*row, + w*row, ... in that order: the
// order of the reference's expert loop (src/layer.cu:93-101).  resid, when
// given, is added last (the decoder's add_inplace, src/layer.cu:160).
template <int CONTRACT>
__global__ __launch_bounds__(256) void combine_kernel(
        const float* __restrict__ out_rows, const int32_t* __restrict__ idx,
        const float* __restrict__ wts, const int32_t* __restrict__ inv,
        const float* __restrict__ resid, float* __restrict__ y, int64_t T,
        int64_t k, int64_t d, int64_t rows_total) {
    __shared__ int32_t order_row[kMaxTopK];
    __shared__ float order_w[kMaxTopK];
    __shared__ int n_live;
    const int64_t t = blockIdx.x;
    if (threadIdx.x == 0) {
        int prev_e = -1, prev_s = -1, n = 0;
        for (int q = 0; q < k; ++q) {
            int best_e = INT_MAX, best_s = INT_MAX;
            for (int s = 0; s < k; ++s) {
                const int e = idx[t * k + s];
                const bool after = e > prev_e || (e == prev_e && s > prev_s);
                if (after && (e < best_e || (e == best_e && s < best_s))) {
                    best_e = e;
                    best_s = s;
                }
            }
            prev_e = best_e;
            prev_s = best_s;
            const int32_t r = inv[t * k + best_s];
            if (r >= 0 && r < rows_total) {
                order_row[n] = r;
                order_w[n] = wts[t * k + best_s];
                ++n;
            }
        }
        n_live = n;
    }
    __syncthreads();
    const int n = n_live;
    const bool vec = (d & 3) == 0;
    if (vec) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const int64_t d4 = d >> 2;
        for (int64_t j = threadIdx.x; j < d4; j += blockDim.x) {
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            for (int q = 0; q < n; ++q) {
                const f4 v = reinterpret_cast<const f4*>(out_rows + order_row[q] * d)[j];
                const float wq = order_w[q];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[c] = mac<CONTRACT>(acc[c], wq, v[c]);
            }
            if (resid != nullptr) {
                const f4 rv = reinterpret_cast<const f4*>(resid + t * d)[j];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[c] = acc[c] + rv[c];
            }
            reinterpret_cast<f4*>(y + t * d)[j] = acc;
        }
    } else {
        for (int64_t j = threadIdx.x; j < d; j += blockDim.x) {
            float acc = 0.0f;
            for (int q = 0; q < n; ++q)
                acc = mac<CONTRACT>(acc, order_w[q], out_rows[order_row[q] * d + j]);
            if (resid != nullptr) acc = acc + resid[t * d + j];
            y[t * d + j] = acc;
        }
    }
}

}  // namespace

void launch_gate_logits(const float* x, const float* w, float* logits,
                        int64_t T, int64_t d, int64_t E, int contract,
                        hipStream_t s) {
    if (T == 0 || E == 0) return;
    const dim3 grid(static_cast<unsigned>(ceil_div(T, GATE_ROWS)),
                    static_cast<unsigned>(ceil_div(E, GATE_EXPERTS)));
    if (contract)
        hipLaunchKernelGGL(gate_logits_kernel<1>, grid, dim3(256), 0, s, x, w, logits, T, d, E);
    else
        hipLaunchKernelGGL(gate_logits_kernel<0>, grid, dim3(256), 0, s, x, w, logits, T, d, E);
}

void launch_route(const float* logits, const float* bias, int64_t T, int64_t E,
                  int64_t k, int mode, float quantum, float tie_eps,
                  int32_t* idx, float* w, hipStream_t s) {
    if (T == 0) return;
    if (mode == MOE_ROUTER_PHI_QUANT) {
        hipLaunchKernelGGL(route_phi_kernel, dim3(static_cast<unsigned>(ceil_div(T, 256))),
                           dim3(256), 0, s, logits, bias, T, E, k, quantum, tie_eps, idx, w);
        return;
    }
    int G = 1;
    while (G < E && G < 64) G <<= 1;
    const int64_t threads = T * G;
    hipLaunchKernelGGL(route_softmax_kernel, dim3(static_cast<unsigned>(ceil_div(threads, 256))),
                       dim3(256), 0, s, logits, bias, T, E, k, G, idx, w);
}

void launch_perm_count(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                       int32_t* counts, hipStream_t s) {
    const int64_t nb = ceil_div(T, kPermTokens);
    if (nb == 0) return;
    hipLaunchKernelGGL(perm_count_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s,
                       idx, T, k, E, counts);
}

void launch_perm_scan(int32_t* counts, int64_t nblocks, int64_t E,
                      int32_t* offsets, int32_t* tile_start, hipStream_t s) {
    hipLaunchKernelGGL(perm_scan_kernel, dim3(1), dim3(1024), 0, s, counts, nblocks, E,
                       offsets, tile_start);
}

void launch_perm_place(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                       const int32_t* base, int32_t* perm, int32_t* inv,
                       hipStream_t s) {
    const int64_t nb = ceil_div(T, kPermTokens);
    if (nb == 0) return;
    hipLaunchKernelGGL(perm_place_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s,
                       idx, T, k, E, base, perm, inv);
}

void launch_tile_start(const int32_t* offsets, int64_t E, int32_t* tile_start,
                       hipStream_t s) {
    hipLaunchKernelGGL(tile_start_kernel, dim3(1), dim3(64), 0, s, offsets, E, tile_start);
}

void launch_combine(const float* out_rows, const int32_t* idx, const float* w,
                    const int32_t* inv, const float* resid, float* y,
                    int64_t T, int64_t k, int64_t d, int64_t rows_total,
                    int contract, hipStream_t s) {
    if (T == 0 || d == 0) return;
    if (contract)
        hipLaunchKernelGGL(combine_kernel<1>, dim3(static_cast<unsigned>(T)), dim3(256), 0, s,
                           out_rows, idx, w, inv, resid, y, T, k, d, rows_total);
    else
        hipLaunchKernelGGL(combine_kernel<0>, dim3(static_cast<unsigned>(T)), dim3(256), 0, s,
                           out_rows, idx, w, inv, resid, y, T, k, d, rows_total);
}

}  // namespace moe
