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
// The gate is a row-times-[E, d] product whose every output must be the
// CPU's sequential k-ascending chain, so its parallelism is the T*E outputs:
// one thread per output, or per TB outputs of one expert (TB tokens' chains
// advanced together: the expert's 16-byte LDS read then feeds TB tokens, the
// cut in LDS traffic that large E needs -- at E = 64 one read per output made
// the kernel LDS-bound).  A workgroup covers R = TB * 256/EB token rows x EB
// experts (EB = E rounded up to a power of two, 8..64); in a wave the lanes
// sharing a row read the same LDS word (a broadcast).  K streams through a
// double-buffered LDS tile of R + EB rows x 64 columns; the next chunk's
// coalesced global loads are in flight while the current one is consumed, 4
// columns per 16-byte LDS read.
constexpr int GATE_KC = 64;
constexpr int GATE_LDS = GATE_KC + 4;  // 16-byte aligned, conflict-free rows

template <int CONTRACT>
__device__ __forceinline__ float mac(float acc, float a, float b) {
    if (CONTRACT) return __builtin_fmaf(a, b, acc);
    const float prod = a * b;
    return acc + prod;
}

template <int CONTRACT, int EB, int TB>
__global__ __launch_bounds__(256) void gate_logits_kernel(
        const float* __restrict__ x, const float* __restrict__ w,
        float* __restrict__ logits, int64_t T, int64_t d, int64_t E) {
    constexpr int R = TB * (256 / EB);        // token rows per workgroup
    constexpr int ROWS = R + EB;              // staged rows: x rows, then w rows
    constexpr int PER = ROWS * GATE_KC / 256; // staged floats per thread
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float tile[2][ROWS * GATE_LDS];

    const int tid = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * R;
    const int64_t e0 = static_cast<int64_t>(blockIdx.y) * EB;
    const int el = tid % EB, r = tid / EB;

    // Staging: element i*256 + tid of the tile -> (row, col); 64 lanes of a
    // wave read 64 consecutive floats of one row (256 contiguous bytes).
    const float* src[PER];
    bool ok[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = i * 256 + tid;
        const int row = idx / GATE_KC, col = idx % GATE_KC;
        if (row < R) {
            const int64_t t = t0 + row;
            ok[i] = t < T;
            src[i] = x + (ok[i] ? t : 0) * d + col;
        } else {
            const int64_t e = e0 + (row - R);
            ok[i] = e < E;
            src[i] = w + (ok[i] ? e : 0) * d + col;
        }
    }
    float stage[PER];
    auto gload = [&](int64_t k0) {
        const int64_t kn = d - k0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int col = (i * 256 + tid) % GATE_KC;
            stage[i] = (ok[i] && col < kn) ? src[i][k0] : 0.0f;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = i * 256 + tid;
            tile[buf][(idx / GATE_KC) * GATE_LDS + idx % GATE_KC] = stage[i];
        }
    };

    float acc[TB];
#pragma unroll
    for (int u = 0; u < TB; ++u) acc[u] = 0.0f;
    const int64_t nchunks = (d + GATE_KC - 1) / GATE_KC;
    if (nchunks > 0) {
        gload(0);
        lstore(0);
        __syncthreads();
    }
    for (int64_t c = 0; c < nchunks; ++c) {
        const int buf = static_cast<int>(c & 1);
        const int64_t k0 = c * GATE_KC;
        if (c + 1 < nchunks) gload(k0 + GATE_KC);
        // Only the kn real columns enter the sum: the chain is exactly the
        // CPU's, with no padding term.
        const int kn = static_cast<int>(d - k0 < GATE_KC ? d - k0 : GATE_KC);
        const float* xr = &tile[buf][r * TB * GATE_LDS];  // this thread's TB rows
        const float* wr = &tile[buf][(R + el) * GATE_LDS];
        int kk = 0;
        for (; kk + 4 <= kn; kk += 4) {
            const f4 wv = *reinterpret_cast<const f4*>(wr + kk);
#pragma unroll
            for (int u = 0; u < TB; ++u) {
                const f4 xv = *reinterpret_cast<const f4*>(xr + u * GATE_LDS + kk);
                acc[u] = mac<CONTRACT>(acc[u], xv[0], wv[0]);
                acc[u] = mac<CONTRACT>(acc[u], xv[1], wv[1]);
                acc[u] = mac<CONTRACT>(acc[u], xv[2], wv[2]);
                acc[u] = mac<CONTRACT>(acc[u], xv[3], wv[3]);
            }
        }
        for (; kk < kn; ++kk)
#pragma unroll
            for (int u = 0; u < TB; ++u) acc[u] = mac<CONTRACT>(acc[u], xr[u * GATE_LDS + kk], wr[kk]);
        if (c + 1 < nchunks) lstore(buf ^ 1);
        __syncthreads();
    }
    const int64_t e = e0 + el;
#pragma unroll
    for (int u = 0; u < TB; ++u) {
        const int64_t t = t0 + r * TB + u;
        if (t < T && e < E) logits[t * E + e] = acc[u];
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
// then the per-expert offsets.
__global__ __launch_bounds__(1024) void perm_scan_kernel(
        int32_t* __restrict__ counts, int64_t nb, int64_t E,
        int32_t* __restrict__ offsets) {
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


// -------------------------------------------------------------- combine
// One workgroup per token.  The token's slots are ordered by ascending
// expert (ties by slot), then y = 0 + w*row, + w*row, ... in that order: the
// order of the reference's expert loop (src/layer.cu:93-101).  resid, when
// given, is added last (the decoder's add_inplace, src/layer.cu:160).  When
// the w2 GEMM ran split-K, a row is the sum of its PARTS partial rows, added
// in part order before weighting.
template <int CONTRACT, int PARTS>
__global__ __launch_bounds__(256) void combine_kernel(
        const float* __restrict__ out_rows, const int32_t* __restrict__ idx,
        const float* __restrict__ wts, const int32_t* __restrict__ inv,
        const float* __restrict__ resid, float* __restrict__ y, int64_t T,
        int64_t k, int64_t d, int64_t rows_total, int64_t part_stride) {
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
                f4 v = reinterpret_cast<const f4*>(out_rows + order_row[q] * d)[j];
#pragma unroll
                for (int p = 1; p < PARTS; ++p) {
                    const f4 u =
                        reinterpret_cast<const f4*>(out_rows + p * part_stride + order_row[q] * d)[j];
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] = v[c] + u[c];
                }
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
            for (int q = 0; q < n; ++q) {
                float v = out_rows[order_row[q] * d + j];
#pragma unroll
                for (int p = 1; p < PARTS; ++p) v = v + out_rows[p * part_stride + order_row[q] * d + j];
                acc = mac<CONTRACT>(acc, order_w[q], v);
            }
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
    int eb = 8;
    while (eb < E && eb < 64) eb <<= 1;
    // 4 tokens per thread from 32 experts up (small E keeps one output per
    // thread: its rows per workgroup are already many, and the grid stays wide)
    const int tb = eb >= 32 ? 4 : 1;
    const dim3 grid(static_cast<unsigned>(ceil_div(T, tb * (256 / eb))),
                    static_cast<unsigned>(ceil_div(E, eb)));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, x, w, logits, T, d, E);
    };
    switch (eb * 2 + (contract ? 1 : 0)) {
        case 16: go(gate_logits_kernel<0, 8, 1>); break;
        case 17: go(gate_logits_kernel<1, 8, 1>); break;
        case 32: go(gate_logits_kernel<0, 16, 1>); break;
        case 33: go(gate_logits_kernel<1, 16, 1>); break;
        case 64: go(gate_logits_kernel<0, 32, 4>); break;
        case 65: go(gate_logits_kernel<1, 32, 4>); break;
        case 128: go(gate_logits_kernel<0, 64, 4>); break;
        default: go(gate_logits_kernel<1, 64, 4>); break;
    }
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
                      int32_t* offsets, hipStream_t s) {
    hipLaunchKernelGGL(perm_scan_kernel, dim3(1), dim3(1024), 0, s, counts, nblocks, E,
                       offsets);
}

void launch_perm_place(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                       const int32_t* base, int32_t* perm, int32_t* inv,
                       hipStream_t s) {
    const int64_t nb = ceil_div(T, kPermTokens);
    if (nb == 0) return;
    hipLaunchKernelGGL(perm_place_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s,
                       idx, T, k, E, base, perm, inv);
}


void launch_combine(const float* out_rows, const int32_t* idx, const float* w,
                    const int32_t* inv, const float* resid, float* y,
                    int64_t T, int64_t k, int64_t d, int64_t rows_total,
                    int contract, int parts, int64_t part_stride, hipStream_t s) {
    if (T == 0 || d == 0) return;
    static_assert(kMaxW2Splits == 4, "combine instantiates 1, 2 and 4 parts");
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(T)), dim3(256), 0, s, out_rows, idx,
                           w, inv, resid, y, T, k, d, rows_total, part_stride);
    };
    if (parts == 4) {
        if (contract) go(combine_kernel<1, 4>); else go(combine_kernel<0, 4>);
    } else if (parts == 2) {
        if (contract) go(combine_kernel<1, 2>); else go(combine_kernel<0, 2>);
    } else if (parts == 1) {
        if (contract) go(combine_kernel<1, 1>); else go(combine_kernel<0, 1>);
    } else {
        throw Unsupported("combine: partial-row count must be 1, 2 or 4");
    }
}

}  // namespace moe
