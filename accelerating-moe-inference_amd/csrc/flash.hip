// Causal attention in one pass per (sequence, head, 128-query tile): the
// scores never leave the chip.
//
// Each wave owns 32 queries.  It computes the transposed scores
// S^T[key][query] = K Q^T on fp32 MFMA (32x32x2), so the accumulator column,
// i.e. the lane, is the query: every per-query quantity of the softmax (the
// running max, the denominator, the rescale) is lane-local, and the two lane
// halves, which hold different keys of the same query, meet through one
// shuffle.  The output is accumulated transposed too, O^T[dim][query] +=
// V^T P^T, with P^T fed to the MFMA straight from the score registers: the
// MFMA only needs the A and B operands to agree on which k each lane half
// supplies, so step j of the P V product takes key 8*(j/4) + 4*half + j%4,
// the key the score accumulator's register j holds, and V is read at that
// key.  No transpose through LDS, no S x S buffer in HBM.
//
// Softmax (PhiAttention::forward, src/layer.cu:118-140): score / sqrt(hd),
// keys ki <= qi within the window, weights exp(s - m); the maximum is carried
// online (rescaling the partial sums by exp(m_old - m_new)), and the output
// divides the weighted sum by the denominator at the end -- the same values
// as the reference's loop up to rounding.  The reference rounds
// float(exp(double(x))); here exp(x) is the single-precision hardware exp2 of
// x * log2(e) (relative error about |x| * 6e-8 + 1 ulp, x <= 0), which the
// online rescaling's different rounding already puts outside bit-exactness:
// the fp64 exp took about half as long as the MFMAs of a key block.  For the
// same reason the division by sqrt(hd) is folded into that multiply.
#include "common.hpp"

#include <cmath>

namespace moe {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kQTile = 128;  // queries per workgroup (4 waves x 32)
constexpr int kKBlock = 32;  // keys per block

// At least two waves per SIMD: at most 256 registers a lane, which keeps
// head_dim 128 at two waves (it took 289 and one wave) and keeps the
// accumulators in VGPRs, where the rescale needs no AGPR moves.
template <int HD>
__global__ __launch_bounds__(256, 2) void flash_attn_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, int64_t S, int64_t H, int64_t KVH, int64_t window, float scale) {
    static_assert(HD % 32 == 0 && HD <= 128, "head_dim 32, 64, 96 or 128");
    constexpr int LD = HD + 8;      // LDS row stride: the lane halves land 32 banks apart
    constexpr int QK = HD / 2;      // MFMA steps of the score product (2 dims each)
    constexpr int MB = HD / 32;     // 32-dim blocks of the output
    // two K/V buffers: block j is staged into buffer j % 2 while the waves
    // read block j - 1 from the other, so one barrier per block suffices
    __shared__ __align__(16) float Ks[2][kKBlock * LD];
    __shared__ __align__(16) float Vs[2][kKBlock * LD];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
    const int lq = lane & 31, half = lane >> 5;
    // Causal work grows with the tile index (tile t walks 4t + 4 key blocks).
    // Workgroups half a grid apart share a CU when the grid fills two per CU
    // (the dispatcher deals ids round-robin over the XCDs and their CUs), so
    // the order is tile-major with heavy and light tiles interleaved -- rank
    // r < T/2 takes tile T-1-r, the rest tile r - T/2 -- and each CU gets a
    // heavy and a light tile (measured: 0.41 -> 0.29 ms per config-5 prefill).
    const int64_t T = gridDim.x, BH = gridDim.y;
    const int64_t L = static_cast<int64_t>(blockIdx.y) * T + blockIdx.x;
    const int64_t rank = L / BH, z = L % BH;
    const int tile = static_cast<int>(rank < (T + 1) / 2 ? T - 1 - rank : rank - (T + 1) / 2);
    const int64_t b = z / H, h = z % H, kh = h / (H / KVH);
    const int64_t qw = H * HD, kw = KVH * HD;
    // key and query indices fit 32 bits (the launcher checks seq_len)
    const int S32 = static_cast<int>(S), W = static_cast<int>(window);
    const int row0 = tile * kQTile;
    const int q0 = row0 + 32 * wave;                  // this wave's first query
    const int qi = q0 + lq;                           // this lane's query
    const bool wave_live = q0 < S32;
    const float* kb = k + b * S * kw + kh * HD;
    const float* vb = v + b * S * kw + kh * HD;

    // Q^T operand: step j, half h supplies dim h*QK + j of this lane's query
    float qr[QK];
    {
        const float* qrow = q + (b * S + (qi < S32 ? qi : S32 - 1)) * qw + h * HD + half * QK;
#pragma unroll
        for (int j = 0; j < QK; j += 4) {
            const f32x4 t = *reinterpret_cast<const f32x4*>(qrow + j);
            qr[j] = t[0];
            qr[j + 1] = t[1];
            qr[j + 2] = t[2];
            qr[j + 3] = t[3];
        }
    }

    // keys this tile can see: [k_lo, k_hi)
    const int k_hi = (row0 + kQTile < S32 ? row0 + kQTile : S32);
    int k_lo = 0;
    if (W > 0 && row0 - (W - 1) > 0) k_lo = ((row0 - (W - 1)) / kKBlock) * kKBlock;

    // block staging: 32 keys x HD floats of K and of V, 16-byte chunks
    constexpr int CHUNKS = kKBlock * HD / 4;       // per matrix
    constexpr int PER_T = (CHUNKS + 255) / 256;
    f32x4 kst[PER_T], vst[PER_T];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int c = tid + 256 * i;
            if (c < CHUNKS) {
                const int r = c / (HD / 4), col = 4 * (c % (HD / 4));
                int key = k0 + r;
                key = key < S32 ? key : S32 - 1;  // past the end: a valid row, masked below
                kst[i] = *reinterpret_cast<const f32x4*>(kb + key * kw + col);
                vst[i] = *reinterpret_cast<const f32x4*>(vb + key * kw + col);
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int c = tid + 256 * i;
            if (c < CHUNKS) {
                const int r = c / (HD / 4), col = 4 * (c % (HD / 4));
                *reinterpret_cast<f32x4*>(&Ks[buf][r * LD + col]) = kst[i];
                *reinterpret_cast<f32x4*>(&Vs[buf][r * LD + col]) = vst[i];
            }
        }
    };

    f32x16 acc[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
    // the running maximum is kept on the unscaled scores: s / scale is
    // monotone in s, so exp(s/scale - m/scale) = exp2((s - m) * c) with
    // c = log2(e) / scale, one multiply per weight instead of a division
    const float c2 = 1.44269504088896340736f / scale;
    float m_run = -INFINITY, den = 0.0f;
    const int wq_last = q0 + 31 < S32 ? q0 + 31 : S32 - 1;  // the wave's last query

    fetch(k_lo);
    stage(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = k_lo; k0 < k_hi; k0 += kKBlock) {
        const bool more = k0 + kKBlock < k_hi;
        if (more) fetch(k0 + kKBlock);
        // the wave skips blocks wholly after its last query or before its
        // first query's window (wave-uniform)
        bool active = wave_live && k0 <= wq_last;
        if (W > 0 && k0 + kKBlock - 1 < q0 - (W - 1)) active = false;
        if (active) {
            // S^T = K Q^T: lane = query, register r = key 8*(r/4) + 4*half + r%4
            f32x16 s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.0f;
            const float* krow = &Ks[buf][lq * LD + half * QK];
#pragma unroll
            for (int j = 0; j < QK; j += 4) {
                const f32x4 kk = *reinterpret_cast<const f32x4*>(krow + j);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[t], qr[j + t], s, 0, 0, 0);
            }
            // every key of the block visible to every query of the wave:
            // no mask (wave-uniform)
            const bool full = k0 + kKBlock - 1 <= q0 && (W <= 0 || wq_last - k0 < W);
            if (!full) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + 8 * (r / 4) + 4 * half + (r % 4);
                    const bool vis = key <= qi && key < S32 && (W <= 0 || qi - key < W);
                    s[r] = vis ? s[r] : -INFINITY;
                }
            }
            float bmax = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) bmax = fmaxf(bmax, s[r]);
            bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
            const float m_new = fmaxf(m_run, bmax);
            // rescale of the sums so far (none yet, or nothing visible: 1)
            const float alpha = m_run == -INFINITY || m_new == -INFINITY
                                    ? 1.0f
                                    : __builtin_amdgcn_exp2f((m_run - m_new) * c2);
            // a query with nothing visible yet has m_new = -inf: its masked
            // scores give weight 0
            const float mc = m_new == -INFINITY ? 0.0f : m_new * c2;
            float psum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = __builtin_amdgcn_exp2f(fmaf(s[r], c2, -mc));
                psum += s[r];
            }
            den = den * alpha + psum;
            m_run = m_new;
#pragma unroll
            for (int m = 0; m < MB; ++m)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[m][r] *= alpha;
            // O^T += V^T P^T: step j takes key 8*(j/4) + 4*half + j%4
            const float* vcol = &Vs[buf][lq];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int key = 8 * (j / 4) + 4 * half + (j % 4);
#pragma unroll
                for (int m = 0; m < MB; ++m)
                    acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(vcol[key * LD + 32 * m], s[j],
                                                                  acc[m], 0, 0, 0);
            }
        }
        if (more) stage(buf ^ 1);  // the other buffer's last readers passed the previous barrier
        __syncthreads();
        buf ^= 1;
    }

    // out[query][dim] = O^T[dim][query] / den; register r of block m is dim
    // 32m + 8*(r/4) + 4*half + r%4: four consecutive dims per group
    const float den_all = den + __shfl_xor(den, 32, 64);
    if (wave_live && qi < S32) {
        float* orow = out + (b * S + qi) * qw + h * HD;
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 o;
#pragma unroll
                for (int t = 0; t < 4; ++t) o[t] = acc[m][4 * g + t] / den_all;
                *reinterpret_cast<f32x4*>(orow + 32 * m + 8 * g + 4 * half) = o;
            }
    }
}

}  // namespace

bool launch_flash_attention(const float* q, const float* k, const float* v, float* out,
                            int64_t batch, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                            int64_t head_dim, int64_t window, hipStream_t s) {
    if (seq_len > INT32_MAX) return false;  // key indices are 32-bit
    const dim3 grid(static_cast<unsigned>(ceil_div(seq_len, kQTile)),
                    static_cast<unsigned>(batch * q_heads));
    const float scale = sqrtf(static_cast<float>(head_dim));
    switch (head_dim) {
        case 64:
            hipLaunchKernelGGL(flash_attn_kernel<64>, grid, dim3(256), 0, s, q, k, v, out,
                               seq_len, q_heads, kv_heads, window, scale);
            return true;
        case 128:
            hipLaunchKernelGGL(flash_attn_kernel<128>, grid, dim3(256), 0, s, q, k, v, out,
                               seq_len, q_heads, kv_heads, window, scale);
            return true;
        default:
            return false;
    }
}

}  // namespace moe
