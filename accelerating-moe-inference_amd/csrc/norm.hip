// Post-attention layer norm of the MoE block (the reference's
// tensor_ops::layer_norm, src/tensor.cu:175-189, and its GPU form
// layer_norm_rows / DeviceNorm::forward_stats, src/model.cu:720-846,
// 1440-1480), bit-identical to the CPU loop:
//
//   mean = (sum over j ascending, one float accumulator) / h
//   var  = (sum over j ascending of d*d, d = x - mean) / h
//   inv  = 1 / sqrt(var + eps)
//   y    = (x - mean) * inv * w + b
//
// The two sums are sequential chains, so one lane owns one row.  A wave
// covers 64 rows: it stages a 64-row x 32-column chunk in LDS (coalesced
// 128-byte row segments on the global side, transposed with a 65-float
// stride so each lane then walks its own row conflict-free) and every lane
// advances its chain by 32 terms per chunk.  The stats kernel stops at
// (mean, inv): the MoE layer applies the last line inside the gate and the
// w1/w3 GEMM as they stage x, so the normalised rows are never written.  The
// apply kernel writes y for the standalone op.
#include "common.hpp"

namespace moe {
namespace {

constexpr int kNormRows = 64;   // rows per wave (one per lane)
constexpr int kNormChunk = 32;  // columns staged per step
constexpr int kNormWaves = 4;   // waves per workgroup
constexpr int kNormStride = kNormRows + 1;

template <int CONTRACT>
__device__ __forceinline__ float mac(float acc, float a, float b) {
    if (CONTRACT == MOE_CONTRACT_FMA) return __builtin_fmaf(a, b, acc);
    const float prod = a * b;
    return acc + prod;
}

template <int CONTRACT>
__global__ __launch_bounds__(64 * kNormWaves) void norm_stats_kernel(
        const float* __restrict__ x, int64_t rows, int64_t h, float eps,
        float* __restrict__ row_mean, float* __restrict__ row_inv) {
    __shared__ float tile[kNormWaves][kNormChunk * kNormStride];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* s = tile[wave];
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kNormWaves + wave) * kNormRows;
    if (row0 >= rows) return;  // wave-uniform: no barrier below spans waves
    const int64_t here = rows - row0 < kNormRows ? rows - row0 : kNormRows;

    // Staging: load i of a lane reads row (64 i + lane) / 32 of the chunk,
    // column lane % 32; rows past the end re-read the wave's first row.
    auto stage = [&](int64_t j0) {
        const int64_t cols = h - j0 < kNormChunk ? h - j0 : kNormChunk;
        float v[kNormChunk];
#pragma unroll
        for (int i = 0; i < kNormChunk; ++i) {
            const int flat = i * 64 + lane;
            const int r = flat / kNormChunk, c = flat % kNormChunk;
            const int64_t rr = r < here ? r : 0;
            v[i] = c < cols ? x[(row0 + rr) * h + j0 + c] : 0.0f;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < kNormChunk; ++i) {
            const int flat = i * 64 + lane;
            s[(flat % kNormChunk) * kNormStride + flat / kNormChunk] = v[i];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        return cols;
    };

    float sum = 0.0f;
    for (int64_t j0 = 0; j0 < h; j0 += kNormChunk) {
        const int64_t cols = stage(j0);
        for (int c = 0; c < cols; ++c) sum = sum + s[c * kNormStride + lane];
        __builtin_amdgcn_wave_barrier();
    }
    const float mean = sum / static_cast<float>(h);
    float var = 0.0f;
    for (int64_t j0 = 0; j0 < h; j0 += kNormChunk) {
        const int64_t cols = stage(j0);
        for (int c = 0; c < cols; ++c) {
            const float dv = s[c * kNormStride + lane] - mean;
            var = mac<CONTRACT>(var, dv, dv);
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (lane < here) {
        row_mean[row0 + lane] = mean;
        row_inv[row0 + lane] = 1.0f / sqrtf(var / static_cast<float>(h) + eps);
    }
}

template <int CONTRACT>
__global__ __launch_bounds__(256) void norm_apply_kernel(
        const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
        const float* __restrict__ row_mean, const float* __restrict__ row_inv, int64_t rows,
        int64_t h, float* __restrict__ y) {
    const int64_t n = rows * h;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        const int64_t r = i / h, j = i - r * h;
        y[i] = layer_norm_value<CONTRACT>(x[i], row_mean[r], row_inv[r], w[j], b[j]);
    }
}

}  // namespace

void launch_norm_stats(const float* x, int64_t rows, int64_t h, float eps, int contract,
                       float* row_mean, float* row_inv, hipStream_t s) {
    if (rows <= 0) return;
    const unsigned blocks =
        static_cast<unsigned>(ceil_div(ceil_div(rows, kNormRows), kNormWaves));
    if (contract == MOE_CONTRACT_FMA)
        hipLaunchKernelGGL(norm_stats_kernel<MOE_CONTRACT_FMA>, dim3(blocks),
                           dim3(64 * kNormWaves), 0, s, x, rows, h, eps, row_mean, row_inv);
    else
        hipLaunchKernelGGL(norm_stats_kernel<MOE_CONTRACT_NONE>, dim3(blocks),
                           dim3(64 * kNormWaves), 0, s, x, rows, h, eps, row_mean, row_inv);
}

void launch_norm_apply(const float* x, const float* w, const float* b, const float* row_mean,
                       const float* row_inv, int64_t rows, int64_t h, int contract, float* y,
                       hipStream_t s) {
    const int64_t n = rows * h;
    if (n <= 0) return;
    const int64_t blocks = ceil_div(n, 256);
    const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
    if (contract == MOE_CONTRACT_FMA)
        hipLaunchKernelGGL(norm_apply_kernel<MOE_CONTRACT_FMA>, grid, dim3(256), 0, s, x, w, b,
                           row_mean, row_inv, rows, h, y);
    else
        hipLaunchKernelGGL(norm_apply_kernel<MOE_CONTRACT_NONE>, grid, dim3(256), 0, s, x, w, b,
                           row_mean, row_inv, rows, h, y);
}

}  // namespace moe
