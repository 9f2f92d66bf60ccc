// Post-attention layer norm of the MoE block (the reference's
// tensor_ops::layer_norm, src/tensor.cu:175-189, and its GPU form
// layer_norm_rows, src/model.cu:720-846), bit-identical to the CPU loop:
//
//   mean = (sum over j ascending, one float accumulator) / h
//   var  = (sum over j ascending of d*d, d = x - mean) / h
//   inv  = 1 / sqrt(var + eps)
//   y    = (x - mean) * inv * w + b
//
// and the RMS norm config 5's decoder names (no reference code; defined in
// the same style): inv = 1 / sqrt(sum of x*x / h + eps), y = x * inv * w.
//
// The two sums are sequential chains, so one lane owns one row's chain; the
// work is feeding those chains.  Main kernel: a workgroup stages R whole
// rows in LDS with every thread loading (all of the rows' bytes in flight at
// once, the only way a latency-bound chain kernel reaches HBM bandwidth),
// R lanes then run the chains out of LDS, and all threads write y from the
// staged rows.  x is read once and y written once.  Two 79 KiB workgroups
// fit a CU (160 KiB of LDS), so one stages while the other runs its chains.
// Rows too wide for LDS take a streaming pair of kernels instead
// (statistics, then y).
//
// The layer writes the normalised rows once and its gate and w1/w3 GEMM read
// them like any x: the GEMM stages every A row once per 128-column tile of
// d_ff, so normalising inside it (the reference folds the norm into its
// gate and w13 staging, src/model.cu:225-246,549-559) repeats the work
// d_ff/128 times -- measured 12 % slower w1/w3 at config 3 -- where one
// write and one read of x cost about 0.03 ms.
#include "common.hpp"

namespace moe {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kResidentFloats = 20224;  // 79 KiB of staged rows: two workgroups per CU
constexpr int kMaxResidentRows = 64;
constexpr int kRowPad = 4;  // row stride h + 4: 16-byte aligned, chains on distinct banks

template <int CONTRACT>
__device__ __forceinline__ float mac(float acc, float a, float b) {
    if (CONTRACT == MOE_CONTRACT_FMA) return __builtin_fmaf(a, b, acc);
    const float prod = a * b;
    return acc + prod;
}

// The last line of the CPU loop: (x - mean) * inv * w + b, left to right,
// the final `* w + b` fused under MOE_CONTRACT_FMA.  RMS: x * inv * w.
template <int CONTRACT, bool RMS>
__device__ __forceinline__ float normalise(float x, float mean, float inv, float w, float b) {
    if (RMS) return (x * inv) * w;
    const float scaled = (x - mean) * inv;
    if (CONTRACT == MOE_CONTRACT_FMA) return __builtin_fmaf(scaled, w, b);
    const float prod = scaled * w;
    return prod + b;
}

// VEC4: h % 4 == 0 and 16-byte aligned x / y / w / b (16-byte accesses).
// RMS: no mean (the second chain sums x*x itself), no bias; row_mean unused.
template <int CONTRACT, bool VEC4, bool RMS>
__global__ __launch_bounds__(256) void norm_rows_kernel(
        const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
        int64_t rows, int64_t h, int R, float eps, float* __restrict__ row_mean,
        float* __restrict__ row_inv, float* __restrict__ y) {
    __shared__ __align__(16) float buf[kResidentFloats];
    __shared__ float smean[kMaxResidentRows], sinv[kMaxResidentRows];
    const int tid = threadIdx.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * R;
    const int nr = static_cast<int>(rows - r0 < R ? rows - r0 : R);
    const int64_t hs = h + kRowPad;
    const int64_t n = nr * h;  // the workgroup's rows are one contiguous span of x
    const float* src = x + r0 * h;

    if (VEC4) {
        for (int64_t i = 4 * tid; i < n; i += 4 * 256) {
            const int64_t r = i / h, j = i - r * h;
            *reinterpret_cast<f32x4*>(&buf[r * hs + j]) = *reinterpret_cast<const f32x4*>(src + i);
        }
    } else {
        for (int64_t i = tid; i < n; i += 256) {
            const int64_t r = i / h, j = i - r * h;
            buf[r * hs + j] = src[i];
        }
    }
    __syncthreads();

    if (tid < nr) {
        // The chains read 32 values ahead (8 16-byte LDS reads issued together),
        // so each add waits on an LDS round trip once per 32 terms, not per 4.
        constexpr int kAhead = 32;
        const float* row = &buf[tid * hs];
        float sum = 0.0f;
        int64_t j = RMS ? h : 0;  // RMS: no mean chain
        if (VEC4)
            for (; j + kAhead <= h; j += kAhead) {
                f32x4 v[kAhead / 4];
#pragma unroll
                for (int u = 0; u < kAhead / 4; ++u)
                    v[u] = *reinterpret_cast<const f32x4*>(row + j + 4 * u);
#pragma unroll
                for (int u = 0; u < kAhead / 4; ++u)
#pragma unroll
                    for (int q = 0; q < 4; ++q) sum = sum + v[u][q];
            }
#pragma unroll 16
        for (; j < h; ++j) sum = sum + row[j];
        const float mean = RMS ? 0.0f : sum / static_cast<float>(h);
        float var = 0.0f;
        j = 0;
        if (VEC4)
            for (; j + kAhead <= h; j += kAhead) {
                f32x4 v[kAhead / 4];
#pragma unroll
                for (int u = 0; u < kAhead / 4; ++u)
                    v[u] = *reinterpret_cast<const f32x4*>(row + j + 4 * u);
#pragma unroll
                for (int u = 0; u < kAhead / 4; ++u)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float dv = RMS ? v[u][q] : v[u][q] - mean;
                        var = mac<CONTRACT>(var, dv, dv);
                    }
            }
#pragma unroll 16
        for (; j < h; ++j) {
            const float dv = RMS ? row[j] : row[j] - mean;
            var = mac<CONTRACT>(var, dv, dv);
        }
        const float inv = 1.0f / sqrtf(var / static_cast<float>(h) + eps);
        smean[tid] = mean;
        sinv[tid] = inv;
        if (!RMS) row_mean[r0 + tid] = mean;
        row_inv[r0 + tid] = inv;
    }
    __syncthreads();
    if (y == nullptr) return;

    float* dst = y + r0 * h;
    if (VEC4) {
        for (int64_t i = 4 * tid; i < n; i += 4 * 256) {
            const int64_t r = i / h, j = i - r * h;
            const f32x4 v = *reinterpret_cast<const f32x4*>(&buf[r * hs + j]);
            const f32x4 wv = *reinterpret_cast<const f32x4*>(w + j);
            const f32x4 bv = RMS ? wv : *reinterpret_cast<const f32x4*>(b + j);
            f32x4 o;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[q] = normalise<CONTRACT, RMS>(v[q], smean[r], sinv[r], wv[q], bv[q]);
            *reinterpret_cast<f32x4*>(dst + i) = o;
        }
    } else {
        for (int64_t i = tid; i < n; i += 256) {
            const int64_t r = i / h, j = i - r * h;
            dst[i] = normalise<CONTRACT, RMS>(buf[r * hs + j], smean[r], sinv[r], w[j],
                                              RMS ? 0.0f : b[j]);
        }
    }
}

// ---- rows wider than kResidentFloats - kRowPad: streaming statistics.  One
// lane per row, 64 rows per wave, a 64-row x 32-column chunk staged in LDS
// at a time (transposed, 65-float stride) and consumed by every lane's
// chain; then an elementwise pass writes y.
constexpr int kStreamRows = 64;
constexpr int kStreamChunk = 32;
constexpr int kStreamWaves = 4;
constexpr int kStreamStride = kStreamRows + 1;

template <int CONTRACT, bool RMS>
__global__ __launch_bounds__(64 * kStreamWaves) void norm_stats_stream_kernel(
        const float* __restrict__ x, int64_t rows, int64_t h, float eps,
        float* __restrict__ row_mean, float* __restrict__ row_inv) {
    __shared__ float tile[kStreamWaves][kStreamChunk * kStreamStride];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* s = tile[wave];
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kStreamWaves + wave) * kStreamRows;
    if (row0 >= rows) return;  // wave-uniform; no barrier below spans waves
    const int64_t here = rows - row0 < kStreamRows ? rows - row0 : kStreamRows;

    // load i of a lane: row (64 i + lane) / 32 of the chunk, column lane % 32;
    // rows past the end re-read the wave's first row (never consumed)
    auto stage = [&](int64_t j0) {
        const int64_t cols = h - j0 < kStreamChunk ? h - j0 : kStreamChunk;
        float v[kStreamChunk];
#pragma unroll
        for (int i = 0; i < kStreamChunk; ++i) {
            const int flat = i * 64 + lane;
            const int r = flat / kStreamChunk, c = flat % kStreamChunk;
            const int64_t rr = r < here ? r : 0;
            v[i] = c < cols ? x[(row0 + rr) * h + j0 + c] : 0.0f;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < kStreamChunk; ++i) {
            const int flat = i * 64 + lane;
            s[(flat % kStreamChunk) * kStreamStride + flat / kStreamChunk] = v[i];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        return cols;
    };

    float sum = 0.0f;
    for (int64_t j0 = 0; !RMS && j0 < h; j0 += kStreamChunk) {
        const int64_t cols = stage(j0);
        for (int c = 0; c < cols; ++c) sum = sum + s[c * kStreamStride + lane];
        __builtin_amdgcn_wave_barrier();
    }
    const float mean = RMS ? 0.0f : sum / static_cast<float>(h);
    float var = 0.0f;
    for (int64_t j0 = 0; j0 < h; j0 += kStreamChunk) {
        const int64_t cols = stage(j0);
        for (int c = 0; c < cols; ++c) {
            const float v = s[c * kStreamStride + lane];
            const float dv = RMS ? v : v - mean;
            var = mac<CONTRACT>(var, dv, dv);
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (lane < here) {
        if (!RMS) row_mean[row0 + lane] = mean;
        row_inv[row0 + lane] = 1.0f / sqrtf(var / static_cast<float>(h) + eps);
    }
}

template <int CONTRACT, bool RMS>
__global__ __launch_bounds__(256) void norm_apply_kernel(
        const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
        const float* __restrict__ row_mean, const float* __restrict__ row_inv, int64_t rows,
        int64_t h, float* __restrict__ y) {
    const int64_t n = rows * h;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        const int64_t r = i / h, j = i - r * h;
        y[i] = RMS ? normalise<CONTRACT, true>(x[i], 0.0f, row_inv[r], w[j], 0.0f)
                   : normalise<CONTRACT, false>(x[i], row_mean[r], row_inv[r], w[j], b[j]);
    }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <int CONTRACT, bool RMS>
void launch(const float* x, const float* w, const float* b, int64_t rows, int64_t h, float eps,
            float* row_mean, float* row_inv, float* y, int cus, hipStream_t s) {
    const int64_t hs = h + kRowPad;
    if (hs <= kResidentFloats) {
        // rows per workgroup: enough workgroups for two per CU, as many rows
        // as the LDS holds
        int64_t R = ceil_div(rows, 2 * static_cast<int64_t>(cus > 0 ? cus : 1));
        R = R < 1 ? 1 : R;
        const int64_t fit = kResidentFloats / hs;
        R = R < fit ? R : fit;
        R = R < kMaxResidentRows ? R : kMaxResidentRows;
        const dim3 grid(static_cast<unsigned>(ceil_div(rows, R)));
        const bool vec4 = h % 4 == 0 && aligned16(x) && (y == nullptr || aligned16(y)) &&
                          (y == nullptr || (aligned16(w) && (RMS || aligned16(b))));
        if (vec4)
            hipLaunchKernelGGL((norm_rows_kernel<CONTRACT, true, RMS>), grid, dim3(256), 0, s, x,
                               w, b, rows, h, static_cast<int>(R), eps, row_mean, row_inv, y);
        else
            hipLaunchKernelGGL((norm_rows_kernel<CONTRACT, false, RMS>), grid, dim3(256), 0, s,
                               x, w, b, rows, h, static_cast<int>(R), eps, row_mean, row_inv, y);
        return;
    }
    const unsigned blocks =
        static_cast<unsigned>(ceil_div(ceil_div(rows, kStreamRows), kStreamWaves));
    hipLaunchKernelGGL((norm_stats_stream_kernel<CONTRACT, RMS>), dim3(blocks),
                       dim3(64 * kStreamWaves), 0, s, x, rows, h, eps, row_mean, row_inv);
    if (y == nullptr) return;
    const int64_t nblk = ceil_div(rows * h, 256);
    hipLaunchKernelGGL((norm_apply_kernel<CONTRACT, RMS>),
                       dim3(static_cast<unsigned>(nblk < 65536 ? nblk : 65536)), dim3(256), 0, s,
                       x, w, b, row_mean, row_inv, rows, h, y);
}

}  // namespace

void launch_layer_norm(const float* x, const float* w, const float* b, int64_t rows, int64_t h,
                       float eps, int contract, bool rms, float* row_mean, float* row_inv,
                       float* y, int cus, hipStream_t s) {
    if (rows <= 0 || h <= 0) return;
    if (contract == MOE_CONTRACT_FMA) {
        if (rms) launch<MOE_CONTRACT_FMA, true>(x, w, b, rows, h, eps, row_mean, row_inv, y, cus, s);
        else launch<MOE_CONTRACT_FMA, false>(x, w, b, rows, h, eps, row_mean, row_inv, y, cus, s);
    } else {
        if (rms) launch<MOE_CONTRACT_NONE, true>(x, w, b, rows, h, eps, row_mean, row_inv, y, cus, s);
        else launch<MOE_CONTRACT_NONE, false>(x, w, b, rows, h, eps, row_mean, row_inv, y, cus, s);
    }
}

}  // namespace moe
