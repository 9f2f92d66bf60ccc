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
// work is feeding those chains.  Narrow rows: a workgroup stages R whole
// rows in LDS with every thread loading (all of the rows' bytes in flight at
// once, the only way a latency-bound chain kernel reaches HBM bandwidth),
// R lanes then run the chains out of LDS, and all threads write y from the
// staged rows.  x is read once and y written once.  Two 79 KiB workgroups
// fit a CU (160 KiB of LDS), so one stages while the other runs its chains.
// Wide rows, of which few fit: the ring kernel (a wave streams its rows'
// chains through an LDS ring, many rows per CU in flight) and a 16-byte
// elementwise pass for y; unaligned wide rows, a register-staged streaming
// pair.
//
// The layer writes the normalised rows once and its gate and w1/w3 GEMM read
// them like any x: the GEMM stages every A row once per 128-column tile of
// d_ff, so normalising inside it (the reference folds the norm into its
// gate and w13 staging, src/model.cu:225-246,549-559) repeats the work
// d_ff/128 times -- measured 12 % slower w1/w3 at config 3 -- where one
// write and one read of x cost about 0.03 ms.
#include "common.hpp"

#include <utility>

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

// ---- wide rows with few resident per CU: the streaming ring kernel.
//
// One wave per workgroup owns G rows (lane r runs row r's chains; lanes past
// G read a valid row and are ignored).  The rows stream through an LDS ring
// of RING stages of G rows x 64 columns, filled with direct global->LDS
// buffer loads RING - 1 stages ahead of the chains, so each wave keeps
// ~28 KiB in flight and a CU holds four or five such waves: the kernel is
// HBM-bound (x is read twice -- the sum, then the squared deviations; the
// apply pass below reads it a third time and writes y) instead of bound by
// the few chains whole staged rows leave room for.  Load instruction i of a stage writes 16-byte slot
// p = 64 i + lane of the stage, i.e. slot s = p % 16 of row r = p / 16, and
// fetches the row's 16-byte chunk q = s ^ (r % 16): a chain lane reading
// chunk q of its row finds it at slot q ^ (r % 16), so the 64 lanes' reads
// of one chunk spread over all banks.
constexpr int kStreamCols = 64;                  // columns per stage
constexpr int kStreamSlots = kStreamCols / 4;    // 16-byte chunks per row and stage
constexpr int kRingFloats = 8192;                // 32 KiB ring per wave

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void ring_load16(const float* base, lds_void_t* dst, uint32_t voff) {
    const uint64_t v = reinterpret_cast<uint64_t>(base);
    const uint64_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v))));
    const uint64_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v >> 32))));
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>((hi << 32) | lo), static_cast<short>(0), -1, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, 0, 0, 0);
}

template <int... I, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}), ...);
}

template <int CONTRACT, bool RMS, int G>
__global__ __launch_bounds__(64) void norm_ring_kernel(
        const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
        int64_t rows, int64_t h, float eps, float* __restrict__ row_mean,
        float* __restrict__ row_inv, float* __restrict__ y) {
    constexpr int STAGE = G * kStreamCols;                 // floats per stage
    constexpr int RING = kRingFloats / STAGE < 8 ? kRingFloats / STAGE : 8;
    constexpr int INS = G * kStreamSlots / 64;             // load instructions per stage
    static_assert(INS >= 1 && RING >= 4 && (RING - 2) * INS <= 63, "ring shape");
    // One array per stage: the compiler then knows which loads land in the
    // stage being read and waits for those alone (with one array it would
    // wait for every load in flight before each read).
    __shared__ __align__(16) float r0[STAGE], r1[STAGE], r2[STAGE], r3[STAGE];
    __shared__ __align__(16) float r4[RING > 4 ? STAGE : 4], r5[RING > 4 ? STAGE : 4],
        r6[RING > 4 ? STAGE : 4], r7[RING > 4 ? STAGE : 4];
    auto buf = [&](auto u) -> float* {
        constexpr int U = decltype(u)::value;
        if constexpr (U == 0) return r0;
        else if constexpr (U == 1) return r1;
        else if constexpr (U == 2) return r2;
        else if constexpr (U == 3) return r3;
        else if constexpr (U == 4) return r4;
        else if constexpr (U == 5) return r5;
        else if constexpr (U == 6) return r6;
        else return r7;
    };
    using Stages = std::make_integer_sequence<int, RING>;

    const int lane = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * G;
    const int here = static_cast<int>(rows - row0 < G ? rows - row0 : G);
    const float* base = x + row0 * h;  // wave-uniform; offsets below stay under G * h floats
    const int64_t nst = (h + kStreamCols - 1) / kStreamCols;

    // source row and chunk of this lane's slot in load instruction i
    int lrow[INS], lchunk[INS];
#pragma unroll
    for (int i = 0; i < INS; ++i) {
        const int p = 64 * i + lane, r = p / kStreamSlots, sl = p % kStreamSlots;
        lrow[i] = r < here ? r : here - 1;
        lchunk[i] = sl ^ (r % kStreamSlots);
    }
    auto issue = [&](int64_t st, float* dst) {
        const int64_t j0 = st * kStreamCols;
#pragma unroll
        for (int i = 0; i < INS; ++i) {
            int64_t col = j0 + 4 * lchunk[i];
            col = col <= h - 4 ? col : h - 4;  // past the row end: a valid chunk, never used
            ring_load16(base, (lds_void_t*)(dst + 256 * i),
                        static_cast<uint32_t>((lrow[i] * h + col) * 4));
        }
    };
    // Waits until stage st has landed.  When it is awaited, the stages
    // issued after it are st + 1 .. st + RING - 2 (the prologue issues
    // RING - 1 stages, each step one more after its wait), and no other
    // vector-memory operation is in flight, so vmcnt((RING - 2) * INS)
    // leaves exactly those; near the end fewer follow, and it waits for all.
    auto wait_stage = [&](int64_t st) {
        if (st + RING - 2 < nst) {
            constexpr int N = (RING - 2) * INS;
            __builtin_amdgcn_s_waitcnt(0x3f70 | (N & 15) | ((N >> 4) << 14));
        } else {
            __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
        }
    };
    // walks every stage in order: consume(stage floats, st) once each stage
    // has landed, the ring kept RING - 1 stages ahead
    auto stream = [&](auto consume) {
        static_for(std::make_integer_sequence<int, RING - 1>{}, [&](auto u) {
            if (decltype(u)::value < nst) issue(decltype(u)::value, buf(u));
        });
        for (int64_t st0 = 0; st0 < nst; st0 += RING) {
            static_for(Stages{}, [&](auto u) {
                constexpr int U = decltype(u)::value;
                const int64_t st = st0 + U;
                if (st < nst) {
                    wait_stage(st);
                    consume(buf(u), st);
                    // the stage's reads are done before its buffer is refilled
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                    if (st + RING - 1 < nst)
                        issue(st + RING - 1, buf(std::integral_constant<int, (U + RING - 1) % RING>{}));
                }
            });
        }
    };
    const int rr = lane < G ? lane : G - 1;
    const int sw = rr % kStreamSlots;
    // one pass of a row chain over every stage, in column order
    auto chain_pass = [&](auto step) {
        float acc = 0.0f;
        stream([&](const float* stage, int64_t st) {
            const float* src = stage + rr * kStreamCols;
            const int64_t j0 = st * kStreamCols;
            if (j0 + kStreamCols <= h) {
                // all 16 reads first, then the 64 dependent adds
                f32x4 v[kStreamSlots];
#pragma unroll
                for (int q = 0; q < kStreamSlots; ++q)
                    v[q] = *reinterpret_cast<const f32x4*>(src + 4 * (q ^ sw));
#pragma unroll
                for (int q = 0; q < kStreamSlots; ++q)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc = step(acc, v[q][c]);
            } else {
                for (int q = 0; q < kStreamSlots; ++q) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * (q ^ sw));
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (j0 + 4 * q + c < h) acc = step(acc, v[c]);
                }
            }
        });
        return acc;
    };

    float mean = 0.0f;
    if (!RMS) {
        const float sum = chain_pass([](float a, float v) { return a + v; });
        mean = sum / static_cast<float>(h);
    }
    const float var = chain_pass([&](float a, float v) {
        const float dv = RMS ? v : v - mean;
        return mac<CONTRACT>(a, dv, dv);
    });
    const float inv = 1.0f / sqrtf(var / static_cast<float>(h) + eps);
    if (lane < here) {
        if (!RMS) row_mean[row0 + lane] = mean;
        row_inv[row0 + lane] = inv;
    }
}

// y from the row statistics, 16 bytes per thread (h % 4 == 0, aligned).
template <int CONTRACT, bool RMS>
__global__ __launch_bounds__(256) void norm_apply4_kernel(
        const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
        const float* __restrict__ row_mean, const float* __restrict__ row_inv, int64_t rows,
        int64_t h, float* __restrict__ y) {
    const int64_t h4 = h >> 2, n4 = rows * h4;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    // 32-bit row division when every index fits (the launch grid-strides
    // at most 2^24 past n4): a 64-bit division costs a long instruction
    // sequence per 16 bytes moved
    const bool narrow = n4 < (int64_t(1) << 31);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4;
         i += stride) {
        const int64_t r = narrow ? static_cast<int64_t>(static_cast<uint32_t>(i) /
                                                        static_cast<uint32_t>(h4))
                                 : i / h4;
        const int64_t j = 4 * (i - r * h4);
        const f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
        const f32x4 wv = *reinterpret_cast<const f32x4*>(w + j);
        const f32x4 bv = RMS ? wv : *reinterpret_cast<const f32x4*>(b + j);
        const float mean = RMS ? 0.0f : row_mean[r], inv = row_inv[r];
        f32x4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = normalise<CONTRACT, RMS>(v[c], mean, inv, wv[c], bv[c]);
        reinterpret_cast<f32x4*>(y)[i] = o;
    }
}

// The ring kernel takes aligned rows of which fewer than this many fit a
// resident workgroup's LDS (h > 1260 floats): measured on MI355X, d = 2048
// 0.160 -> 0.097 ms, d = 4096 0.45 -> 0.20 ms at 15,583 rows; d = 1024 (19
// rows fit) is as fast resident.
constexpr int64_t kRingBelowRows = 16;

template <int CONTRACT, bool RMS>
void launch(const float* x, const float* w, const float* b, int64_t rows, int64_t h, float eps,
            float* row_mean, float* row_inv, float* y, int cus, hipStream_t s) {
    const int64_t hs = h + kRowPad;
    const bool aligned = h % 4 == 0 && aligned16(x) &&
                         (y == nullptr || (aligned16(y) && aligned16(w) && (RMS || aligned16(b))));
    if (aligned && kResidentFloats / hs < kRingBelowRows &&
        int64_t(32) * h * 4 < (int64_t(1) << 31)) {
        // rows per wave: enough waves for every CU to hold several (measured
        // on MI355X: 8 rows per wave beat 16 by 1-4 % from 4,096 to 16,384
        // rows of 2048-4096 floats, and 32 by 7-20 %)
        const int64_t c = cus > 0 ? cus : 256;
#ifndef MOE_NORM_RING_G
#define MOE_NORM_RING_G 0
#endif
        int G = rows >= 32 * 4 * c ? 32 : 8;
        if (MOE_NORM_RING_G == 8 || MOE_NORM_RING_G == 16 || MOE_NORM_RING_G == 32) G = MOE_NORM_RING_G;
        const dim3 grid(static_cast<unsigned>(ceil_div(rows, G)));
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(64), 0, s, x, w, b, rows, h, eps, row_mean,
                               row_inv, y);
        };
        if (G == 32) go(norm_ring_kernel<CONTRACT, RMS, 32>);
        else if (G == 16) go(norm_ring_kernel<CONTRACT, RMS, 16>);
        else go(norm_ring_kernel<CONTRACT, RMS, 8>);
        if (y == nullptr) return;
        const int64_t nblk = ceil_div(rows * (h / 4), 256);
        hipLaunchKernelGGL((norm_apply4_kernel<CONTRACT, RMS>),
                           dim3(static_cast<unsigned>(nblk < 8 * c ? nblk : 8 * c)), dim3(256), 0,
                           s, x, w, b, row_mean, row_inv, rows, h, y);
        return;
    }
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
