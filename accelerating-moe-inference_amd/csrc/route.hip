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
#include <utility>

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

// Zeroes zero[0 .. nzero) with every thread of the launch (2D grids
// included): the layer's routing counters, cleared by the launch before the
// one that adds into them.  A no-op when zero is null.
__device__ __forceinline__ void zero_words(uint32_t* __restrict__ zero, int64_t nzero) {
    if (zero == nullptr) return;
    const int64_t nthreads = int64_t(gridDim.x) * gridDim.y * blockDim.x;
    for (int64_t i = (int64_t(blockIdx.y) * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
         i < nzero; i += nthreads)
        zero[i] = 0u;
}

// TE > 1: each thread runs TB tokens x TE experts (experts el, el + EB/TE,
// ...: the lanes of a wave then read TE distinct expert rows per read), so a
// 16-byte LDS read of x feeds TE chains and one of w feeds TB: at 64 experts
// with TE = 1 the reads, not the multiply-adds, bounded the kernel.
template <int CONTRACT, int EB, int TB, int TE = 1>
__global__ __launch_bounds__(256) void gate_logits_kernel(
        const float* __restrict__ x, const float* __restrict__ w,
        float* __restrict__ logits, int64_t T, int64_t d, int64_t E,
        uint32_t* __restrict__ zero, int64_t nzero) {
    constexpr int EG = EB / TE;               // expert groups (threads per token row group)
    constexpr int R = TB * (256 / EG);        // token rows per workgroup
    constexpr int ROWS = R + EB;              // staged rows: x rows, then w rows
    constexpr int PER = ROWS * GATE_KC / 256; // staged floats per thread
    static_assert(EB % TE == 0 && 256 % EG == 0 && ROWS * GATE_KC % 256 == 0, "gate tile");
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float tile[2][ROWS * GATE_LDS];
    zero_words(zero, nzero);

    const int tid = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * R;
    const int64_t e0 = static_cast<int64_t>(blockIdx.y) * EB;
    const int el = tid % EG, r = tid / EG;

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

    float acc[TB][TE];
#pragma unroll
    for (int u = 0; u < TB; ++u)
#pragma unroll
        for (int v = 0; v < TE; ++v) acc[u][v] = 0.0f;
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
        const float* wr = &tile[buf][(R + el) * GATE_LDS];  // its TE rows, EG apart
        int kk = 0;
        for (; kk + 4 <= kn; kk += 4) {
            f4 wv[TE];
#pragma unroll
            for (int v = 0; v < TE; ++v)
                wv[v] = *reinterpret_cast<const f4*>(wr + v * EG * GATE_LDS + kk);
#pragma unroll
            for (int u = 0; u < TB; ++u) {
                const f4 xv = *reinterpret_cast<const f4*>(xr + u * GATE_LDS + kk);
#pragma unroll
                for (int v = 0; v < TE; ++v) {
                    acc[u][v] = mac<CONTRACT>(acc[u][v], xv[0], wv[v][0]);
                    acc[u][v] = mac<CONTRACT>(acc[u][v], xv[1], wv[v][1]);
                    acc[u][v] = mac<CONTRACT>(acc[u][v], xv[2], wv[v][2]);
                    acc[u][v] = mac<CONTRACT>(acc[u][v], xv[3], wv[v][3]);
                }
            }
        }
        for (; kk < kn; ++kk)
#pragma unroll
            for (int u = 0; u < TB; ++u)
#pragma unroll
                for (int v = 0; v < TE; ++v)
                    acc[u][v] = mac<CONTRACT>(acc[u][v], xr[u * GATE_LDS + kk],
                                              wr[v * EG * GATE_LDS + kk]);
        if (c + 1 < nchunks) lstore(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int v = 0; v < TE; ++v) {
        const int64_t e = e0 + el + v * EG;
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            const int64_t t = t0 + r * TB + u;
            if (t < T && e < E) logits[t * E + e] = acc[u][v];
        }
    }
}

// Small E (up to 8): the ring form.  One wave per workgroup; lane
// (r, e) = (lane / EB, lane % EB) owns the chain of token t0 + r and expert
// e.  The R token rows and the EB expert rows stream through an LDS ring of
// 64-column stages, filled with direct global->LDS buffer loads RING - 1
// stages ahead (load instruction i of a stage fills 16-byte slot
// p = 64 i + lane: row p / 16, slot p % 16, which holds the row's chunk
// (p % 16) ^ (row % 16), so the lanes' reads of one chunk from different
// rows hit different banks).  Each stage is its own __shared__ array and the
// stage loop is unrolled over the ring, so the compiler waits only for the
// stage being read.  Every lane then runs 64 multiply-adds per stage in
// column order -- the chain of the kernel above -- with T/R workgroups
// instead of T/32 (at config 3, 512 instead of 128).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kGateRingCols = 64;
constexpr int kGateRing = 8;
// Up to this many token x expert logits, 9-64 experts take the per-wave ring
// with expert blocks (gate_ring_kernel over grid.y); measured on MI355X, us,
// expert blocks against the workgroup ring / staged kernel: the reference's
// E = 16 at d 4096, 1 / 64 / 1,024 / 4,096 tokens 39.2 / 38.9 / 40.1 / 43.9
// against 45.3 / 47.1 / 47.6 / 48.9, at 15,583 tokens 209.9 against 88.8;
// config 4's E = 64 at d 2048, 16 / 1,024 tokens 23.1 / 25.9 against 86.6 /
// 91.3, 4,096 86.9 against 88.2, 16,384 352.6 against 105.6.
constexpr int64_t kGateFewLogits = 65536;

typedef __attribute__((address_space(3))) void gate_lds_t;

__device__ __forceinline__ void gate_load16(const float* base, gate_lds_t* dst, uint32_t voff) {
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
__device__ __forceinline__ void gate_static_for(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}), ...);
}

template <int CONTRACT, int EB>
__global__ __launch_bounds__(64) void gate_ring_kernel(
        const float* __restrict__ x, const float* __restrict__ w,
        float* __restrict__ logits, int64_t T, int64_t d, int64_t E,
        uint32_t* __restrict__ zero, int64_t nzero) {
    constexpr int R = 64 / EB;                     // token rows per wave
    constexpr int ROWS = R + EB;                   // staged rows: tokens, then experts
    constexpr int STAGE = ROWS * kGateRingCols;    // floats per stage
    constexpr int INS = ROWS * 16 / 64;            // load instructions per stage
    constexpr int RING = kGateRing;
    static_assert(R % 4 == 0 && EB % 4 == 0, "an instruction's 4 rows come from one matrix");
    static_assert((RING - 2) * INS <= 63, "vmcnt range");
    __shared__ __align__(16) float r0[STAGE], r1[STAGE], r2[STAGE], r3[STAGE], r4[STAGE],
        r5[STAGE], r6[STAGE], r7[STAGE];
    auto buf = [&](auto u) __attribute__((always_inline)) -> float* {
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

    zero_words(zero, nzero);
    const int lane = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * R;
    const int64_t nt = T - t0 < R ? T - t0 : R;  // tokens of this wave (>= 1)
    const int64_t e0 = static_cast<int64_t>(blockIdx.y) * EB;  // this wave's expert block
    const int64_t ne = E - e0 < EB ? E - e0 : EB;                // its experts (>= 1)
    const int64_t nst = (d + kGateRingCols - 1) / kGateRingCols;

    // instruction i: rows 4i .. 4i + 3 of the stage, one matrix each
    const float* ibase[INS];
    uint32_t ioff[INS];
#pragma unroll
    for (int i = 0; i < INS; ++i) {
        const int p = 64 * i + lane, row = p / 16, sl = p % 16;
        const int chunk = sl ^ (row % 16);
        if (4 * i < R) {  // token rows
            const int64_t rr = row < nt ? row : nt - 1;
            ibase[i] = x + t0 * d;
            ioff[i] = static_cast<uint32_t>((rr * d + 4 * chunk) * 4);
        } else {          // expert rows
            const int64_t e = row - R < ne ? row - R : ne - 1;
            ibase[i] = w + e0 * d;
            ioff[i] = static_cast<uint32_t>((e * d + 4 * chunk) * 4);
        }
    }
    auto issue = [&](int64_t st, float* dst) __attribute__((always_inline)) {
        const int64_t j0 = st * kGateRingCols;
#pragma unroll
        for (int i = 0; i < INS; ++i) {
            // a chunk past the row end loads the row's last chunk (never used)
            const int chunk = (64 * i + lane) % 16 ^ (((64 * i + lane) / 16) % 16);
            const int64_t shift = j0 + 4 * chunk <= d - 4 ? j0 : d - 4 - 4 * chunk;
            gate_load16(ibase[i], (gate_lds_t*)(dst + 256 * i),
                        static_cast<uint32_t>(ioff[i] + shift * 4));
        }
    };
    auto wait_stage = [&](int64_t st) __attribute__((always_inline)) {
        if (st + RING - 2 < nst) {
            constexpr int N = (RING - 2) * INS;
            __builtin_amdgcn_s_waitcnt(0x3f70 | (N & 15) | ((N >> 4) << 14));
        } else {
            __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
        }
    };

    const int r = lane / EB, e = lane % EB;
    const int xsw = r % 16, wsw = (R + e) % 16;
    float acc = 0.0f;
    auto consume = [&](const float* stage, int64_t st) __attribute__((always_inline)) {
        const float* xr = stage + r * kGateRingCols;
        const float* wr = stage + (R + e) * kGateRingCols;
        const int64_t j0 = st * kGateRingCols;
        if (j0 + kGateRingCols <= d) {
            // the stage's 32 LDS reads first, then the 64-step chain: the
            // chain no longer waits on a read every 4 steps (bit-identical;
            // the reference's gate at 1 and 64 tokens 39.6 / 38.6 -> 35.3 /
            // 34.2 us, config 4's at 64 tokens 24.1 -> 20.7, config 3's 41.3
            // -> 39.9).  In the workgroup ring below, at four waves per SIMD,
            // the same 128 registers spilled: 81 -> 428 us at the
            // reference's 15,583 tokens.
            f32x4_t xs[16], ws[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                xs[q] = *reinterpret_cast<const f32x4_t*>(xr + 4 * (q ^ xsw));
                ws[q] = *reinterpret_cast<const f32x4_t*>(wr + 4 * (q ^ wsw));
            }
#pragma unroll
            for (int q = 0; q < 16; ++q)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc = mac<CONTRACT>(acc, xs[q][c], ws[q][c]);
        } else {
            for (int q = 0; q < 16; ++q) {
                const f32x4_t xv = *reinterpret_cast<const f32x4_t*>(xr + 4 * (q ^ xsw));
                const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(wr + 4 * (q ^ wsw));
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (j0 + 4 * q + c < d) acc = mac<CONTRACT>(acc, xv[c], wv[c]);
            }
        }
    };
    gate_static_for(std::make_integer_sequence<int, RING - 1>{}, [&](auto u) __attribute__((always_inline)) {
        if (decltype(u)::value < nst) issue(decltype(u)::value, buf(u));
    });
    for (int64_t st0 = 0; st0 < nst; st0 += RING) {
        gate_static_for(std::make_integer_sequence<int, RING>{}, [&](auto u) __attribute__((always_inline)) {
            constexpr int U = decltype(u)::value;
            const int64_t st = st0 + U;
            if (st < nst) {
                wait_stage(st);
                consume(buf(u), st);
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this stage is read
                if (st + RING - 1 < nst)
                    issue(st + RING - 1, buf(std::integral_constant<int, (U + RING - 1) % RING>{}));
            }
        });
    }
    if (r < nt && e < ne) logits[(t0 + r) * E + e0 + e] = acc;
}

// E of 9-16: the ring form with the workgroup sharing each stage.  A wave of
// its own would stream all EB expert rows for its few tokens (at E = 16, 4
// tokens: four times the token bytes); here 256 threads hold
// R = TB * 256 / EB tokens x EB experts, as in the staged kernel above
// (thread (r, e) runs the chains of tokens r TB .. r TB + TB - 1 for expert
// e), and the R token rows and EB expert rows stream through a RING-stage
// LDS ring of 64-column stages filled by direct buffer loads RING - 1 stages
// ahead, so each workgroup keeps (RING - 1) stages of loads in flight instead
// of one register-staged chunk.  Chunk p = 256 i + tid of a stage is row
// p / 16, slot p % 16, holding the row's chunk (p % 16) ^ (row % 16) (the
// reads of one chunk from 16 rows hit distinct banks).  Per stage every
// thread waits for its own loads, the workgroup meets at a barrier (so every
// thread's loads of the stage have landed and the stage read last has been
// consumed by all), the loads RING - 1 stages ahead go into that consumed
// stage, and the stage is consumed: 64 multiply-adds per chain in column
// order, the chain of the kernels above.  (Two tokens per thread, and the
// 64-expert form with four, kept too many chains' reads in registers and ran
// 1.5-6x slower; those keep the staged kernel.)
// Ring depth and the waves per SIMD the register budget is set for
// (measured on MI355X at the reference's 15,583 x 4096 x 16: 3 stages at 4
// waves 84 us; 4 stages at 3 waves 132 us, at 4 waves 217 us; 6 at 2, 112 us;
// 8 at 2, 242 us; the staged kernel 110 us in the same runs).  A grid of at
// most one workgroup per CU is bound by each workgroup's stage round trips
// instead (62-67 us from 1 to 4,096 tokens at 16 experts; 5 stages at 2
// waves 45-49 us): such small batches take the per-wave ring with expert
// blocks (kGateFewLogits), faster still.
template <int CONTRACT, int EB, int TB, int RING, int OCC>
__global__ __launch_bounds__(256, OCC) void gate_wg_ring_kernel(
        const float* __restrict__ x, const float* __restrict__ w,
        float* __restrict__ logits, int64_t T, int64_t d, int64_t E,
        uint32_t* __restrict__ zero, int64_t nzero) {
    constexpr int R = TB * (256 / EB);             // token rows per workgroup
    constexpr int ROWS = R + EB;                   // staged rows: tokens, then experts
    constexpr int STAGE = ROWS * kGateRingCols;    // floats per stage
    constexpr int INS = ROWS * 16 / 256;           // load instructions per thread and stage
    static_assert(ROWS * 16 % 256 == 0 && R % 4 == 0, "whole instructions, 4 rows of one matrix each");
    static_assert(RING >= 3 && RING <= 8 && (RING - 2) * INS <= 63, "ring depth");
    __shared__ __align__(16) float r0[STAGE], r1[STAGE], r2[STAGE], r3[RING > 3 ? STAGE : 1],
        r4[RING > 4 ? STAGE : 1], r5[RING > 5 ? STAGE : 1], r6[RING > 6 ? STAGE : 1],
        r7[RING > 7 ? STAGE : 1];
    auto buf = [&](auto u) __attribute__((always_inline)) -> float* {
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

    zero_words(zero, nzero);
    const int tid = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * R;
    const int64_t e0 = static_cast<int64_t>(blockIdx.y) * EB;
    const int64_t nt = T - t0 < R ? T - t0 : R;    // tokens of this workgroup (>= 1)
    const int64_t ne = E - e0 < EB ? E - e0 : EB;  // experts of this workgroup (>= 1)
    const int64_t nst = (d + kGateRingCols - 1) / kGateRingCols;

    // instruction i of this thread: chunk 256 i + tid; the 64 lanes of a
    // wave cover rows 4 j .. 4 j + 3 of one matrix (R is a multiple of 4)
    const float* ibase[INS];
    uint32_t ioff[INS];
    int ichunk[INS];
#pragma unroll
    for (int i = 0; i < INS; ++i) {
        const int p = 256 * i + tid, row = p / 16, sl = p % 16;
        ichunk[i] = sl ^ (row % 16);
        if (row < R) {  // token rows (past the last token: the last one, never stored)
            const int64_t rr = row < nt ? row : nt - 1;
            ibase[i] = x + t0 * d;
            ioff[i] = static_cast<uint32_t>((rr * d + 4 * ichunk[i]) * 4);
        } else {        // expert rows
            const int64_t e = row - R < ne ? row - R : ne - 1;
            ibase[i] = w + e0 * d;
            ioff[i] = static_cast<uint32_t>((e * d + 4 * ichunk[i]) * 4);
        }
    }
    auto issue = [&](int64_t st, float* dst) __attribute__((always_inline)) {
        const int64_t j0 = st * kGateRingCols;
#pragma unroll
        for (int i = 0; i < INS; ++i) {
            // a chunk past the row end loads the row's last chunk (never used)
            const int64_t shift = j0 + 4 * ichunk[i] <= d - 4 ? j0 : d - 4 - 4 * ichunk[i];
            gate_load16(ibase[i], (gate_lds_t*)(dst + 1024 * i + 256 * (tid >> 6)),
                        static_cast<uint32_t>(ioff[i] + shift * 4));
        }
    };
    // before consuming stage st: this thread's loads of it have landed; the
    // stages issued after it (at most RING - 2) may stay in flight
    auto wait_stage = [&](int64_t st) __attribute__((always_inline)) {
        const int64_t after = (st + RING - 1 < nst ? st + RING - 1 : nst) - st - 1;
        gate_static_for(std::make_integer_sequence<int, RING - 1>{}, [&](auto c) __attribute__((always_inline)) {
            constexpr int A = decltype(c)::value, N = A * INS;
            if (after == A) __builtin_amdgcn_s_waitcnt(0x3f70 | (N & 15) | ((N >> 4) << 14));
        });
    };

    const int r = tid / EB, e = tid % EB;
    const int wsw = (R + e) % 16;
    float acc[TB];
#pragma unroll
    for (int u = 0; u < TB; ++u) acc[u] = 0.0f;
    auto consume = [&](const float* stage, int64_t st) __attribute__((always_inline)) {
        const float* wr = stage + (R + e) * kGateRingCols;
        const int64_t j0 = st * kGateRingCols;
        if (j0 + kGateRingCols <= d) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(wr + 4 * (q ^ wsw));
#pragma unroll
                for (int u = 0; u < TB; ++u) {
                    const int row = r * TB + u;
                    const f32x4_t xv = *reinterpret_cast<const f32x4_t*>(
                        stage + row * kGateRingCols + 4 * (q ^ (row % 16)));
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[u] = mac<CONTRACT>(acc[u], xv[c], wv[c]);
                }
            }
        } else {
            for (int q = 0; q < 16; ++q) {
                const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(wr + 4 * (q ^ wsw));
#pragma unroll
                for (int u = 0; u < TB; ++u) {
                    const int row = r * TB + u;
                    const f32x4_t xv = *reinterpret_cast<const f32x4_t*>(
                        stage + row * kGateRingCols + 4 * (q ^ (row % 16)));
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (j0 + 4 * q + c < d) acc[u] = mac<CONTRACT>(acc[u], xv[c], wv[c]);
                }
            }
        }
    };
    gate_static_for(std::make_integer_sequence<int, RING - 1>{}, [&](auto u) __attribute__((always_inline)) {
        if (decltype(u)::value < nst) issue(decltype(u)::value, buf(u));
    });
    for (int64_t st0 = 0; st0 < nst; st0 += RING) {
        gate_static_for(std::make_integer_sequence<int, RING>{}, [&](auto u) __attribute__((always_inline)) {
            constexpr int U = decltype(u)::value;
            const int64_t st = st0 + U;
            if (st < nst) {
                wait_stage(st);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this thread's reads of st - 1 are done
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                if (st + RING - 1 < nst)
                    issue(st + RING - 1, buf(std::integral_constant<int, (U + RING - 1) % RING>{}));
                consume(buf(u), st);
            }
        });
    }
    // the ring's loads have all been waited for (the last stage's wait is
    // vmcnt(0)), so the workgroup's LDS is quiet when it ends
#pragma unroll
    for (int u = 0; u < TB; ++u) {
        const int64_t t = t0 + r * TB + u;
        if (r * TB + u < nt && e < ne) logits[t * E + e0 + e] = acc[u];
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
// Writes token t's k picks and weights; picks[] receives the experts.
__device__ __forceinline__ void route_phi_token(const float* __restrict__ row,
                                                const float* __restrict__ bias, int64_t E,
                                                int64_t k, float quantum, float tie_eps,
                                                int32_t* __restrict__ idx_t,
                                                float* __restrict__ w_t, int32_t* picks) {
    const float weight = 1.0f / static_cast<float>(k);
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
        idx_t[s] = best;
        w_t[s] = weight;
    }
}

__global__ __launch_bounds__(256) void route_phi_kernel(
        const float* __restrict__ logits, const float* __restrict__ bias,
        int64_t T, int64_t E, int64_t k, float quantum, float tie_eps,
        int32_t* __restrict__ idx, float* __restrict__ w) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    int32_t picks[kMaxTopK];
    route_phi_token(logits + t * E, bias, E, k, quantum, tie_eps, idx + t * k, w + t * k, picks);
}

// SOFTMAX_TOPK: a group of G lanes (a power of two, <= 64) per token; lane j
// holds experts j, j+G, ...  Each of the k rounds takes every lane's best
// unpicked expert and reduces over the group with xor-shuffles under the
// total order (value descending, index ascending), NaN ranking as -inf.
// The group's first lane then forms the weights in double, as the oracle.
__device__ __forceinline__ bool beats(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

// Token t's top-k by the group of G lanes this lane belongs to (sub: the
// lane's index in it); every lane of the group must call it, live or not.
// Round s takes every lane's best unpicked expert and reduces over the group
// with xor-shuffles, so every lane learns pick s; lane s keeps it (k <= E <=
// G).  Then lane s forms exp(v_s - v_0) in double, the group's first lane
// adds the k of them in pick order (the oracle's sum), and lane s writes
// pick s and its weight exp(v_s - v_0) / sum, rounded once.  Returns pick
// `sub` on the lanes that hold one (live, sub < k), else -1.
__device__ __forceinline__ int route_softmax_group(const float* __restrict__ row,
                                                    const float* __restrict__ bias, int64_t E,
                                                    int64_t k, int G, int sub, bool live,
                                                    int32_t* __restrict__ idx_t,
                                                    float* __restrict__ w_t) {
    // experts of this lane: sub + G*j, j < per_lane (<= kMaxExperts / G)
    const int per_lane = static_cast<int>((E + G - 1) / G);
    uint32_t picked = 0;  // bit j: expert sub + G*j already selected (per_lane <= 32)
    float my_v = -INFINITY;
    int my_i = INT_MAX;
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
        if (sub == s) {
            my_v = bv;
            my_i = bi;
        }
    }
    const double top = static_cast<double>(__shfl(my_v, 0, G));
    const double ex = exp(static_cast<double>(my_v) - top);
    double sum = 0.0;
    for (int s = 0; s < k; ++s) sum += __shfl(ex, s, G);  // pick order, on every lane
    if (live && sub < k) {
        idx_t[sub] = my_i;
        w_t[sub] = static_cast<float>(ex / sum);
        return my_i;
    }
    return -1;
}

__global__ __launch_bounds__(256) void route_softmax_kernel(
        const float* __restrict__ logits, const float* __restrict__ bias,
        int64_t T, int64_t E, int64_t k, int G,
        int32_t* __restrict__ idx, float* __restrict__ w) {
    const int lane = threadIdx.x & 63;
    const int sub = lane & (G - 1);
    const int64_t t = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / G;
    const bool live = t < T;
    const int64_t tt = live ? t : 0;
    route_softmax_group(logits + tt * E, bias, E, k, G, sub, live, idx + tt * k, w + tt * k);
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

// Exclusive scan of counts[E * nb] in place by one workgroup of THREADS
// threads, then the per-expert offsets.
template <int THREADS>
__device__ void scan_counts(int32_t* __restrict__ counts, int64_t nb, int64_t E,
                            int32_t* __restrict__ offsets) {
    __shared__ int32_t wave_sums[THREADS / 64];
    __shared__ int32_t carry;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid == 0) carry = 0;
    __syncthreads();
    const int64_t n = E * nb;
    for (int64_t base = 0; base < n; base += THREADS) {
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
        if (tid == THREADS - 1) carry = before + incl;
        __syncthreads();
    }
    // offsets[e] = base of (e, block 0); offsets[E] = total pairs
    for (int64_t e = tid; e < E; e += THREADS) offsets[e] = nb > 0 ? counts[e * nb] : 0;
    if (tid == 0) offsets[E] = carry;
}

__global__ __launch_bounds__(1024) void perm_scan_kernel(
        int32_t* __restrict__ counts, int64_t nb, int64_t E,
        int32_t* __restrict__ offsets) {
    scan_counts<1024>(counts, nb, E, offsets);
}

// Routing and the per-block expert counts in one launch, as the reference's
// route_count routes each token and counts it in one launch
// (src/model.cu:921-942).  The routing keeps the standalone routers' full
// parallelism: a thread per token (PHI_QUANT) or a group of G lanes per
// token (SOFTMAX_TOPK), RC_THREADS threads per workgroup.  A workgroup's
// tokens fill one or more permutation blocks of kPermTokens, or part of one;
// it counts its picks per (permutation block, expert) in LDS and adds each
// non-zero count into counts[e][b], which the launch before this one (the
// gate) zeroed.  Nothing here waits for the other workgroups: the counts are
// read by the next launch (perm_place_scan_kernel), after this one ends.
template <int MODE, int RC_THREADS>
__global__ __launch_bounds__(RC_THREADS) void route_count_kernel(
        const float* __restrict__ logits, const float* __restrict__ bias, int64_t T,
        int64_t E, int64_t k, int G, float quantum, float tie_eps,
        int32_t* __restrict__ idx, float* __restrict__ w, int32_t* __restrict__ counts) {
    // tokens per workgroup: RC_THREADS (PHI_QUANT) or RC_THREADS / G, in pb
    // permutation blocks (RC_THREADS / kPermTokens for a thread per token,
    // 1 when a workgroup holds kPermTokens tokens or fewer)
    constexpr int PBMAX = RC_THREADS / kPermTokens;
    __shared__ int32_t hist[PBMAX * kMaxExperts];
    const int tid = threadIdx.x;
    const int64_t nb = (T + kPermTokens - 1) / kPermTokens;
    const int tpw = MODE == MOE_ROUTER_PHI_QUANT ? RC_THREADS : RC_THREADS / G;
    const int64_t tw = static_cast<int64_t>(blockIdx.x) * tpw;  // first token
    const int pb = tpw >= kPermTokens ? tpw / kPermTokens : 1;
    for (int i = tid; i < pb * E; i += RC_THREADS) hist[i] = 0;
    __syncthreads();
    if (MODE == MOE_ROUTER_PHI_QUANT) {
        const int64_t t = tw + tid;
        if (t < T) {
            int32_t picks[kMaxTopK];
            route_phi_token(logits + t * E, bias, E, k, quantum, tie_eps, idx + t * k,
                            w + t * k, picks);
            const int hb = tid / kPermTokens;
            for (int s = 0; s < k; ++s) {
                const int e = picks[s];
                if (e >= 0 && e < E) atomicAdd(&hist[hb * E + e], 1);
            }
        }
    } else {
        const int sub = (tid & 63) & (G - 1);
        const int64_t t = tw + tid / G;
        const bool live = t < T;
        const int64_t tt = live ? t : 0;
        // lane s of the group holds pick s: its count
        const int e = route_softmax_group(logits + tt * E, bias, E, k, G, sub, live,
                                          idx + tt * k, w + tt * k);
        if (e >= 0 && e < E) {
            const int hb = static_cast<int>((t - tw) / kPermTokens);
            atomicAdd(&hist[hb * E + e], 1);
        }
    }
    __syncthreads();
    const int64_t b0 = tw / kPermTokens;
    for (int i = tid; i < pb * E; i += RC_THREADS) {
        const int hb = i / static_cast<int>(E), e = i % static_cast<int>(E);
        if (hist[i] != 0 && b0 + hb < nb) atomicAdd(&counts[e * nb + b0 + hb], hist[i]);
    }
}

// perm_place with the scan folded in, for the layer: block b computes the
// bases it needs from the raw per-block counts (counts[e][b'] of every
// block, as route_count_kernel left them) -- for each expert the count of
// its pairs in blocks before b and in all blocks -- then the experts'
// offsets as an exclusive scan of those totals, so base(e, b) = offset(e) +
// pairs of e in blocks before b, the value perm_scan_kernel would have
// written.  Block 0 writes the offsets.  Each block reads all E * nb counts,
// so the layer takes this path only while E * nb is small (kPlaceScanMax).
__global__ __launch_bounds__(256) void perm_place_scan_kernel(
        const int32_t* __restrict__ idx, int64_t T, int64_t k, int64_t E,
        const int32_t* __restrict__ counts, int32_t* __restrict__ perm,
        int32_t* __restrict__ inv, int32_t* __restrict__ offsets) {
    __shared__ unsigned long long masks[kMaxExperts * 4];
    __shared__ int32_t before[kMaxExperts], base[kMaxExperts];
    __shared__ int32_t wave_sums[4];
    const int64_t b = blockIdx.x, nb = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int e = tid; e < E; e += 256) {
        before[e] = 0;
        base[e] = 0;
    }
    __syncthreads();
    // per expert: pairs in blocks before b (before[]), in all blocks (base[])
    for (int64_t i = tid; i < E * nb; i += 256) {
        const int c = counts[i];
        if (c == 0) continue;
        const int64_t e = i / nb;
        atomicAdd(&base[e], c);
        if (i - e * nb < b) atomicAdd(&before[e], c);
    }
    build_masks(idx, T, k, E, b * kPermTokens, masks);  // its barriers order the adds above
    // exclusive scan of the totals over the experts, 256 at a time
    int32_t carry = 0;
    for (int e0 = 0; e0 < E; e0 += 256) {
        const int e = e0 + tid;
        const int32_t v = e < E ? base[e] : 0;
        int32_t incl = v;
        for (int off = 1; off < 64; off <<= 1) {
            const int32_t o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        if (lane == 63) wave_sums[wv] = incl;
        __syncthreads();
        int32_t pre = carry;
        for (int j = 0; j < wv; ++j) pre += wave_sums[j];
        const int32_t chunk = wave_sums[0] + wave_sums[1] + wave_sums[2] + wave_sums[3];
        __syncthreads();
        if (e < E) {
            const int32_t off = pre + incl - v;
            if (b == 0) offsets[e] = off;
            base[e] = off + before[e];
        }
        carry += chunk;
    }
    if (b == 0 && tid == 0) offsets[E] = carry;
    __syncthreads();
    const int64_t t = b * kPermTokens + tid;
    if (tid < kPermTokens && t < T) {
        const int word = tid >> 6;
        const unsigned long long below = (1ull << (tid & 63)) - 1ull;
        for (int s = 0; s < k; ++s) {
            const int e = idx[t * k + s];
            if (e < 0 || e >= E) { inv[t * k + s] = -1; continue; }
            int rank = __popcll(masks[e * 4 + word] & below);
            for (int q = 0; q < word; ++q) rank += __popcll(masks[e * 4 + q]);
            const int32_t pos = base[e] + rank;
            perm[pos] = static_cast<int32_t>(t);
            inv[t * k + s] = pos;
        }
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



// A layer whose tokens fill one permutation block (T <= kPermTokens): the
// routing, the block's expert masks, the offsets and the placement in one
// workgroup -- route_count_kernel and perm_place_scan_kernel as one launch,
// each pick kept in LDS instead of passing through the block counts in
// global memory.  The picks, weights, offsets and positions are those of the
// two launches: position = the expert's offset + the rank of the token among
// the expert's tokens (ascending token order, the reference's
// assignments[e], src/layer.cu:86-92).  SOFTMAX_TOPK routes THREADS / G
// tokens per round (the layer takes this path for at most two rounds).
template <int MODE, int THREADS>
__global__ __launch_bounds__(THREADS) void route_place_one_kernel(
        const float* __restrict__ logits, const float* __restrict__ bias, int64_t T,
        int64_t E, int64_t k, int G, float quantum, float tie_eps,
        int32_t* __restrict__ idx, float* __restrict__ w, int32_t* __restrict__ perm,
        int32_t* __restrict__ inv, int32_t* __restrict__ offsets) {
    constexpr int NW = THREADS / 64;
    __shared__ unsigned long long masks[kMaxExperts * 4];
    __shared__ int32_t picks[kPermTokens * kMaxTopK];
    __shared__ int32_t base[kMaxExperts];
    __shared__ int32_t wave_sums[NW];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid; i < E * 4; i += THREADS) masks[i] = 0ull;
    __syncthreads();
    // pick s of token t (t < kPermTokens): kept, and its token's bit set
    auto mark = [&](int64_t t, int64_t s, int e) {
        picks[t * k + s] = e;
        if (e >= 0 && e < E) atomicOr(&masks[e * 4 + (t >> 6)], 1ull << (t & 63));
    };
    if (MODE == MOE_ROUTER_PHI_QUANT) {
        for (int64_t t = tid; t < T; t += THREADS) {
            int32_t p[kMaxTopK];
            route_phi_token(logits + t * E, bias, E, k, quantum, tie_eps, idx + t * k,
                            w + t * k, p);
            for (int64_t s2 = 0; s2 < k; ++s2) mark(t, s2, p[s2]);
        }
    } else {
        const int sub = lane & (G - 1);
        const int per = THREADS / G;  // tokens per round
        for (int64_t t0 = 0; t0 < T; t0 += per) {  // every lane calls the group routine
            const int64_t t = t0 + tid / G;
            const bool live = t < T;
            const int64_t tt = live ? t : 0;
            const int e = route_softmax_group(logits + tt * E, bias, E, k, G, sub, live,
                                              idx + tt * k, w + tt * k);
            if (live && sub < k) mark(t, sub, e);
        }
    }
    __syncthreads();
    // offsets: exclusive scan of the experts' pair counts, THREADS at a time
    int32_t carry = 0;
    for (int64_t e0 = 0; e0 < E; e0 += THREADS) {
        const int64_t e = e0 + tid;
        const int32_t v = e < E ? __popcll(masks[e * 4]) + __popcll(masks[e * 4 + 1]) +
                                      __popcll(masks[e * 4 + 2]) + __popcll(masks[e * 4 + 3])
                                : 0;
        int32_t incl = v;
        for (int off = 1; off < 64; off <<= 1) {
            const int32_t o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        if (lane == 63) wave_sums[wv] = incl;
        __syncthreads();
        int32_t pre = carry, chunk = 0;
        for (int j = 0; j < NW; ++j) {
            if (j < wv) pre += wave_sums[j];
            chunk += wave_sums[j];
        }
        __syncthreads();
        if (e < E) {
            offsets[e] = pre + incl - v;
            base[e] = pre + incl - v;
        }
        carry += chunk;
    }
    if (tid == 0) offsets[E] = carry;
    __syncthreads();
    for (int64_t i = tid; i < T * k; i += THREADS) {
        const int64_t t = i / k;
        const int e = picks[i];
        if (e < 0 || e >= E) {
            inv[i] = -1;
            continue;
        }
        const int word = static_cast<int>(t >> 6);
        int rank = __popcll(masks[e * 4 + word] & ((1ull << (t & 63)) - 1ull));
        for (int q = 0; q < word; ++q) rank += __popcll(masks[e * 4 + q]);
        const int32_t pos = base[e] + rank;
        perm[pos] = static_cast<int32_t>(t);
        inv[i] = pos;
    }
}

// -------------------------------------------------------------- combine
// One workgroup per token.  The token's slots are ordered by ascending
// expert (ties by slot), then y = 0 + w*row, + w*row, ... in that order: the
// order of the reference's expert loop (src/layer.cu:93-101).  resid, when
// given, is added last (the decoder's add_inplace, src/layer.cu:160).  When
// the w2 GEMM ran split-K, a row is the sum of its PARTS partial rows, added
// in part order before weighting.  Threads 0..k-1 load one slot each (expert,
// packed row, weight: independent loads, one latency) and place it at its
// rank among the token's live slots -- the order a sequential selection by
// (expert, slot) would give.
template <int CONTRACT, int PARTS>
__global__ __launch_bounds__(256) void combine_kernel(
        const float* __restrict__ out_rows, const int32_t* __restrict__ idx,
        const float* __restrict__ wts, const int32_t* __restrict__ inv,
        const float* __restrict__ resid, float* __restrict__ y, int64_t T,
        int64_t k, int64_t d, int64_t rows_total, int64_t part_stride) {
    __shared__ int32_t slot_e[kMaxTopK];
    __shared__ int32_t slot_live[kMaxTopK];
    __shared__ int32_t order_row[kMaxTopK];
    __shared__ float order_w[kMaxTopK];
    __shared__ int n_live;
    const int64_t t = blockIdx.x;
    const int s = threadIdx.x;
    int32_t my_e = 0, my_r = 0;
    float my_w = 0.0f;
    bool live = false;
    if (s < k) {
        my_e = idx[t * k + s];
        my_r = inv[t * k + s];
        my_w = wts[t * k + s];
        live = my_r >= 0 && my_r < rows_total;
        slot_e[s] = my_e;
        slot_live[s] = live ? 1 : 0;
    }
    __syncthreads();
    if (s < k) {
        int rank = 0, n = 0;
        for (int q = 0; q < k; ++q) {
            if (!slot_live[q]) continue;
            ++n;
            const int e = slot_e[q];
            rank += (e < my_e || (e == my_e && q < s)) ? 1 : 0;
        }
        if (live) {
            order_row[rank] = my_r;
            order_w[rank] = my_w;
        }
        if (s == 0) n_live = n;
    }
    __syncthreads();
    const int n = n_live;
    const bool vec = (d & 3) == 0;
    if (vec) {
        // JU 16-byte columns per thread at once, 256 apart, and for the
        // common two live slots both rows' loads (and the residual's) before
        // any use: every load of a thread is in flight together (one memory
        // latency per workgroup instead of one per column and slot)
        typedef float f4 __attribute__((ext_vector_type(4)));
        constexpr int JU = 4;
        const int64_t d4 = d >> 2;
        auto row4 = [&](int q, int64_t j) __attribute__((always_inline)) -> f4 {
            f4 v = reinterpret_cast<const f4*>(out_rows + order_row[q] * d)[j];
#pragma unroll
            for (int p = 1; p < PARTS; ++p) {
                const f4 u = reinterpret_cast<const f4*>(out_rows + p * part_stride + order_row[q] * d)[j];
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = v[c] + u[c];
            }
            return v;
        };
        const f4 zero = {0.f, 0.f, 0.f, 0.f};
        for (int64_t j0 = threadIdx.x; j0 < d4; j0 += int64_t(blockDim.x) * JU) {
            f4 acc[JU], rv[JU];
#pragma unroll
            for (int u = 0; u < JU; ++u) {
                const int64_t j = j0 + int64_t(u) * blockDim.x;
                acc[u] = zero;
                rv[u] = (resid != nullptr && j < d4) ? reinterpret_cast<const f4*>(resid + t * d)[j] : zero;
            }
            if (n == 2) {
                f4 v0[JU], v1[JU];
#pragma unroll
                for (int u = 0; u < JU; ++u) {
                    const int64_t j = j0 + int64_t(u) * blockDim.x;
                    v0[u] = j < d4 ? row4(0, j) : zero;
                    v1[u] = j < d4 ? row4(1, j) : zero;
                }
                const float w0 = order_w[0], w1 = order_w[1];
#pragma unroll
                for (int u = 0; u < JU; ++u)
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        acc[u][c] = mac<CONTRACT>(acc[u][c], w0, v0[u][c]);
                        acc[u][c] = mac<CONTRACT>(acc[u][c], w1, v1[u][c]);
                    }
            } else {
                for (int q = 0; q < n; ++q) {
                    f4 v[JU];
#pragma unroll
                    for (int u = 0; u < JU; ++u) {
                        const int64_t j = j0 + int64_t(u) * blockDim.x;
                        v[u] = j < d4 ? row4(q, j) : zero;
                    }
                    const float wq = order_w[q];
#pragma unroll
                    for (int u = 0; u < JU; ++u)
#pragma unroll
                        for (int c = 0; c < 4; ++c) acc[u][c] = mac<CONTRACT>(acc[u][c], wq, v[u][c]);
                }
            }
#pragma unroll
            for (int u = 0; u < JU; ++u) {
                const int64_t j = j0 + int64_t(u) * blockDim.x;
                if (j >= d4) continue;
                if (resid != nullptr)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[u][c] = acc[u][c] + rv[u][c];
                reinterpret_cast<f4*>(y + t * d)[j] = acc[u];
            }
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
                        hipStream_t s, uint32_t* zero, int64_t nzero) {
    if (T == 0 || E == 0) return;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    // The ring form for E <= 8 (16 token rows x 4 experts or 8 x 8 per wave).
    // At E = 16 a wave would hold 4 tokens and stream 16 expert rows for
    // them -- 4x the token bytes (measured 2.4x slower at the reference's
    // layer shape) -- so E of 9-16 takes the workgroup ring below, whose 16
    // expert rows serve 16 tokens.
    if (E <= 8 && d % 4 == 0 && d >= 4 && al(x) && al(w) && d * 16 * 4 < (int64_t(1) << 31)) {
        const int eb = E <= 4 ? 4 : 8;
        const dim3 grid(static_cast<unsigned>(ceil_div(T, 64 / eb)));
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(64), 0, s, x, w, logits, T, d, E, zero, nzero);
        };
        switch (eb * 2 + (contract ? 1 : 0)) {
            case 8: go(gate_ring_kernel<0, 4>); break;
            case 9: go(gate_ring_kernel<1, 4>); break;
            case 16: go(gate_ring_kernel<0, 8>); break;
            default: go(gate_ring_kernel<1, 8>); break;
        }
        return;
    }
    // A few tokens over 9-64 experts: the per-wave ring above with 4 experts
    // per wave and E / 4 expert blocks over grid.y, so that many waves
    // stream the expert rows at once (the workgroup ring below runs every
    // expert of a 16-token block in one workgroup, bound by its stages'
    // round trips while the grid is small); the 16 token rows a wave holds
    // are re-read once per expert block, which only pays while they are few.
    if (E > 8 && E <= 64 && T * E <= kGateFewLogits && d % 4 == 0 && d >= 4 && al(x) && al(w) &&
        d * 16 * 4 < (int64_t(1) << 31)) {
        const dim3 grid(static_cast<unsigned>(ceil_div(T, 16)), static_cast<unsigned>(ceil_div(E, 4)));
        if (contract)
            hipLaunchKernelGGL((gate_ring_kernel<1, 4>), grid, dim3(64), 0, s, x, w, logits, T, d, E,
                               zero, nzero);
        else
            hipLaunchKernelGGL((gate_ring_kernel<0, 4>), grid, dim3(64), 0, s, x, w, logits, T, d, E,
                               zero, nzero);
        return;
    }
    int eb = 8;
    while (eb < E && eb < 64) eb <<= 1;
    // E of 9-16: the workgroup ring, when rows are 16-byte aligned and every
    // load offset (16 token or expert rows) fits 31 bits
    if (eb == 16 && d % 4 == 0 && d >= 4 && al(x) && al(w) && d * 16 * 4 < (int64_t(1) << 31)) {
        const dim3 grid(static_cast<unsigned>(ceil_div(T, 16)), static_cast<unsigned>(ceil_div(E, 16)));
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, x, w, logits, T, d, E, zero,
                               nzero);
        };
        if (contract) go(gate_wg_ring_kernel<1, 16, 1, 3, 4>);
        else go(gate_wg_ring_kernel<0, 16, 1, 3, 4>);
        return;
    }
    // 4 tokens per thread from 32 experts up (small E keeps one output per
    // thread: its rows per workgroup are already many, and the grid stays
    // wide), and at 64-expert blocks 2 or 4 experts per thread as well: 4
    // where that still leaves 512 workgroups or more.  Measured on MI355X
    // (us, 1 / 2 / 4 experts per thread): config 4's 16,384 x 2048 x 64
    // 189.5 / 100.2 / 137.6; 4096 x 4096 x 64 182.1 / 171.1 / 265.9;
    // 16,384 x 2048 x 100 (two expert blocks) 300.3 / 182.5 / 146.8.
    const int tb = eb >= 32 ? 4 : 1;
    const int te = eb < 64 ? 1 : (ceil_div(T, 64) * ceil_div(E, 64) >= 512 ? 4 : 2);
    const dim3 grid(static_cast<unsigned>(ceil_div(T, tb * (256 / (eb / te)))),
                    static_cast<unsigned>(ceil_div(E, eb)));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, x, w, logits, T, d, E, zero, nzero);
    };
    switch (eb * 2 + (contract ? 1 : 0)) {
        case 16: go(gate_logits_kernel<0, 8, 1>); break;
        case 17: go(gate_logits_kernel<1, 8, 1>); break;
        case 32: go(gate_logits_kernel<0, 16, 1>); break;
        case 33: go(gate_logits_kernel<1, 16, 1>); break;
        case 64: go(gate_logits_kernel<0, 32, 4>); break;
        case 65: go(gate_logits_kernel<1, 32, 4>); break;
        case 128:
            if (te == 4) go(gate_logits_kernel<0, 64, 4, 4>);
            else go(gate_logits_kernel<0, 64, 4, 2>);
            break;
        default:
            if (te == 4) go(gate_logits_kernel<1, 64, 4, 4>);
            else go(gate_logits_kernel<1, 64, 4, 2>);
            break;
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

void launch_route_count(const float* logits, const float* bias, int64_t T, int64_t E,
                        int64_t k, int mode, float quantum, float tie_eps, int32_t* idx,
                        float* w, int32_t* counts, hipStream_t s) {
    if (T == 0) return;
    int G = 1;
    while (G < E && G < 64) G <<= 1;
    // Threads per workgroup, measured on MI355X (HIP events, us, 256 / 1024
    // threads): PHI_QUANT at the reference's 15,583 x 16 11.5 / 18.7 (a
    // thread per token: the smaller workgroups spread the sequential selects
    // over 4x the CUs); SOFTMAX_TOPK at config 3 8.8 / 8.0, config 5 8.8 /
    // 8.0, config 4 (64 experts, top-8) 48.4 / 37.9.
    const int threads = mode == MOE_ROUTER_PHI_QUANT ? 256 : 1024;
    const int64_t tpw = mode == MOE_ROUTER_PHI_QUANT ? threads : threads / G;
    const dim3 grid(static_cast<unsigned>(ceil_div(T, tpw)));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(threads), 0, s, logits, bias, T, E, k, G,
                           quantum, tie_eps, idx, w, counts);
    };
    if (mode == MOE_ROUTER_PHI_QUANT) go(route_count_kernel<MOE_ROUTER_PHI_QUANT, 256>);
    else go(route_count_kernel<MOE_ROUTER_SOFTMAX_TOPK, 1024>);
}

void launch_perm_place_scan(const int32_t* idx, int64_t T, int64_t k, int64_t E,
                            const int32_t* counts, int32_t* perm, int32_t* inv,
                            int32_t* offsets, hipStream_t s) {
    const int64_t nb = ceil_div(T, kPermTokens);
    if (nb == 0) return;
    hipLaunchKernelGGL(perm_place_scan_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s,
                       idx, T, k, E, counts, perm, inv, offsets);
}

bool route_place_one_fits(int64_t T, int64_t E, int64_t k, int mode) {
    if (T <= 0 || T > kPermTokens || k < 1 || k > kMaxTopK || E < 1 || E > kMaxExperts)
        return false;
    if (mode == MOE_ROUTER_PHI_QUANT) return true;
    // each round of the softmax router is one token per G-lane group; past two
    // rounds the two-launch path's parallel workgroups are faster
    int64_t G = 1;
    while (G < E && G < 64) G <<= 1;
    return T * G <= 2 * 1024;
}

void launch_route_place_one(const float* logits, const float* bias, int64_t T, int64_t E,
                            int64_t k, int mode, float quantum, float tie_eps, int32_t* idx,
                            float* w, int32_t* perm, int32_t* inv, int32_t* offsets,
                            hipStream_t s) {
    if (!route_place_one_fits(T, E, k, mode)) throw Unsupported("one-block routing shape");
    int G = 1;
    while (G < E && G < 64) G <<= 1;
    if (mode == MOE_ROUTER_PHI_QUANT)
        hipLaunchKernelGGL((route_place_one_kernel<MOE_ROUTER_PHI_QUANT, 256>), dim3(1), dim3(256),
                           0, s, logits, bias, T, E, k, G, quantum, tie_eps, idx, w, perm, inv,
                           offsets);
    else
        hipLaunchKernelGGL((route_place_one_kernel<MOE_ROUTER_SOFTMAX_TOPK, 1024>), dim3(1),
                           dim3(1024), 0, s, logits, bias, T, E, k, G, quantum, tie_eps, idx, w,
                           perm, inv, offsets);
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
