// The decoder pieces around the MoE block (config 5's prefill): rotary
// position embedding, the masked softmax of causal attention, the residual
// and bias adds, and the embedding gather.  The attention's two products
// (Q K^T and P V) run on the GEMM engine as batched launches over
// (sequence, head); this file holds the elementwise and row-wise steps.
#include "common.hpp"

#include <cmath>

namespace moe {
namespace {

// tensor_ops::apply_rope (src/tensor.cu:191-210) with the cos/sin of every
// (position, pair) read from a table built on the host by libm (as the
// reference's GPU path does, src/model.cu:1784-1798 and rope_rows
// :1046-1083): pair (j, j + half) of every head becomes (x0 c - x1 s,
// x1 c + x0 s), each product rounded on its own (this file is built without
// contraction).  One thread per pair; row r is at position
// first_pos + r % seq_len.
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ q, float* __restrict__ k,
                                                   const float* __restrict__ table, int64_t rows,
                                                   int64_t seq_len, int64_t first_pos,
                                                   int64_t q_heads, int64_t kv_heads,
                                                   int64_t head_dim) {
    const int64_t half = head_dim / 2, heads = q_heads + kv_heads;
    const int64_t n = rows * heads * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        const int64_t j = i % half, hh = (i / half) % heads, r = i / (half * heads);
        float* x = hh < q_heads ? q + r * q_heads * head_dim + hh * head_dim
                                : k + r * kv_heads * head_dim + (hh - q_heads) * head_dim;
        const float* trig = table + ((first_pos + r % seq_len) * half + j) * 2;
        const float c = trig[0], sn = trig[1];
        const float x0 = x[j], x1 = x[j + half];
        x[j] = x0 * c - x1 * sn;
        x[j + half] = x1 * c + x0 * sn;
    }
}

// The same rotation, 4 adjacent pairs per thread with 16-byte loads and
// stores, and 32-bit index arithmetic (the launcher takes it when
// head_dim % 8 == 0, the buffers are 16-byte aligned and the pair count /
// 4 fits 31 bits): each element's two products and sum are the ones above,
// so the results are bit-identical.  ROWS: positions[r] clamped into the
// table (rope_rows_kernel); else first_pos + r % seq_len (rope_kernel).
template <bool ROWS>
__global__ __launch_bounds__(256) void rope4_kernel(float* __restrict__ q, float* __restrict__ k,
                                                    const float* __restrict__ table,
                                                    int64_t table_positions,
                                                    const int32_t* __restrict__ positions,
                                                    uint32_t seq_len, int64_t first_pos,
                                                    uint32_t rows, uint32_t q_heads,
                                                    uint32_t kv_heads, uint32_t head_dim) {
    const uint32_t half = head_dim / 2, h4 = half / 4, heads = q_heads + kv_heads;
    const uint32_t n4 = rows * heads * h4;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const uint32_t t = i / h4, j = 4 * (i - t * h4);
        const uint32_t r = t / heads, hh = t - r * heads;
        float* x = hh < q_heads ? q + (static_cast<int64_t>(r) * q_heads + hh) * head_dim
                                : k + (static_cast<int64_t>(r) * kv_heads + (hh - q_heads)) * head_dim;
        int64_t pos;
        if (ROWS) {
            pos = positions[r];
            pos = pos < 0 ? 0 : (pos >= table_positions ? table_positions - 1 : pos);
        } else {
            pos = first_pos + r % seq_len;
        }
        const float4* trig = reinterpret_cast<const float4*>(table + (pos * half + j) * 2);
        const float4 t01 = trig[0], t23 = trig[1];  // (cos, sin) of pairs j .. j + 3
        const float4 a = *reinterpret_cast<const float4*>(x + j);
        const float4 b = *reinterpret_cast<const float4*>(x + j + half);
        const float c[4] = {t01.x, t01.z, t23.x, t23.z}, sn[4] = {t01.y, t01.w, t23.y, t23.w};
        const float x0[4] = {a.x, a.y, a.z, a.w}, x1[4] = {b.x, b.y, b.z, b.w};
        float y0[4], y1[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            y0[u] = x0[u] * c[u] - x1[u] * sn[u];
            y1[u] = x1[u] * c[u] + x0[u] * sn[u];
        }
        *reinterpret_cast<float4*>(x + j) = float4{y0[0], y0[1], y0[2], y0[3]};
        *reinterpret_cast<float4*>(x + j + half) = float4{y1[0], y1[1], y1[2], y1[3]};
    }
}

bool rope4_ok(const float* q, const float* k, const float* table, int64_t rows, int64_t heads,
              int64_t head_dim) {
    auto al = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return head_dim % 8 == 0 && al(q) && al(k) && al(table) &&
           rows * heads * (head_dim / 8) < (int64_t(1) << 31) && rows < (int64_t(1) << 31);
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// The softmax of PhiAttention::forward (src/layer.cu:118-140) on one score
// row per wave: scaled = score / sqrt(head_dim) over the visible keys
// (ki <= qi, qi - ki < window), m = max, p = exp(scaled - m) / sum, with the
// reference's accurate_exp (double exp, one rounding); invisible keys get 0.
// The row's score entries past the diagonal were never written (the score
// GEMM skips those tiles) and are not read.
__global__ __launch_bounds__(256) void attn_softmax_kernel(float* __restrict__ scores,
                                                           int64_t rows_total, int64_t S,
                                                           float scale, int64_t window) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows_total) return;  // wave-uniform
    const int64_t qi = row % S;
    const int64_t lo = window > 0 && qi - window + 1 > 0 ? qi - window + 1 : 0;
    float* p = scores + row * S;
    float m = -INFINITY;
    for (int64_t ki = lo + lane; ki <= qi; ki += 64) m = fmaxf(m, p[ki] / scale);
    m = wave_max(m);
    float den = 0.0f;
    for (int64_t ki = lo + lane; ki <= qi; ki += 64)
        den += static_cast<float>(exp(static_cast<double>(p[ki] / scale - m)));
    den = wave_sum(den);
    for (int64_t ki = lane; ki < S; ki += 64) {
        const bool vis = ki >= lo && ki <= qi;
        p[ki] = vis ? static_cast<float>(exp(static_cast<double>(p[ki] / scale - m))) / den : 0.0f;
    }
}

// Attention of the last position of every sequence (the rows the model's
// logits read): one workgroup per (sequence b, query head h), q row b of
// [batch, q_heads*hd] against keys [lo, S) of sequence b, lo = S - window
// (window > 0) or 0.  Every sum runs in the oracle's order -- the score's
// d-ascending chain per thread, the denominator ki-ascending on one thread,
// each output value ki-ascending on its own thread -- so given the same
// inputs the result is bit-identical to the reference's loop
// (src/layer.cu:117-140).  The row's scores live in LDS when they fit
// (LDS_ROW: S <= kAttnLastLds), else in `scores` (batch*q_heads*S floats).
constexpr int kAttnLastLds = 8192;
template <bool VEC4, bool LDS_ROW>
__global__ __launch_bounds__(256) void attn_last_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, float* __restrict__ scores, int64_t S, int64_t H, int64_t KVH,
    int64_t hd, int64_t window, float scale) {
    __shared__ float red[4];
    __shared__ float row[LDS_ROW ? kAttnLastLds : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t b = blockIdx.x / H, h = blockIdx.x % H, kh = h / (H / KVH);
    const int64_t kw = KVH * hd;
    const float* qr = q + b * H * hd + h * hd;
    const float* kb = k + b * S * kw + kh * hd;
    const float* vb = v + b * S * kw + kh * hd;
    float* sc = LDS_ROW ? row : scores + static_cast<int64_t>(blockIdx.x) * S;
    const int64_t lo = window > 0 && S > window ? S - window : 0;
    float m = -INFINITY;
    for (int64_t ki = lo + tid; ki < S; ki += blockDim.x) {
        const float* kr = kb + ki * kw;
        float acc = 0.0f;
        if (VEC4) {
            for (int64_t d = 0; d < hd; d += 4) {
                const float4 a = *reinterpret_cast<const float4*>(qr + d);
                const float4 c = *reinterpret_cast<const float4*>(kr + d);
                acc += a.x * c.x;
                acc += a.y * c.y;
                acc += a.z * c.z;
                acc += a.w * c.w;
            }
        } else {
            for (int64_t d = 0; d < hd; ++d) acc += qr[d] * kr[d];
        }
        const float sv = acc / scale;
        sc[ki] = sv;
        m = fmaxf(m, sv);
    }
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int64_t ki = lo + tid; ki < S; ki += blockDim.x)
        sc[ki] = static_cast<float>(exp(static_cast<double>(sc[ki] - m)));
    __syncthreads();  // the weights of every thread, before the ordered sum
    if (tid == 0) {
        float den = 0.0f;
#pragma unroll 8
        for (int64_t ki = lo; ki < S; ++ki) den += sc[ki];
        red[0] = den;
    }
    __syncthreads();
    const float den = red[0];
    // each weight divided once (the same operands and rounding as dividing
    // in every output chain that uses it)
    for (int64_t ki = lo + tid; ki < S; ki += blockDim.x) sc[ki] = sc[ki] / den;
    __syncthreads();
    float* o = out + b * H * hd + h * hd;
    for (int64_t d = tid; d < hd; d += blockDim.x) {
        float value = 0.0f;
#pragma unroll 8
        for (int64_t ki = lo; ki < S; ++ki) value += sc[ki] * vb[ki * kw + d];
        o[d] = value;
    }
}

// RoPE with an explicit position per row (the depth of a prefix-trie node,
// src/model.cu:1046-1083 with `pos`): row r at positions[r], clamped into
// the table so that a bad position cannot read past it.
__global__ __launch_bounds__(256) void rope_rows_kernel(float* __restrict__ q,
                                                        float* __restrict__ k,
                                                        const float* __restrict__ table,
                                                        int64_t table_positions,
                                                        const int32_t* __restrict__ positions,
                                                        int64_t rows, int64_t q_heads,
                                                        int64_t kv_heads, int64_t head_dim) {
    const int64_t half = head_dim / 2, heads = q_heads + kv_heads;
    const int64_t n = rows * heads * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        const int64_t j = i % half, hh = (i / half) % heads, r = i / (half * heads);
        float* x = hh < q_heads ? q + r * q_heads * head_dim + hh * head_dim
                                : k + r * kv_heads * head_dim + (hh - q_heads) * head_dim;
        int64_t pos = positions[r];
        pos = pos < 0 ? 0 : (pos >= table_positions ? table_positions - 1 : pos);
        const float* trig = table + (pos * half + j) * 2;
        const float c = trig[0], sn = trig[1];
        const float x0 = x[j], x1 = x[j + half];
        x[j] = x0 * c - x1 * sn;
        x[j + half] = x1 * c + x0 * sn;
    }
}

// Attention of query row i over an explicit key list: key rows
// key_rows[key_beg[i] .. key_end[i]) of k and v, ascending positions ending
// at the query's own (a prefix-trie node's root path, src/model.cu:1667-1680;
// attention_heads :1161-1283), of which the last `window` are visible
// (window > 0).  One workgroup per (query, head); every sum in the
// reference loop's order, as attn_last_kernel: bit-identical to it given the
// same inputs.  Key indices are clamped into [0, kv_rows).  The scores live
// in LDS when the list fits (LDS_ROW), else in `scores` at key_beg[i] * H +
// h * len.
template <bool VEC4, bool LDS_ROW>
__global__ __launch_bounds__(256) void attn_paths_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, float* __restrict__ scores, const int32_t* __restrict__ key_rows,
    const int32_t* __restrict__ key_beg, const int32_t* __restrict__ key_end, int64_t kv_rows,
    int64_t key_total, int64_t scores_floats, int64_t H, int64_t KVH, int64_t hd, int64_t window,
    float scale) {
    __shared__ float red[4];
    __shared__ float row[LDS_ROW ? kAttnLastLds : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t i = blockIdx.x / H, h = blockIdx.x % H, kh = h / (H / KVH);
    const int64_t kw = KVH * hd;
    const float* qr = q + i * H * hd + h * hd;
    int64_t beg = key_beg[i];
    const int64_t end = key_end[i];
    if (window > 0 && end - beg > window) beg = end - window;
    const int64_t len = end > beg ? end - beg : 0;
    float* sc = LDS_ROW ? row : scores + static_cast<int64_t>(key_beg[i]) * H + h * len;
    float* o = out + i * H * hd + h * hd;
    if (len == 0) {  // an empty key list (not a trie path): zeros
        for (int64_t d = tid; d < hd; d += blockDim.x) o[d] = 0.0f;
        return;
    }
    // a list outside key_rows, or longer than the caller's bound (it would
    // overrun the score row): NaN output instead (block-uniform)
    const bool fits = key_beg[i] >= 0 && end <= key_total &&
                      (LDS_ROW ? len <= kAttnLastLds
                               : static_cast<int64_t>(key_beg[i]) * H + (h + 1) * len <=
                                     scores_floats);
    if (!fits) {
        for (int64_t d = tid; d < hd; d += blockDim.x) o[d] = NAN;
        return;
    }
    auto key_row = [&](int64_t t) {
        int64_t r = key_rows[beg + t];
        return r < 0 ? 0 : (r >= kv_rows ? kv_rows - 1 : r);
    };
    float m = -INFINITY;
    for (int64_t t = tid; t < len; t += blockDim.x) {
        const float* kr = k + key_row(t) * kw + kh * hd;
        float acc = 0.0f;
        if (VEC4) {
            for (int64_t d = 0; d < hd; d += 4) {
                const float4 a = *reinterpret_cast<const float4*>(qr + d);
                const float4 c = *reinterpret_cast<const float4*>(kr + d);
                acc += a.x * c.x;
                acc += a.y * c.y;
                acc += a.z * c.z;
                acc += a.w * c.w;
            }
        } else {
            for (int64_t d = 0; d < hd; ++d) acc += qr[d] * kr[d];
        }
        const float sv = acc / scale;
        sc[t] = sv;
        m = fmaxf(m, sv);
    }
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int64_t t = tid; t < len; t += blockDim.x)
        sc[t] = static_cast<float>(exp(static_cast<double>(sc[t] - m)));
    __syncthreads();
    if (tid == 0) {
        float den = 0.0f;
#pragma unroll 8
        for (int64_t t = 0; t < len; ++t) den += sc[t];
        red[0] = den;
    }
    __syncthreads();
    const float den = red[0];
    // each weight divided once (as in attn_last_kernel)
    for (int64_t t = tid; t < len; t += blockDim.x) sc[t] = sc[t] / den;
    __syncthreads();
    for (int64_t d = tid; d < hd; d += blockDim.x) {
        float value = 0.0f;
#pragma unroll 8
        for (int64_t t = 0; t < len; ++t) value += sc[t] * v[key_row(t) * kw + kh * hd + d];
        o[d] = value;
    }
}

// The same attention for lists of up to 64 keys (prefix-trie paths are
// short: the reference's contest sequences are 10-29 tokens), one wave per
// (query, key head), all G query heads of that key head at once: lane t owns
// key t's G scores (each the same d-ascending chain as above, the key row
// read once for the G heads), the max is a wave reduction, every lane runs
// the denominator's t-ascending chain from shuffled weights, and each output
// value's t-ascending chain runs on the lane of its column -- the order of
// attn_paths_kernel, so the results are bit-identical to it, on 1/4 of the
// threads with no barrier (one workgroup of 256 per (query, head) left most
// of its lanes idle: the reference's model shape spent 2.2 ms per layer
// there).  head_dim a multiple of 4, at most 256; 16-byte aligned q and k.
template <int G>
__global__ __launch_bounds__(256) void attn_paths_wave_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, const int32_t* __restrict__ key_rows,
    const int32_t* __restrict__ key_beg, const int32_t* __restrict__ key_end, int64_t nq,
    int64_t kv_rows, int64_t key_total, int64_t KVH, int64_t hd, int64_t window, float scale) {
    const int lane = threadIdx.x & 63;
    // the wave's (query, key head), wave-uniform by construction: readfirstlane
    // lets the compiler see that, so q (the same for every lane) is read
    // through scalar loads and fed to the chains as scalar operands instead of
    // 64 lanes' vector loads of one address
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if (gw >= nq * KVH) return;  // no barrier in this kernel
    const int64_t i = gw / KVH, kh = gw % KVH, H = KVH * G;
    const int64_t kw = KVH * hd;
    int64_t beg = key_beg[i];
    const int64_t end = key_end[i];
    if (window > 0 && end - beg > window) beg = end - window;
    const int64_t len = end > beg ? end - beg : 0;
    float* o = out + i * H * hd + kh * G * hd;  // G heads side by side
    if (len == 0) {
        for (int64_t d = lane; d < G * hd; d += 64) o[d] = 0.0f;
        return;
    }
    if (!(key_beg[i] >= 0 && end <= key_total && len <= 64)) {
        for (int64_t d = lane; d < G * hd; d += 64) o[d] = NAN;
        return;
    }
    const float* qi = q + i * H * hd + kh * G * hd;
    int64_t my_row = 0;
    float sc[G];
    if (lane < len) {
        int64_t r = key_rows[beg + lane];
        my_row = r < 0 ? 0 : (r >= kv_rows ? kv_rows - 1 : r);
        const float* kr = k + my_row * kw + kh * hd;
        float acc[G];
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g] = 0.0f;
        // 32 columns of the key row at a time, all 8 loads issued before
        // the chain consumes them (one memory round trip per chunk)
        for (int64_t d0 = 0; d0 < hd; d0 += 32) {
            float4 c[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                c[u] = d0 + 4 * u < hd ? *reinterpret_cast<const float4*>(kr + d0 + 4 * u)
                                       : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (d0 + 4 * u >= hd) break;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float4 a = *reinterpret_cast<const float4*>(qi + g * hd + d0 + 4 * u);
                    acc[g] += a.x * c[u].x;
                    acc[g] += a.y * c[u].y;
                    acc[g] += a.z * c[u].z;
                    acc[g] += a.w * c[u].w;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g] = acc[g] / scale;
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g] = -INFINITY;
    }
    float den[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float m = wave_max(sc[g]);
        sc[g] = lane < len ? static_cast<float>(exp(static_cast<double>(sc[g] - m))) : 0.0f;
        float dsum = 0.0f;
        for (int64_t t = 0; t < len; ++t) dsum += __shfl(sc[g], static_cast<int>(t), 64);
        den[g] = dsum;
    }
    // key t's weight exp_t / den, divided once on its own lane (the same
    // operands and rounding as dividing on every lane that uses it)
    float pw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) pw[g] = sc[g] / den[g];
    // output columns d = d0 + lane and d0 + 64 + lane together; the value
    // rows of 16 keys at a time are loaded before their t-ascending chains
    // consume them (one memory round trip per 16 keys, not per key)
    for (int64_t d0 = 0; d0 < hd; d0 += 128) {
        const int64_t da = d0 + lane, db = d0 + 64 + lane;
        const bool ina = da < hd, inb = db < hd;
        float va[G], vb[G];
#pragma unroll
        for (int g = 0; g < G; ++g) va[g] = vb[g] = 0.0f;
        for (int64_t t0 = 0; t0 < len; t0 += 16) {
            float xa[16], xb[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int64_t t = t0 + u < len ? t0 + u : t0;  // wave-uniform
                const float* vr = v + __shfl(my_row, static_cast<int>(t), 64) * kw + kh * hd;
                xa[u] = ina ? vr[da] : 0.0f;
                xb[u] = inb ? vr[db] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (t0 + u >= len) break;  // wave-uniform
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float pr = __shfl(pw[g], static_cast<int>(t0 + u), 64);
                    va[g] += pr * xa[u];
                    vb[g] += pr * xb[u];
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (ina) o[g * hd + da] = va[g];
            if (inb) o[g * hd + db] = vb[g];
        }
    }
}

__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ a, const float* __restrict__ b,
                                                  int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        a[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void add_bias_kernel(float* __restrict__ a,
                                                       const float* __restrict__ bias,
                                                       int64_t n, int64_t cols) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        a[i] = a[i] + bias[i % cols];
}

// out[i, :] = table[tokens[i], :]; a token outside [0, vocab) gives a zero row.
__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ table,
                                                    const int32_t* __restrict__ tokens,
                                                    int64_t n, int64_t d, int64_t vocab,
                                                    float* __restrict__ out) {
    const int64_t total = n * d;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const int64_t r = i / d, c = i - r * d;
        const int64_t t = tokens[r];
        out[i] = t >= 0 && t < vocab ? table[t * d + c] : 0.0f;
    }
}

unsigned grid_for(int64_t n) {
    const int64_t blocks = ceil_div(n, 256);
    return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

}  // namespace

void launch_rope(float* q, float* k, const float* table, int64_t rows, int64_t seq_len,
                 int64_t first_pos, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                 hipStream_t s) {
    const int64_t n = rows * (q_heads + kv_heads) * (head_dim / 2);
    if (n <= 0) return;
    if (rope4_ok(q, k, table, rows, q_heads + kv_heads, head_dim) && seq_len > 0 &&
        seq_len < (int64_t(1) << 31)) {
        hipLaunchKernelGGL((rope4_kernel<false>), dim3(grid_for(n / 4)), dim3(256), 0, s, q, k,
                           table, int64_t(0), nullptr, static_cast<uint32_t>(seq_len), first_pos,
                           static_cast<uint32_t>(rows), static_cast<uint32_t>(q_heads),
                           static_cast<uint32_t>(kv_heads), static_cast<uint32_t>(head_dim));
        return;
    }
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(n)), dim3(256), 0, s, q, k, table, rows,
                       seq_len, first_pos, q_heads, kv_heads, head_dim);
}

void launch_attn_last(const float* q, const float* k, const float* v, float* out, float* scores,
                      int64_t batch, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                      int64_t head_dim, int64_t window, hipStream_t s) {
    const int64_t blocks = batch * q_heads;
    if (blocks <= 0 || seq_len <= 0) return;
    const float scale = sqrtf(static_cast<float>(head_dim));
    const bool vec4 = head_dim % 4 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(k) % 16 == 0;
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, q, k, v,
                           out, scores, seq_len, q_heads, kv_heads, head_dim, window, scale);
    };
    const bool lds = seq_len <= kAttnLastLds;
    if (vec4 && lds) go(attn_last_kernel<true, true>);
    else if (vec4) go(attn_last_kernel<true, false>);
    else if (lds) go(attn_last_kernel<false, true>);
    else go(attn_last_kernel<false, false>);
}

void launch_attn_softmax(float* scores, int64_t batches, int64_t seq_len, int64_t head_dim,
                         int64_t window, hipStream_t s) {
    const int64_t rows = batches * seq_len;
    if (rows <= 0) return;
    const float scale = sqrtf(static_cast<float>(head_dim));
    hipLaunchKernelGGL(attn_softmax_kernel, dim3(static_cast<unsigned>(ceil_div(rows, 4))),
                       dim3(256), 0, s, scores, rows, seq_len, scale, window);
}

void launch_rope_rows(float* q, float* k, const float* table, int64_t table_positions,
                      const int32_t* positions, int64_t rows, int64_t q_heads, int64_t kv_heads,
                      int64_t head_dim, hipStream_t s) {
    const int64_t n = rows * (q_heads + kv_heads) * (head_dim / 2);
    if (n <= 0) return;
    if (rope4_ok(q, k, table, rows, q_heads + kv_heads, head_dim)) {
        hipLaunchKernelGGL((rope4_kernel<true>), dim3(grid_for(n / 4)), dim3(256), 0, s, q, k,
                           table, table_positions, positions, uint32_t(1), int64_t(0),
                           static_cast<uint32_t>(rows), static_cast<uint32_t>(q_heads),
                           static_cast<uint32_t>(kv_heads), static_cast<uint32_t>(head_dim));
        return;
    }
    hipLaunchKernelGGL(rope_rows_kernel, dim3(grid_for(n)), dim3(256), 0, s, q, k, table,
                       table_positions, positions, rows, q_heads, kv_heads, head_dim);
}

void launch_attn_paths(const float* q, const float* k, const float* v, float* out,
                       float* scores, const int32_t* key_rows, const int32_t* key_beg,
                       const int32_t* key_end, int64_t nq, int64_t kv_rows, int64_t max_len,
                       int64_t key_total, int64_t scores_floats, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, int64_t window, hipStream_t s) {
    const int64_t blocks = nq * q_heads;
    if (blocks <= 0) return;
    const float scale = sqrtf(static_cast<float>(head_dim));
    const bool vec4 = head_dim % 4 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(k) % 16 == 0;
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, q, k, v,
                           out, scores, key_rows, key_beg, key_end, kv_rows, key_total,
                           scores_floats, q_heads, kv_heads, head_dim, window, scale);
    };
    const int64_t G = q_heads / kv_heads;
    if (vec4 && max_len <= 64 && head_dim <= 256 && (G == 1 || G == 2 || G == 4 || G == 8)) {
        const dim3 grid(static_cast<unsigned>(ceil_div(nq * kv_heads, 4)));
        auto wave = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, q, k, v, out, key_rows, key_beg,
                               key_end, nq, kv_rows, key_total, kv_heads, head_dim, window, scale);
        };
        if (G == 1) wave(attn_paths_wave_kernel<1>);
        else if (G == 2) wave(attn_paths_wave_kernel<2>);
        else if (G == 4) wave(attn_paths_wave_kernel<4>);
        else wave(attn_paths_wave_kernel<8>);
        return;
    }
    const bool lds = max_len <= kAttnLastLds;
    if (vec4 && lds) go(attn_paths_kernel<true, true>);
    else if (vec4) go(attn_paths_kernel<true, false>);
    else if (lds) go(attn_paths_kernel<false, true>);
    else go(attn_paths_kernel<false, false>);
}

void launch_add(float* a, const float* b, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, s, a, b, n);
}

void launch_add_bias(float* a, const float* bias, int64_t rows, int64_t cols, hipStream_t s) {
    const int64_t n = rows * cols;
    if (n <= 0) return;
    hipLaunchKernelGGL(add_bias_kernel, dim3(grid_for(n)), dim3(256), 0, s, a, bias, n, cols);
}

void launch_embed(const float* table, const int32_t* tokens, int64_t n, int64_t d, int64_t vocab,
                  float* out, hipStream_t s) {
    if (n <= 0 || d <= 0) return;
    hipLaunchKernelGGL(embed_kernel, dim3(grid_for(n * d)), dim3(256), 0, s, table, tokens, n,
                       d, vocab, out);
}

}  // namespace moe
