/*
 * moe_oracle.c -- CPU restatement of the reference MoE forward path.
 *
 * TEST INFRASTRUCTURE ONLY (see moe_oracle.h): the parity checker for tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py.  The product
 * never links it.
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off).
 * Contraction is spelled out in the source (fmaf versus separately rounded
 * multiply and add), never left to the compiler.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Bounds-checked element offset of a row-major [rows, cols] matrix.  The
 * reference reads every operand through Tensor::at(), which checks the rank
 * and every index before computing the offset (src/tensor.cu:90-110); the
 * check is kept so the CPU-path timing keeps the cost the reference pays. */
static inline size_t orc_at(size_t rows, size_t cols, size_t i, size_t j) {
    if (i >= rows || j >= cols) {
        fprintf(stderr, "oracle: index (%zu,%zu) outside [%zu,%zu]\n", i, j,
                rows, cols);
        abort();
    }
    return i * cols + j;
}

/* One multiply-accumulate step `acc += a*b` under the requested contraction. */
static inline float orc_mac(float acc, float a, float b, int contract) {
    if (contract) return fmaf(a, b, acc);
    const float prod = a * b; /* rounded on its own: -ffp-contract=off */
    return acc + prod;
}

/* The reference's accurate_exp: exp evaluated in double, rounded to float once
 * (src/tensor.cu:132-134, src/layer.cu:9-11). */
static inline float orc_accurate_exp(float x) {
    return (float)exp((double)x);
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* LCG used by the reference's MoE microbenchmark to fill weights and
 * activations: s = s*1664525 + 1013904223, v = ((s>>8)&0xFFFF)/32768 - 1
 * (docs/microworld/exp-003-moe-bench.cu:27).
 * Pinned by: the published per-expert routing histograms
 * (docs/microworld/exp-003-moe.html:399-405), which this fill feeds. */
void orc_lcg_fill(float* out, size_t n, uint32_t seed) {
    uint32_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        out[i] = (float)((s >> 8) & 0xFFFFu) / 32768.0f - 1.0f;
    }
}

/* NT SGEMM c[i,j] = sum_{p ascending} a[i,p]*b[j,p], one float accumulator
 * starting at 0, OpenMP over rows, c zeroed first
 * (src/tensor.cu:136-148, tensor_ops::matmul_transposed).
 * Pinned by: float64 brute force (tests/test_oracle.py), the sequential
 * rounding model on hand-built sums, and the routing-histogram KAT (the gate
 * logits are this function). */
int orc_matmul_nt(const float* a, const float* b, float* c, size_t m,
                  size_t n, size_t k, int contract) {
    if ((m && n && k) && (!a || !b)) return 1;
    if (m && n && !c) return 1;
    if (m && n) memset(c, 0, m * n * sizeof(float));
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p)
                sum = orc_mac(sum, a[orc_at(m, k, (size_t)i, p)],
                              b[orc_at(n, k, j, p)], contract);
            c[orc_at(m, n, (size_t)i, j)] = sum;
        }
    }
    return 0;
}

/* NN SGEMM c[i,j] = sum_{p ascending} a[i,p]*b[p,j].  The reference declares
 * tensor_ops::matmul (include/tensor.h:61) and never defines it; this follows
 * matmul_transposed's loop nest with b read as [K,N].
 * Pinned by: float64 brute force and the identity matmul_nn(a, b) ==
 * matmul_nt(a, b^T) bit-for-bit (tests/test_oracle.py). */
int orc_matmul_nn(const float* a, const float* b, float* c, size_t m,
                  size_t n, size_t k, int contract) {
    if ((m && n && k) && (!a || !b)) return 1;
    if (m && n && !c) return 1;
    if (m && n) memset(c, 0, m * n * sizeof(float));
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p)
                sum = orc_mac(sum, a[orc_at(m, k, (size_t)i, p)],
                              b[orc_at(k, n, p, j)], contract);
            c[orc_at(m, n, (size_t)i, j)] = sum;
        }
    }
    return 0;
}

/* y = x / (1 + accurate_exp(-x)) (src/tensor.cu:169-173).
 * Pinned by: a float64 evaluation of the same expression rounded at the same
 * points, and silu(0) = 0, silu(x) - silu(-x) = x (tests/test_oracle.py).
 * The glibc double exp underneath is the third-party boundary the reference
 * also sits on (parity unpinned at the last double ulp; invisible after the
 * rounding to float except in double-rounding cases). */
void orc_silu(const float* x, float* y, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        y[i] = x[i] / (1.0f + orc_accurate_exp(-x[i]));
}

/* tensor_ops::layer_norm (src/tensor.cu:175-189), the post-attention norm
 * in front of the MoE block.  Per row: mean = (one float accumulator over
 * j ascending) / h; var = (one float accumulator of d*d, d = x - mean) / h;
 * inv = 1 / sqrt(var + eps); y = (x - mean) * inv * weight + bias, left to
 * right.  `contract` decides whether the two `a*b + c` sites (var += d*d and
 * ... * weight + bias) are fused, as for the gate (an FMA host build of the
 * reference contracts them, its no-FMA Xeon build does not).  The
 * reference's GPU form keeps the same chains (src/model.cu:720-846; the
 * epilogue's four ops at :235-246).  y, row_mean and row_inv may each be
 * NULL.
 * Pinned by: closed forms (constant rows give y = bias exactly; small
 * integer rows give exact mean and variance), float64 within rounding, and
 * cases that fail the plausible slips -- a double or compensated
 * accumulator, variance as E[x^2] - mean^2, eps outside the sqrt, the bias
 * scaled by the weight (tests/test_oracle.py). */
int orc_layer_norm(const float* x, const float* weight, const float* bias,
                   float eps, size_t rows, size_t h, int contract, float* y,
                   float* row_mean, float* row_inv) {
    if (rows && (!x || h == 0 || !weight || !bias)) return 1;
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < (long long)rows; ++r) {
        float mean = 0.0f;
        for (size_t j = 0; j < h; ++j) mean += x[orc_at(rows, h, (size_t)r, j)];
        mean /= (float)h;
        float var = 0.0f;
        for (size_t j = 0; j < h; ++j) {
            const float dv = x[orc_at(rows, h, (size_t)r, j)] - mean;
            var = orc_mac(var, dv, dv, contract);
        }
        const float inv = 1.0f / sqrtf(var / (float)h + eps);
        if (row_mean) row_mean[r] = mean;
        if (row_inv) row_inv[r] = inv;
        if (!y) continue;
        for (size_t j = 0; j < h; ++j) {
            const size_t o = orc_at(rows, h, (size_t)r, j);
            const float scaled = (x[o] - mean) * inv;
            y[o] = contract ? fmaf(scaled, weight[j], bias[j]) : scaled * weight[j] + bias[j];
        }
    }
    return 0;
}

/* RMS norm (config 5's decoder names RMSNorm; the reference has none -- its
 * norm is layer_norm above).  Defined in the same style as tensor_ops::
 * layer_norm: ss = one float accumulator of x*x over j ascending (fused under
 * `contract`), inv = 1 / sqrt(ss / h + eps), y = x * inv * weight, left to
 * right.  y and row_inv may be NULL.
 * Pinned by: closed forms (a constant row c gives inv = 1/sqrt(c*c + eps);
 * 3, 4 gives ss = 25 exactly), float64 within rounding, and a row whose
 * single-float sum of squares differs from a double one (tests/test_oracle.py). */
int orc_rms_norm(const float* x, const float* weight, float eps, size_t rows,
                 size_t h, int contract, float* y, float* row_inv) {
    if (rows && (!x || h == 0 || !weight)) return 1;
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < (long long)rows; ++r) {
        float ss = 0.0f;
        for (size_t j = 0; j < h; ++j) {
            const float v = x[orc_at(rows, h, (size_t)r, j)];
            ss = orc_mac(ss, v, v, contract);
        }
        const float inv = 1.0f / sqrtf(ss / (float)h + eps);
        if (row_inv) row_inv[r] = inv;
        if (!y) continue;
        for (size_t j = 0; j < h; ++j) {
            const size_t o = orc_at(rows, h, (size_t)r, j);
            y[o] = (x[o] * inv) * weight[j];
        }
    }
    return 0;
}

/* The cos/sin of RoPE for positions [0, positions) and pairs j < head_dim/2:
 * inv = powf(theta, -2j/head_dim), table[(pos*half + j)*2 + {0,1}] =
 * {cosf, sinf}(pos * inv) -- the float libm calls of tensor_ops::apply_rope
 * (src/tensor.cu:196-197) and of the reference's host-built GPU table
 * (src/model.cu:1791-1797).
 * Pinned by: angles against float64 (tests/test_oracle.py); libm's
 * powf/cosf/sinf last ulp: parity unpinned, as for exp. */
int orc_rope_table(float theta, size_t head_dim, size_t positions, float* table) {
    if (head_dim % 2 || (positions > 0 && !table)) return 1;
    const size_t half = head_dim / 2;
    for (size_t s = 0; s < positions; ++s)
        for (size_t j = 0; j < half; ++j) {
            const float inv = powf(theta, -2.0f * (float)j / (float)head_dim);
            table[(s * half + j) * 2] = cosf((float)s * inv);
            table[(s * half + j) * 2 + 1] = sinf((float)s * inv);
        }
    return 0;
}

/* tensor_ops::apply_rope (src/tensor.cu:191-210) over `batch` sequences of
 * seq_len rows (row r sits at position r % seq_len), cos/sin from
 * orc_rope_table's layout: (x0, x1) = (x[j], x[j + half]) -> (x0 c - x1 s,
 * x1 c + x0 s), each product rounded on its own (this file is built with
 * -ffp-contract=off), as rope_rows does on the GPU (src/model.cu:1066-1081,
 * __fmul_rn / __fsub_rn / __fadd_rn); q has q_heads heads, k kv_heads, rows
 * of heads * head_dim.
 * Pinned by: position 0 is the identity exactly; each (x0, x1) pair keeps its
 * length; a pair at the angles of a 90-degree table turns exactly
 * (tests/test_oracle.py). */
int orc_rope(float* q, float* k, const float* table, size_t batch, size_t seq_len,
             size_t q_heads, size_t kv_heads, size_t head_dim) {
    if (head_dim % 2 || (batch * seq_len > 0 && (!q || !k || !table))) return 1;
    const size_t half = head_dim / 2, rows = batch * seq_len;
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < (long long)rows; ++r) {
        const size_t s = (size_t)r % seq_len;
        for (int which = 0; which < 2; ++which) {
            float* x = which == 0 ? q : k;
            const size_t heads = which == 0 ? q_heads : kv_heads;
            for (size_t h = 0; h < heads; ++h)
                for (size_t j = 0; j < half; ++j) {
                    const float c = table[(s * half + j) * 2], sn = table[(s * half + j) * 2 + 1];
                    const size_t o = orc_at(rows, heads * head_dim, (size_t)r, h * head_dim + j);
                    const float x0 = x[o], x1 = x[o + half];
                    x[o] = x0 * c - x1 * sn;
                    x[o + half] = x1 * c + x0 * sn;
                }
        }
    }
    return 0;
}

/* The attention core of PhiAttention::forward (src/layer.cu:111-143) over
 * `batch` sequences of seq_len rows: for query row qi and head qh (key head
 * qh / (q_heads / kv_heads)), keys ki <= qi with qi - ki < window;
 * score = sum_d q*k (one float accumulator, d ascending), scaled =
 * score / sqrt(head_dim); m = max scaled; denom = sum accurate_exp(scaled - m)
 * over ki ascending; out[qi, qh, d] = sum over ki ascending of
 * accurate_exp(scaled - m) / denom * v[ki, kh, d].  The reference recomputes
 * each score three times; it is computed once here (the same value).
 * Pinned by: one visible key gives out = v exactly; window 1 gives
 * out = v[qi]; identical keys give the mean of the visible values; float64
 * brute force (tests/test_oracle.py). */
int orc_attention(const float* q, const float* k, const float* v, float* out,
                  size_t batch, size_t seq_len, size_t q_heads, size_t kv_heads,
                  size_t head_dim, size_t window) {
    if (!kv_heads || q_heads % kv_heads || window == 0) return 1;
    if (batch * seq_len > 0 && (!q || !k || !v || !out)) return 1;
    const size_t group = q_heads / kv_heads, rows = batch * seq_len;
    const size_t qw = q_heads * head_dim, kw = kv_heads * head_dim;
    const float scale = sqrtf((float)head_dim);
#pragma omp parallel for schedule(dynamic, 4)
    for (long long r = 0; r < (long long)rows; ++r) {
        const size_t b = (size_t)r / seq_len, qi = (size_t)r % seq_len;
        float* scaled = (float*)malloc((seq_len + 1) * sizeof(float));
        float* wts = (float*)malloc((seq_len + 1) * sizeof(float));
        for (size_t qh = 0; qh < q_heads; ++qh) {
            const size_t kh = qh / group;
            float maxv = -INFINITY;
            for (size_t ki = 0; ki <= qi; ++ki) {
                if (qi - ki >= window) continue;
                float score = 0.0f;
                for (size_t d = 0; d < head_dim; ++d)
                    score += q[orc_at(rows, qw, (size_t)r, qh * head_dim + d)] *
                             k[orc_at(rows, kw, b * seq_len + ki, kh * head_dim + d)];
                scaled[ki] = score / scale;
                maxv = fmaxf(maxv, scaled[ki]);
            }
            float denom = 0.0f;
            for (size_t ki = 0; ki <= qi; ++ki)
                if (qi - ki < window) {
                    wts[ki] = orc_accurate_exp(scaled[ki] - maxv);
                    denom += wts[ki];
                }
            for (size_t d = 0; d < head_dim; ++d) {
                float value = 0.0f;
                for (size_t ki = 0; ki <= qi; ++ki)
                    if (qi - ki < window)
                        value += wts[ki] / denom * v[orc_at(rows, kw, b * seq_len + ki, kh * head_dim + d)];
                out[orc_at(rows, qw, (size_t)r, qh * head_dim + d)] = value;
            }
        }
        free(scaled);
        free(wts);
    }
    return 0;
}

/* c = a * b elementwise (src/tensor.cu:163-167). Pinned by direct products. */
void orc_mul(const float* a, const float* b, float* c, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) c[i] = a[i] * b[i];
}

/* Score canonicalisation of PhiMoE::route: round |s| to the quantum, restore
 * the sign (src/layer.cu:50-55; identical on the GPU at src/model.cu:880-886).
 * A quantum <= 0 leaves the score unchanged (an extension; the reference's
 * quantum is the constant 1e-3, include/config.h:22). */
static inline float orc_quantise(float score, float quantum) {
    if (!(quantum > 0.0f)) return score;
    const float rounded = floorf(fabsf(score) / quantum + 0.5f) * quantum;
    return score < 0.0f ? -rounded : rounded;
}

/* Reference select(): ascending scan, take e when nothing is held yet or when
 * it beats the held score by more than tie_eps (src/layer.cu:56-65).  The
 * reference excludes one expert; the k > 2 extension excludes every earlier
 * pick, which is the same rule for k = 2. */
static int orc_phi_select(const float* scores, size_t E,
                          const unsigned char* taken, float tie_eps) {
    int best = -1;
    float best_value = -INFINITY;
    for (size_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || scores[e] > best_value + tie_eps) {
            best = (int)e;
            best_value = scores[e];
        }
    }
    return best;
}

/* Selection order key of the softmax router: a NaN logit ranks as -inf so
 * that (value descending, index ascending) is a total order. */
static inline float orc_rank_value(float v) { return isnan(v) ? -INFINITY : v; }

/* Router, two modes.
 *
 * ORC_ROUTER_PHI_QUANT follows PhiMoE::route (src/layer.cu:47-70): quantise,
 * select, select again excluding the first, fixed weights 0.5/0.5 (emitted in
 * selection order).  For k != 2 (an extension) the select is repeated k times
 * and every weight is 1/k.
 * Pinned by: the routing-histogram KAT of docs/microworld/exp-003-moe.html
 * (E=16, k=2, LCG inputs, six token counts) and hand cases whose answer
 * follows from the rule (non-argmax chains, 0.0199/0.0201 gaps, exact ties,
 * quantisation boundaries, negative scores, +-0) in tests/test_oracle.py.
 *
 * ORC_ROUTER_SOFTMAX_TOPK has no reference code (the reference declares
 * softmax_last_dim, include/tensor.h:67, and never defines it): the k largest
 * scores, ties to the lower index, emitted in descending order; weights
 * w_s = exp(v_s - v_0) / sum_j exp(v_j - v_0) over the selected k, evaluated
 * in double and rounded to float once, the reference's accurate_exp
 * convention.
 * Pinned by: brute force against a sorted order and a float64 softmax
 * (tests/test_oracle.py).
 *
 * expert_bias (may be NULL) is added to every logit before either mode. */
int orc_route(const float* logits, const float* expert_bias, size_t T,
              size_t E, size_t k, int mode, float quantum, float tie_eps,
              int32_t* topk_idx, float* topk_w) {
    if (k == 0 || k > E) return 1;
    if (T && (!logits || !topk_idx || !topk_w)) return 1;
    if (mode != ORC_ROUTER_PHI_QUANT && mode != ORC_ROUTER_SOFTMAX_TOPK) return 1;
    int bad = 0;
#pragma omp parallel
    {
        float* scores = (float*)malloc(E * sizeof(float));
        unsigned char* taken = (unsigned char*)malloc(E);
        if (!scores || !taken) {
#pragma omp atomic write
            bad = 1;
        } else {
#pragma omp for schedule(static)
            for (long long t = 0; t < (long long)T; ++t) {
                const float* row = logits + (size_t)t * E;
                memset(taken, 0, E);
                if (mode == ORC_ROUTER_PHI_QUANT) {
                    for (size_t e = 0; e < E; ++e) {
                        const float s = expert_bias ? row[e] + expert_bias[e] : row[e];
                        scores[e] = orc_quantise(s, quantum);
                    }
                    const float w = 1.0f / (float)k;
                    for (size_t s = 0; s < k; ++s) {
                        const int pick = orc_phi_select(scores, E, taken, tie_eps);
                        taken[pick] = 1;
                        topk_idx[(size_t)t * k + s] = pick;
                        topk_w[(size_t)t * k + s] = w;
                    }
                } else {
                    for (size_t e = 0; e < E; ++e) {
                        const float s = expert_bias ? row[e] + expert_bias[e] : row[e];
                        scores[e] = orc_rank_value(s);
                    }
                    double ex[256];
                    double* exps = k <= 256 ? ex : (double*)malloc(k * sizeof(double));
                    for (size_t s = 0; s < k; ++s) {
                        int best = -1;
                        for (size_t e = 0; e < E; ++e) {
                            if (taken[e]) continue;
                            if (best < 0 || scores[e] > scores[best]) best = (int)e;
                        }
                        taken[best] = 1;
                        topk_idx[(size_t)t * k + s] = best;
                    }
                    const double top = (double)scores[topk_idx[(size_t)t * k]];
                    double sum = 0.0;
                    for (size_t s = 0; s < k; ++s) {
                        exps[s] = exp((double)scores[topk_idx[(size_t)t * k + s]] - top);
                        sum += exps[s];
                    }
                    for (size_t s = 0; s < k; ++s)
                        topk_w[(size_t)t * k + s] = (float)(exps[s] / sum);
                    if (exps != ex) free(exps);
                }
            }
        }
        free(scores);
        free(taken);
    }
    return bad;
}

/* Stable bucket sort of the (token, slot) pairs by expert, tokens ascending
 * within each expert: the order in which PhiMoE::forward appends to
 * assignments[e] (src/layer.cu:86-92).  expert_offsets[E+1] is the exclusive
 * scan of the per-expert counts, perm[r] the token of packed row r, and
 * inv[t*k+s] the packed row of token t's s-th selection.
 * Pinned by: invariants (offsets = scan of histogram, perm ascending within
 * each expert, perm[inv[t*k+s]] == t) and brute force (tests/test_oracle.py). */
int orc_permute(const int32_t* topk_idx, size_t T, size_t k, size_t E,
                int32_t* expert_offsets, int32_t* perm, int32_t* inv) {
    if (!expert_offsets || E == 0) return 1;
    if (T && k && (!topk_idx || !perm || !inv)) return 1;
    int32_t* next = (int32_t*)calloc(E + 1, sizeof(int32_t));
    if (!next) return 1;
    for (size_t i = 0; i < T * k; ++i) {
        const int32_t e = topk_idx[i];
        if (e < 0 || (size_t)e >= E) { free(next); return 1; }
        next[e + 1]++;
    }
    for (size_t e = 0; e < E; ++e) next[e + 1] += next[e];
    memcpy(expert_offsets, next, (E + 1) * sizeof(int32_t));
    for (size_t t = 0; t < T; ++t)
        for (size_t s = 0; s < k; ++s) {
            const int32_t e = topk_idx[t * k + s];
            const int32_t r = next[e]++;
            perm[r] = (int32_t)t;
            inv[t * k + s] = r;
        }
    free(next);
    return 0;
}

/* Per-expert FFN over the packed rows (src/layer.cu:93-98 gathering the rows,
 * then PhiMLP::forward, src/layer.cu:32-45):
 *   SWIGLU:   out = (silu(x w1^T) * (x w3^T)) w2^T
 *   SILU_MLP: out = silu(x w1^T) w2^T   (an extension for the Linear + SiLU +
 *             Linear expert; composed from the same matmul_transposed + silu)
 * w1, w3: [E, d_ff, d]; w2: [E, d, d_ff]; out_rows: [T*k, d] in packed order.
 * Pinned by: its parts (matmul_nt, silu, mul) and the whole layer's float64
 * evaluation (tests/test_oracle.py). */
int orc_expert_ffn(const float* x, size_t T, size_t d, const int32_t* perm,
                   const int32_t* expert_offsets, size_t E, const float* w1,
                   const float* w3, const float* w2, size_t d_ff, int act,
                   int contract, float* out_rows) {
    if (!x || !perm || !expert_offsets || !w1 || !w2 || !out_rows) return 1;
    if (act != ORC_ACT_SWIGLU && act != ORC_ACT_SILU_MLP) return 1;
    if (act == ORC_ACT_SWIGLU && !w3) return 1;
    for (size_t e = 0; e < E; ++e) {
        const size_t r0 = (size_t)expert_offsets[e];
        const size_t n_e = (size_t)expert_offsets[e + 1] - r0;
        if (n_e == 0) continue;
        float* input = (float*)malloc(n_e * d * sizeof(float));
        float* gate = (float*)malloc(n_e * d_ff * sizeof(float));
        float* activated = (float*)malloc(n_e * d_ff * sizeof(float));
        float* up = act == ORC_ACT_SWIGLU ? (float*)malloc(n_e * d_ff * sizeof(float)) : NULL;
        if (!input || !gate || !activated || (act == ORC_ACT_SWIGLU && !up)) {
            free(input); free(gate); free(activated); free(up);
            return 1;
        }
        for (size_t i = 0; i < n_e; ++i) {
            const size_t tok = (size_t)perm[r0 + i];
            if (tok >= T) { free(input); free(gate); free(activated); free(up); return 1; }
            for (size_t j = 0; j < d; ++j)
                input[orc_at(n_e, d, i, j)] = x[orc_at(T, d, tok, j)];
        }
        orc_matmul_nt(input, w1 + e * d_ff * d, gate, n_e, d_ff, d, contract);
        orc_silu(gate, activated, n_e * d_ff);
        if (act == ORC_ACT_SWIGLU) {
            orc_matmul_nt(input, w3 + e * d_ff * d, up, n_e, d_ff, d, contract);
            orc_mul(activated, up, activated, n_e * d_ff);
        }
        orc_matmul_nt(activated, w2 + e * d * d_ff, out_rows + r0 * d, n_e, d,
                      d_ff, contract);
        free(input); free(gate); free(activated); free(up);
    }
    return 0;
}

/* Gate-weighted combine: y starts at zero and each token adds w * out for its
 * experts in ascending expert order, which is the order the reference's
 * expert loop visits them (src/layer.cu:83,93-101: y.zero(), then
 * y[t] += w * out for e = 0..E-1).
 * Pinned by: float64 sums and the k = 2 closed form (tests/test_oracle.py). */
int orc_combine(const float* out_rows, const int32_t* topk_idx,
                const float* topk_w, const int32_t* inv, size_t T, size_t k,
                size_t d, int contract, float* y) {
    if (T && d && (!y || (k && (!out_rows || !topk_idx || !topk_w || !inv)))) return 1;
    if (k > 256) return 1;
    memset(y, 0, T * d * sizeof(float));
#pragma omp parallel for schedule(static)
    for (long long t = 0; t < (long long)T; ++t) {
        int order[256];
        for (size_t s = 0; s < k; ++s) order[s] = (int)s;
        /* insertion sort of the slots by expert id (stable) */
        for (size_t a = 1; a < k; ++a) {
            const int cur = order[a];
            size_t b = a;
            while (b > 0 && topk_idx[(size_t)t * k + order[b - 1]] >
                                topk_idx[(size_t)t * k + cur]) {
                order[b] = order[b - 1];
                --b;
            }
            order[b] = cur;
        }
        for (size_t q = 0; q < k; ++q) {
            const size_t s = (size_t)order[q];
            const float w = topk_w[(size_t)t * k + s];
            const float* row = out_rows + (size_t)inv[(size_t)t * k + s] * d;
            float* dst = y + (size_t)t * d;
            for (size_t j = 0; j < d; ++j) dst[j] = orc_mac(dst[j], w, row[j], contract);
        }
    }
    return 0;
}

/* The whole layer, PhiMoE::forward (src/layer.cu:80-103): gate logits with
 * matmul_transposed, route, bucket by expert, expert FFN, combine. */
int orc_moe_forward(const float* x, size_t T, size_t d, const float* gate_w,
                    const float* expert_bias, size_t E, size_t k,
                    const float* w1, const float* w3, const float* w2,
                    size_t d_ff, int act, int router_mode, float quantum,
                    float tie_eps, int contract, float* y,
                    int32_t* topk_idx_out, float* topk_w_out) {
    if (!x || !gate_w || !y || E == 0 || k == 0 || k > E) return 1;
    int rc = 0;
    float* logits = (float*)malloc(T * E * sizeof(float) + 1);
    int32_t* idx = (int32_t*)malloc(T * k * sizeof(int32_t) + 1);
    float* w = (float*)malloc(T * k * sizeof(float) + 1);
    int32_t* offsets = (int32_t*)malloc((E + 1) * sizeof(int32_t));
    int32_t* perm = (int32_t*)malloc(T * k * sizeof(int32_t) + 1);
    int32_t* inv = (int32_t*)malloc(T * k * sizeof(int32_t) + 1);
    float* out_rows = (float*)malloc(T * k * d * sizeof(float) + 1);
    if (!logits || !idx || !w || !offsets || !perm || !inv || !out_rows) { rc = 1; goto done; }
    if ((rc = orc_matmul_nt(x, gate_w, logits, T, E, d, contract))) goto done;
    if ((rc = orc_route(logits, expert_bias, T, E, k, router_mode, quantum, tie_eps, idx, w))) goto done;
    if ((rc = orc_permute(idx, T, k, E, offsets, perm, inv))) goto done;
    if ((rc = orc_expert_ffn(x, T, d, perm, offsets, E, w1, w3, w2, d_ff, act, contract, out_rows))) goto done;
    if ((rc = orc_combine(out_rows, idx, w, inv, T, k, d, contract, y))) goto done;
    if (topk_idx_out) memcpy(topk_idx_out, idx, T * k * sizeof(int32_t));
    if (topk_w_out) memcpy(topk_w_out, w, T * k * sizeof(float));
done:
    free(logits); free(idx); free(w); free(offsets); free(perm); free(inv); free(out_rows);
    return rc;
}
