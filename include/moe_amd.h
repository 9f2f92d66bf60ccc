/*
 * moe_amd.h -- C ABI of the MI355X (gfx950) MoE forward hot path.
 *
 * Every entry point takes device pointers (fp32 / int32, row-major), plain
 * sizes and a stream given as `void*` (a hipStream_t; NULL = the default
 * stream).  Work is enqueued on that stream and the call returns without
 * synchronising.  Return value: MOE_OK, or an error code whose message
 * moe_last_error() returns (thread-local).  The C++ drop-in layer rethrows
 * MOE_ERR_INVALID as std::invalid_argument and the others as
 * std::runtime_error, the reference's exception types.
 *
 * Replaces (paths relative to the songsnim/accelerating-MoE-inference root):
 *   moe_sgemm_nt        tensor_ops::matmul_transposed     src/tensor.cu:136-148
 *                       and the GPU gemm_nt_body/gemm_nt_bias src/model.cu:182-460
 *   moe_sgemm_nn        tensor_ops::matmul (declared only) include/tensor.h:61
 *   moe_sgemm_nt_residual  DeviceLinear::forward_resid     src/model.cu:1417-1427
 *   moe_gate_logits     router gate GEMM                   src/layer.cu:84,
 *                       gemm_gate                          src/model.cu:505-616
 *   moe_route           PhiMoE::route                      src/layer.cu:47-70,
 *                       route_top2                         src/model.cu:878-904
 *   moe_permute         assignments[e] build               src/layer.cu:86-92,
 *                       route_count/scan/place             src/model.cu:921-1030
 *   moe_expert_ffn_grouped  per-expert PhiMLP::forward     src/layer.cu:32-45,93-98,
 *                       gemm_grouped / w2 launches         src/model.cu:625-667
 *   moe_combine         y[t] += w * out in expert order    src/layer.cu:99-101,
 *                       gemm_grouped_combine epilogue      src/model.cu:436-447
 *   moe_layer_norm      tensor_ops::layer_norm             src/tensor.cu:175-189,
 *                       layer_norm_rows / forward_stats    src/model.cu:720-846,1440-1480
 *   moe_rms_norm        (no counterpart: the RMSNorm config 5's decoder names)
 *   moe_rope_table      the host-built cos/sin table       src/model.cu:1784-1798
 *   moe_rope            tensor_ops::apply_rope             src/tensor.cu:191-210,
 *                       rope_rows                          src/model.cu:1046-1083
 *   moe_attention       PhiAttention::forward, after the projections  src/layer.cu:111-143;
 *                       attention_heads                    src/model.cu:1161-1283
 *   moe_attention_last  attention_heads<true> of the pruned last layer  src/model.cu:1889-1960
 *   moe_rope_rows       rope_rows with per-node positions  src/model.cu:1046-1083
 *   moe_attention_paths attention_heads over trie root paths  src/model.cu:1161-1283,1667-1680
 *   moe_add             tensor_ops::add_inplace            src/tensor.cu:150-154
 *   moe_add_bias        tensor_ops::add_bias_inplace       src/tensor.cu:156-161
 *   moe_embed           embedding row gather (gather_rows) src/model.cu:674-693,1878-1885
 *   moe_layer_forward   PhiMoE::forward                    src/layer.cu:80-103,
 *                       the MoE block of generate()        src/model.cu:1968-2021
 *   moe_ctx_*           DeviceBuffer / Scratch workspace   src/model.cu:45-68,1294-1324
 */
#ifndef MOE_AMD_H
#define MOE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_ERR_INVALID 1     /* bad shape / argument (std::invalid_argument) */
#define MOE_ERR_RUNTIME 2     /* HIP runtime failure (std::runtime_error)     */
#define MOE_ERR_UNSUPPORTED 3 /* argument outside what the kernels support    */

/* Floating-point contraction of `acc += a*b` in the bit-exact kernels (gate
 * logits, combine).  FMA: one rounding per step, what the reference's GPU
 * gate and its CPU build on an FMA host compute.  NONE: product and sum
 * rounded separately, what the reference's CPU build on a host without FMA
 * computes. */
#define MOE_CONTRACT_NONE 0
#define MOE_CONTRACT_FMA 1

/* PHI_QUANT: PhiMoE::route (quantise to `quantum`, sequential select with
 * `tie_eps`, fixed weights 1/k = 0.5 for k = 2).  SOFTMAX_TOPK: k largest
 * logits (ties to the lower index), softmax over the selected k. */
#define MOE_ROUTER_PHI_QUANT 0
#define MOE_ROUTER_SOFTMAX_TOPK 1

/* SWIGLU: w2 (silu(x w1^T) * (x w3^T)) (PhiMLP).  SILU_MLP: w2 silu(x w1^T). */
#define MOE_ACT_SWIGLU 0
#define MOE_ACT_SILU_MLP 1

/* Norm in front of the experts (moe_layer_desc.norm).  NONE: gate and
 * experts read x.  LAYER: they read layer_norm(x, norm_w, norm_b, norm_eps),
 * the reference's post-attention norm (src/model.cu:1968-2002), computed
 * bit-identically to tensor_ops::layer_norm under desc.contract.  The layer
 * writes the normalised rows once, into its workspace, and the gate and the
 * w1/w3 GEMM read them there. */
#define MOE_NORM_NONE 0
#define MOE_NORM_LAYER 1
/* RMS: the RMSNorm config 5's decoder names, which the reference does not
 * have; defined like tensor_ops::layer_norm without the mean and the bias
 * (see moe_rms_norm).  weights.norm_b is ignored. */
#define MOE_NORM_RMS 2

typedef struct moe_ctx moe_ctx;

typedef struct moe_layer_desc {
    int64_t T;        /* tokens (rows of x)                         */
    int64_t d;        /* model width                                */
    int64_t E;        /* experts, 1..1024                           */
    int64_t k;        /* experts per token, 1..min(E, 32)           */
    int64_t d_ff;     /* expert hidden width                        */
    int32_t act;      /* MOE_ACT_*                                  */
    int32_t router;   /* MOE_ROUTER_*                               */
    float quantum;    /* PHI_QUANT score quantum (1e-3 in the reference)   */
    float tie_eps;    /* PHI_QUANT tie margin (2e-2 in the reference)      */
    int32_t contract; /* MOE_CONTRACT_* for the norm, gate logits, combine   */
    int32_t norm;     /* MOE_NORM_*                                         */
    float norm_eps;   /* norm epsilon (MOE_NORM_LAYER, MOE_NORM_RMS)        */
    int32_t residual; /* 1: y = x + MoE(...), x un-normalised (the block's
                         residual, src/model.cu:2009-2012); 0: y = MoE(...) */
} moe_layer_desc;

typedef struct moe_layer_weights {
    const float* gate_w;      /* [E, d]                         */
    const float* expert_bias; /* [E] added to logits, or NULL   */
    const float* w1;          /* [E, d_ff, d]                   */
    const float* w3;          /* [E, d_ff, d]; NULL for SILU_MLP */
    const float* w2;          /* [E, d, d_ff]                   */
    const float* norm_w;      /* [d] norm weight (MOE_NORM_LAYER / RMS) */
    const float* norm_b;      /* [d] layer norm bias (MOE_NORM_LAYER)  */
} moe_layer_weights;

/* ---- context: device binding, grow-only workspace, optional kernel timing.
 * Replaces the reference's DeviceBuffer/Scratch (src/model.cu:45-68,
 * 1294-1324).  A context is not safe for concurrent calls from several
 * threads (the reference's generate() is not either, include/model.h:124-127).
 * Every call on a context uses the same workspace: calls on different streams
 * must be ordered by the caller (an event, or one stream), since two in
 * flight at once would share it.  Growing the workspace synchronises the
 * device before the old buffer is freed. */
int moe_ctx_create(int device, moe_ctx** out);
int moe_ctx_destroy(moe_ctx* ctx);
/* Grow the workspace so that moe_layer_forward(desc) allocates nothing.
 * It also covers moe_expert_ffn_grouped on the same (T, k, d, d_ff, E) and
 * the sgemm / attention calls of that size or smaller. */
int moe_ctx_reserve(moe_ctx* ctx, const moe_layer_desc* desc);
/* The bytes of the context's workspace as it stands (0 before any call
 * that needed one).  No reference counterpart: an introspection query for
 * tests and tools (e.g. that moe_layer_forward_noalloc leaves it at 0). */
int moe_ctx_workspace_bytes(moe_ctx* ctx, int64_t* bytes);
/* Kernel timing (the reference's APS_PROFILE stage timers,
 * src/model.cu:1584-1622): when on, every launch is bracketed by HIP events
 * on its stream.  moe_ctx_kernel_times() synchronises, then returns the
 * number of named kernels and fills up to `cap` entries of names / total
 * milliseconds / launch counts accumulated since the last reset (on an error
 * it returns minus the MOE_ERR_* status). */
int moe_ctx_set_timing(moe_ctx* ctx, int enabled);
int moe_ctx_kernel_times(moe_ctx* ctx, const char** names, double* total_ms,
                         int64_t* launches, int cap);
int moe_ctx_reset_timing(moe_ctx* ctx);
/* Launches one empty kernel (one wave, no work) on `stream`, timed like any
 * other launch under moe_ctx_set_timing (name "empty").  No reference
 * counterpart: the launch-latency floor that the small routing and
 * permutation kernels are reported against. */
int moe_launch_floor(moe_ctx* ctx, void* stream);
const char* moe_last_error(void);
const char* moe_version(void);

/* ---- dense SGEMM, fp32 MFMA.
 * NT: C[M,N] = A[M,K] B[N,K]^T (+ bias[N]); NN: C = A[M,K] B[K,N] (+ bias).
 * Any M, N, K >= 0; K = 0 gives C = bias (or 0).  bias may be NULL. */
int moe_sgemm_nt(moe_ctx* ctx, const float* A, const float* B,
                 const float* bias, float* C, int64_t M, int64_t N, int64_t K,
                 void* stream);
int moe_sgemm_nn(moe_ctx* ctx, const float* A, const float* B,
                 const float* bias, float* C, int64_t M, int64_t N, int64_t K,
                 void* stream);
/* NT with the residual add folded into the GEMM's store: C = (A B^T + bias)
 * + R, R[M,N] (R == C is allowed), bit-identical to moe_sgemm_nt followed by
 * moe_add(C, R) (tensor_ops::add_inplace after the o-projection,
 * src/layer.cu:156).  Replaces DeviceLinear::forward_resid /
 * gemm_nt_bias_resid (src/model.cu:1417-1427, include/model.h:50-51), the
 * o-projection of the reference's generate() (src/model.cu:1965). */
int moe_sgemm_nt_residual(moe_ctx* ctx, const float* A, const float* B,
                          const float* bias, const float* R, float* C, int64_t M,
                          int64_t N, int64_t K, void* stream);

/* ---- elementwise ops of the expert MLP, bit-identical to the CPU loops:
 * moe_silu: y = x / (1 + float(exp(double(-x))))  tensor_ops::silu, src/tensor.cu:169-173
 * moe_mul:  c = a * b                              tensor_ops::mul,  src/tensor.cu:163-167
 * (in place is allowed: y == x, c == a or c == b). */
int moe_silu(moe_ctx* ctx, const float* x, float* y, int64_t n, void* stream);
int moe_mul(moe_ctx* ctx, const float* a, const float* b, float* c, int64_t n,
            void* stream);

/* ---- layer norm over the last axis of x[rows, h], bit-identical to
 * tensor_ops::layer_norm under `contract`: row_mean[r] and row_inv[r] =
 * 1 / sqrt(var + eps) from the CPU loop's sequential sums, and
 * y = (x - mean) * inv * weight + bias.  y, row_mean and row_inv may each be
 * NULL (y NULL: statistics only); y == x (in place) is allowed. */
int moe_layer_norm(moe_ctx* ctx, const float* x, const float* weight,
                   const float* bias, float eps, int64_t rows, int64_t h,
                   int contract, float* y, float* row_mean, float* row_inv,
                   void* stream);

/* ---- RMS norm over the last axis of x[rows, h]: row_inv[r] =
 * 1 / sqrt(ss / h + eps), ss = one float accumulator of x*x over the row in
 * order (fused multiply-add under MOE_CONTRACT_FMA), and
 * y = x * inv * weight.  y and row_inv may each be NULL; y == x is allowed.
 * No reference counterpart (config 5 names RMSNorm; the reference's norm is
 * tensor_ops::layer_norm). */
int moe_rms_norm(moe_ctx* ctx, const float* x, const float* weight, float eps,
                 int64_t rows, int64_t h, int contract, float* y,
                 float* row_inv, void* stream);

/* ---- decoder pieces around the MoE block (config 5's prefill).
 * moe_rope_table: host function, no device work: table[pos][j] = (cosf(pos *
 *   inv_j), sinf(pos * inv_j)), inv_j = powf(theta, -2j/head_dim), for pos <
 *   positions and j < head_dim/2 -- the libm calls of the reference's
 *   host-built table (src/model.cu:1784-1798); `table` is host memory of
 *   positions * head_dim floats.  Copy it to the device for moe_rope.
 * moe_rope: RoPE in place on q [batch*seq_len, q_heads*head_dim] and k
 *   [batch*seq_len, kv_heads*head_dim] with a device copy of that table
 *   (table_positions >= first_pos + seq_len rows); row r is at position
 *   first_pos + r % seq_len (first_pos = seq_len - 1 with seq_len 1 rotates
 *   one row per sequence at its last position, as rope_rows<2> does);
 *   pair (x0, x1) = (x[j], x[j + head_dim/2]) of each head becomes
 *   (x0*c - x1*s, x1*c + x0*s), each product rounded on its own:
 *   bit-identical to tensor_ops::apply_rope and rope_rows
 *   (src/model.cu:1046-1083) given the table.
 * moe_attention: out = softmax(q k^T / sqrt(head_dim), causal, keys within
 *   `window` positions (0 = unlimited)) v per sequence and head; q and out
 *   [batch*seq_len, q_heads*head_dim], k and v [batch*seq_len,
 *   kv_heads*head_dim], query head h reads key head h / (q_heads/kv_heads).
 *   16-byte aligned buffers.  head_dim 64 or 128: one fused pass, any
 *   seq_len, no workspace.  Other head_dims: head_dim and seq_len multiples
 *   of 16 (MOE_ERR_UNSUPPORTED otherwise), batch*q_heads*seq_len^2 floats of
 *   workspace.
 * moe_attention_last: the same attention for the last position of every
 *   sequence only (the rows the model's logits read): q [batch,
 *   q_heads*head_dim], one row per sequence, against k, v [batch*seq_len,
 *   kv_heads*head_dim]; out [batch, q_heads*head_dim].  Every sum runs in
 *   the reference loop's order, so it is bit-identical to that loop given
 *   the same q, k, v.  Any head_dim and seq_len; batch*q_heads*seq_len
 *   floats of workspace.
 * moe_rope_rows: moe_rope with row r at positions[r] (device int32 [rows],
 *   e.g. the depths of prefix-trie nodes); positions outside [0,
 *   table_positions) are clamped into the table.
 * moe_attention_paths: query row i of q [nq, q_heads*head_dim] attends over
 *   the key rows key_rows[key_beg[i] .. key_end[i]) of k, v [kv_rows,
 *   kv_heads*head_dim], listed by ascending position and ending at the
 *   query's own (a prefix-trie node's root path); the last `window` of them
 *   are visible (0 = all).  out [nq, q_heads*head_dim].  Every sum runs in
 *   the reference loop's order: bit-identical to it given the same q, k, v.
 *   max_len bounds every list length; key_total is the length of key_rows
 *   (every list must lie inside it).  Lists
 *   up to 8192 keys use no workspace; longer ones use key_total*q_heads
 *   floats and must not overlap each other in key_rows.  Key indices are
 *   clamped into [0, kv_rows); a list outside key_rows or longer than max_len
 *   allows gives NaN rows instead of reading or writing out of bounds.
 * moe_add: a += b elementwise.  moe_add_bias: a[r, c] += bias[c].
 * moe_embed: out[i, :] = table[tokens[i], :] (table [vocab, d]); a token
 *   outside [0, vocab) gives a zero row. */
int moe_rope_table(float theta, int64_t head_dim, int64_t positions, float* table);
int moe_rope(moe_ctx* ctx, float* q, float* k, const float* table,
             int64_t table_positions, int64_t batch, int64_t seq_len,
             int64_t first_pos, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
             void* stream);
int moe_attention(moe_ctx* ctx, const float* q, const float* k, const float* v,
                  float* out, int64_t batch, int64_t seq_len, int64_t q_heads,
                  int64_t kv_heads, int64_t head_dim, int64_t window, void* stream);
int moe_attention_last(moe_ctx* ctx, const float* q, const float* k, const float* v,
                       float* out, int64_t batch, int64_t seq_len, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, int64_t window, void* stream);
int moe_rope_rows(moe_ctx* ctx, float* q, float* k, const float* table,
                  int64_t table_positions, const int32_t* positions, int64_t rows,
                  int64_t q_heads, int64_t kv_heads, int64_t head_dim, void* stream);
int moe_attention_paths(moe_ctx* ctx, const float* q, const float* k, const float* v,
                        float* out, int64_t nq, int64_t kv_rows, const int32_t* key_rows,
                        const int32_t* key_beg, const int32_t* key_end, int64_t max_len,
                        int64_t key_total, int64_t q_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t window, void* stream);
int moe_add(moe_ctx* ctx, float* a, const float* b, int64_t n, void* stream);
int moe_add_bias(moe_ctx* ctx, float* a, const float* bias, int64_t rows,
                 int64_t cols, void* stream);
int moe_embed(moe_ctx* ctx, const float* table, const int32_t* tokens, int64_t n,
              int64_t d, int64_t vocab, float* out, void* stream);

/* ---- router gate logits[T,E] = x[T,d] Wg[E,d]^T with one k-ascending fp32
 * accumulator per output: bit-identical to the CPU path under `contract`. */
int moe_gate_logits(moe_ctx* ctx, const float* x, const float* gate_w,
                    float* logits, int64_t T, int64_t d, int64_t E,
                    int contract, void* stream);

/* ---- top-k routing of logits[T,E] (+ expert_bias[E] when not NULL).
 * topk_idx[T,k] (int32, selection order) and topk_w[T,k]. */
int moe_route(moe_ctx* ctx, const float* logits, const float* expert_bias,
              int64_t T, int64_t E, int64_t k, int mode, float quantum,
              float tie_eps, int32_t* topk_idx, float* topk_w, void* stream);

/* ---- stable bucket sort of the T*k (token, slot) pairs by expert.
 * expert_offsets[E+1]; perm[T*k]: token of each packed row, tokens ascending
 * within an expert; inv[T*k]: packed row of pair (t, s) at t*k+s.
 * Every row of topk_idx must hold k distinct experts in [0, E). */
int moe_permute(moe_ctx* ctx, const int32_t* topk_idx, int64_t T, int64_t k,
                int64_t E, int32_t* expert_offsets, int32_t* perm,
                int32_t* inv, void* stream);

/* ---- expert FFN over packed rows, one grouped launch per projection.
 * Packed row r of expert e (expert_offsets[e] <= r < expert_offsets[e+1])
 * reads x[perm[r], :].  h[T*k, d_ff] is the hidden activation (written),
 * out_rows[T*k, d] the expert outputs in packed order.
 * w1, w3: [E, d_ff, d]; w2: [E, d, d_ff]; w3 is ignored for SILU_MLP.
 * Where the planner runs a projection stream-K, or w1/w3 on the grouped
 * skinny kernel split over K (few rows per expert), its partial tiles or
 * split sums go to the context's workspace, which the call grows if it is
 * too small (a device
 * synchronisation, a free and an allocation: not allowed under graph
 * capture).  moe_ctx_reserve with a desc of the same T, k, d, d_ff and E
 * sizes it beforehand, after which the call allocates nothing. */
int moe_expert_ffn_grouped(moe_ctx* ctx, const float* x, const int32_t* perm,
                           const int32_t* expert_offsets, const float* w1,
                           const float* w3, const float* w2, int act,
                           int64_t T, int64_t k, int64_t d, int64_t d_ff,
                           int64_t E, float* h, float* out_rows, void* stream);

/* ---- y[t,:] = sum over t's experts in ascending expert id of
 * topk_w[t,s] * out_rows[inv[t,s], :], starting from zero (+ resid[t,:]
 * added last when resid is not NULL). */
int moe_combine(moe_ctx* ctx, const float* out_rows, const int32_t* topk_idx,
                const float* topk_w, const int32_t* inv, const float* resid,
                float* y, int64_t T, int64_t k, int64_t d, int contract,
                void* stream);

/* ---- the whole MoE layer: [layer norm ->] gate -> route -> permute ->
 * expert FFN -> combine [+ x].  topk_idx_out [T,k] / topk_w_out [T,k] may be
 * NULL. */
int moe_layer_forward(moe_ctx* ctx, const moe_layer_desc* desc,
                      const moe_layer_weights* weights, const float* x,
                      float* y, int32_t* topk_idx_out, float* topk_w_out,
                      void* stream);

/* ---- moe_layer_forward without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * layer's workspace (logits, routing, permutation, hidden rows, w2 partials,
 * norm statistics, stream-K partial tiles) lives in a fixed 256 MiB array the
 * library holds on every GPU it runs on, until the process ends; a layer
 * needing more is rejected with MOE_ERR_INVALID.  Every layer up to 4,160
 * tokens at config 5's shape fits (3,840 behind its RMS norm), up to 3,680
 * at the reference's (1,552 behind its layer norm); some larger ones fit as
 * well, since the plan's K splits and stream-K grid change with the token
 * count (moe_ctx_reserve on a fresh context, then moe_ctx_workspace_bytes,
 * gives a layer's need).  The call allocates nothing and records no timing events.
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (two streams, two threads, two
 * contexts) race and must be serialised by the caller.  Same arguments,
 * results and errors as moe_layer_forward otherwise. */
int moe_layer_forward_noalloc(moe_ctx* ctx, const moe_layer_desc* desc,
                              const moe_layer_weights* weights, const float* x,
                              float* y, int32_t* topk_idx_out, float* topk_w_out,
                              void* stream);

/* ---- how the grouped expert GEMMs deal their tiles on this context: mode
 * -1 (the default) lets the planner choose per launch, 0 always runs one
 * tile per workgroup, 1 always runs stream-K (every workgroup the same
 * number of K steps, tiles cut at range boundaries joined by a fix-up
 * launch) wherever the direct-load path applies.  Results of the two differ
 * only in the rounding of the cut tiles' K sums.  Only the default lets the
 * planner run layers with few rows per expert (32 or fewer on average) on
 * the grouped skinny kernel instead of tiles.  No reference counterpart:
 * a tuning and testing control (the environment variable MOE_SK = 0 / 1
 * sets the process default). */
int moe_ctx_set_stream_k(moe_ctx* ctx, int mode);

/* ---- the number of K splits moe_layer_forward(desc) runs its w2 GEMM with
 * on this context's device (its combine then reads that many partial row
 * buffers).  No reference counterpart: an introspection query for
 * measurement tools. */
int moe_layer_w2_splits(moe_ctx* ctx, const moe_layer_desc* desc, int32_t* splits);

/* ---- the plan moe_sgemm_nn (nn != 0) or moe_sgemm_nt runs an M x N x K
 * product with on this context's device, assuming 16-byte aligned operands:
 * the tile shape id (0 128x128, 1 64x128, 2 32x128, 3 256x128, 4 the skinny
 * kernel, 5 the K-group tile) and its K splits.  No reference counterpart:
 * an introspection query for tests and measurement tools. */
int moe_sgemm_plan(moe_ctx* ctx, int nn, int64_t M, int64_t N, int64_t K, int32_t* tile,
                   int32_t* splits);

#ifdef __cplusplus
}
#endif
#endif
