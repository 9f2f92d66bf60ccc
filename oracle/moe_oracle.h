/*
 * moe_oracle.h -- CPU restatement of the reference MoE forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the C++
 * drop-in, bench.py's GPU leg) may call, link or load this code.  It is used
 * by tests/ as the parity checker, by __graft_entry__.smoke() as the checker,
 * and by bench.py's cpu_baseline leg as the timed CPU path.
 *
 * Every function restates one piece of songsnim/accelerating-MoE-inference's
 * CPU path (paths relative to the reference root):
 *   src/tensor.cu:132-173   accurate_exp, matmul_transposed, mul, silu
 *   src/layer.cu:18-103     Linear / PhiMLP / PhiMoE::route / PhiMoE::forward
 *   docs/microworld/exp-003-moe-bench.cu:27   the LCG fill_rand
 * The loop nests, the k-ascending single accumulator, the OpenMP-over-rows
 * schedule and a bounds-checked element access are kept, so that the timing
 * of this code stands for the reference's CPU path.
 *
 * Floating-point contraction is explicit (the file is compiled with
 * -ffp-contract=off): ORC_CONTRACT_FMA computes `acc += a*b` as fmaf(a,b,acc),
 * which is what g++ -O3 -march=native emits on an FMA host and what the
 * reference's CUDA gate kernel emits; ORC_CONTRACT_NONE rounds the product and
 * the sum separately, which is what the reference host without FMA (Xeon
 * E5-2650, docs/exploration-002.md:17-19) executed.
 *
 * Parity status per function is recorded in the header comment of each
 * definition in moe_oracle.c.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_CONTRACT_NONE = 0, ORC_CONTRACT_FMA = 1 };
enum { ORC_ROUTER_PHI_QUANT = 0, ORC_ROUTER_SOFTMAX_TOPK = 1 };
enum { ORC_ACT_SWIGLU = 0, ORC_ACT_SILU_MLP = 1 };

/* Returns 0 on success, nonzero on a shape / argument error. */

void orc_lcg_fill(float* out, size_t n, uint32_t seed);

int orc_matmul_nt(const float* a, const float* b, float* c,
                  size_t m, size_t n, size_t k, int contract);
int orc_matmul_nn(const float* a, const float* b, float* c,
                  size_t m, size_t n, size_t k, int contract);
void orc_silu(const float* x, float* y, size_t n);
void orc_mul(const float* a, const float* b, float* c, size_t n);
int orc_layer_norm(const float* x, const float* weight, const float* bias,
                   float eps, size_t rows, size_t h, int contract, float* y,
                   float* row_mean, float* row_inv);
int orc_rms_norm(const float* x, const float* weight, float eps, size_t rows,
                 size_t h, int contract, float* y, float* row_inv);
int orc_rope_table(float theta, size_t head_dim, size_t positions, float* table);
int orc_rope(float* q, float* k, const float* table, size_t batch, size_t seq_len,
             size_t q_heads, size_t kv_heads, size_t head_dim);
int orc_attention(const float* q, const float* k, const float* v, float* out,
                  size_t batch, size_t seq_len, size_t q_heads, size_t kv_heads,
                  size_t head_dim, size_t window);

int orc_route(const float* logits, const float* expert_bias,
              size_t T, size_t E, size_t k, int mode,
              float quantum, float tie_eps,
              int32_t* topk_idx, float* topk_w);

int orc_permute(const int32_t* topk_idx, size_t T, size_t k, size_t E,
                int32_t* expert_offsets, int32_t* perm, int32_t* inv);

int orc_expert_ffn(const float* x, size_t T, size_t d,
                   const int32_t* perm, const int32_t* expert_offsets,
                   size_t E, const float* w1, const float* w3,
                   const float* w2, size_t d_ff, int act, int contract,
                   float* out_rows);

int orc_combine(const float* out_rows, const int32_t* topk_idx,
                const float* topk_w, const int32_t* inv, size_t T, size_t k,
                size_t d, int contract, float* y);

int orc_moe_forward(const float* x, size_t T, size_t d, const float* gate_w,
                    const float* expert_bias, size_t E, size_t k,
                    const float* w1, const float* w3, const float* w2,
                    size_t d_ff, int act, int router_mode, float quantum,
                    float tie_eps, int contract, float* y,
                    int32_t* topk_idx_out, float* topk_w_out);

/* Number of OpenMP threads the oracle runs with (0 = library default). */
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
