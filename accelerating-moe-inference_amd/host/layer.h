// Layers of the drop-in API: the reference's Linear, PhiMLP and PhiMoE
// (include/layer.h:11-37) with the same constructors, forward signatures,
// weight names and exception types, re-implemented over the C ABI.  Weights
// are uploaded to HBM once, at construction (the reference's GPU engine does
// the same, src/model.cu:1491-1513); forward() copies the input in, runs the
// HIP path and copies the result out.
//
// PhiAttention and PhiDecoderLayer (include/layer.h:39-56) keep the
// reference's constructors, weight names and forward(x, y) on one sequence
// x [s, hidden]; a decoder layer runs on the device from one upload of x to
// one download of y.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../include/moe_amd.h"
#include "config.h"
#include "model_loader.h"
#include "tensor.h"

namespace moe_dropin {
class DeviceBuffer;
class Scratch;
}

// Scratch slots of the trie-row path (the model's own start at kSlotModel).
enum NodeSlot : std::size_t {
    kSlotK, kSlotV, kSlotQ, kSlotAttn, kSlotTailIn, kSlotNorm, kSlotAttnOut, kSlotTailResid,
    kSlotUNorm, kSlotUQ, kSlotUK, kSlotUV,
    kSlotModel = 16
};

class Linear {
public:
    Linear() = default;
    Linear(const ModelLoader& loader, const std::string& weight, const std::string& bias = "");
    // y[rows, out] = x[..., in] W^T (+ bias); y is reassigned.
    void forward(const Tensor& x, Tensor& y) const;

private:
    std::shared_ptr<const moe_dropin::DeviceBuffer> weight_, bias_;
    std::size_t out_ = 0, in_ = 0;
};

class PhiMLP {
public:
    PhiMLP(const ModelLoader& loader, const std::string& prefix);
    // y = w2 (silu(x w1^T) * (x w3^T)), shaped like x.
    void forward(const Tensor& x, Tensor& y) const;

private:
    std::shared_ptr<const moe_dropin::DeviceBuffer> w1_, w2_, w3_;
    std::size_t hidden_ = 0, ff_ = 0;
};

class PhiMoE {
public:
    // Loads model.layers.{layer_idx}.block_sparse_moe.{gate.weight,
    // experts.{e}.w1/w2/w3.weight}; the expert count is the gate's row count.
    // `contract` selects the gate/combine contraction (MOE_CONTRACT_FMA is
    // what the reference computes on an FMA host and on its GPU).
    PhiMoE(const ModelLoader& loader, std::size_t layer_idx, int contract = MOE_CONTRACT_FMA);
    // y[rows, h] = the MoE layer of x[rows, h]; y is reassigned.
    void forward(const Tensor& x, Tensor& y) const;
    // The same, also returning each token's experts in selection order
    // (rows x top_k) -- an extension for callers that audit routing.
    void forward(const Tensor& x, Tensor& y, std::vector<int32_t>* topk_idx) const;

    std::size_t num_experts() const { return experts_; }
    std::size_t hidden() const { return hidden_; }

    // The MoE block on device rows (an extension PhiDecoderLayer uses):
    // dy[rows, h] = (residual ? dx : 0) + MoE(norm(dx)), norm a MOE_NORM_*
    // with its [h] weight and bias; topk_idx (device, rows x top_k) may be null.
    void forward_device(const float* dx, float* dy, std::size_t rows, int norm,
                        const float* norm_w, const float* norm_b, int residual,
                        int32_t* topk_idx) const;

private:
    std::shared_ptr<const moe_dropin::DeviceBuffer> gate_, w1_, w3_, w2_;
    std::size_t experts_ = 0, hidden_ = 0, ff_ = 0;
    int contract_ = MOE_CONTRACT_FMA;
};

// Rows of a packed batch on the device (an extension the model uses): the
// nodes of a prefix trie over the batch's sequences (src/model.cu:1624-1680),
// one row per distinct prefix.  A node's keys are its root path.
struct NodeRows {
    std::size_t rows = 0;
    const int32_t* positions = nullptr;  // [rows] depth of each node
    const int32_t* key_rows = nullptr;   // root paths, flattened, ascending depth
    const int32_t* key_off = nullptr;    // [rows + 1] offsets into key_rows
    std::size_t key_total = 0, max_len = 0;
    // The pruned last layer's rows: the last node of every sequence.
    std::size_t tail_rows = 0;
    const int32_t* tail_nodes = nullptr;      // [tail_rows]
    const int32_t* tail_positions = nullptr;  // [tail_rows]
    const int32_t* tail_key_beg = nullptr;    // [tail_rows] their root paths in key_rows
    const int32_t* tail_key_end = nullptr;
    // Distinct-token rows (set for the first layer only, when they are fewer
    // than the nodes): a first-layer node's input row is its token's
    // embedding, so the input norm and the q/k/v projections depend on the
    // token alone (src/model.cu:1682-1705); they run over the distinct
    // tokens' rows ux[urows, hidden] and node n takes row node_u[n] of each
    // result (RoPE then at the node's own position).
    std::size_t urows = 0;
    const float* ux = nullptr;
    const int32_t* node_u = nullptr;  // [rows]
};

class PhiAttention {
public:
    // Loads model.layers.{layer_idx}.self_attn.{q,k,v,o}_proj.{weight,bias}
    // (a bias is optional, as in Linear); heads, key heads, head_dim, RoPE
    // theta and the sliding window are the apss26 constants.
    PhiAttention(const ModelLoader& loader, std::size_t layer_idx);
    // y[s, hidden] = o_proj(attention(rope(q_proj(x), k_proj(x)), v_proj(x)))
    // over one sequence x[s, hidden]; y is reassigned.
    void forward(const Tensor& x, Tensor& y) const;
    // Device rows (an extension): dx holds padded_rows(s) rows, those past s
    // zero; dy receives as many (rows past s are scratch).
    void forward_device(const float* dx, float* dy, std::size_t s) const;
    // s rounded up to the attention kernels' 16-row granule.
    static std::size_t padded_rows(std::size_t s) { return (s + 15) / 16 * 16; }
    // Trie rows (an extension): dn [rows, hidden] normalised input; dy gets
    // o_proj(attention) + resid for every node, or (tail) for the tail rows
    // only (resid: the residual rows, added in the o-projection's store as
    // src/model.cu:1965 does).
    // With nb.urows set, dn holds the normalised distinct-token rows
    // [urows, hidden] instead, and the projections are expanded to the
    // nodes by row gathers (not for the tail).
    void forward_nodes(const float* dn, float* dy, const float* resid, const NodeRows& nb,
                       bool tail, moe_dropin::Scratch& sc) const;
    std::size_t hidden() const { return hidden_; }

private:
    std::shared_ptr<const moe_dropin::DeviceBuffer> wq_, bq_, wk_, bk_, wv_, bv_, wo_, bo_, rope_;
    std::size_t hidden_ = 0, rope_positions_ = 0;
};

class PhiDecoderLayer {
public:
    // Loads model.layers.{layer_idx}.{input_layernorm,post_attention_layernorm}
    // .{weight,bias}, the attention and the MoE block of the layer.
    PhiDecoderLayer(const ModelLoader& loader, std::size_t layer_idx);
    // y = h + MoE(layer_norm(h)), h = x + attention(layer_norm(x)); y is reassigned.
    void forward(const Tensor& x, Tensor& y) const;
    // Trie rows (an extension): dx [rows, hidden] -> dy [rows, hidden], or
    // (tail) dy [tail_rows, hidden] for the last node of every sequence.
    void forward_nodes(const float* dx, float* dy, const NodeRows& nb, bool tail,
                       moe_dropin::Scratch& sc) const;

private:
    std::shared_ptr<const moe_dropin::DeviceBuffer> in_w_, in_b_, post_w_, post_b_;
    PhiAttention attention_;
    PhiMoE moe_;
};
