// Layers of the drop-in API: the reference's Linear, PhiMLP and PhiMoE
// (include/layer.h:11-37) with the same constructors, forward signatures,
// weight names and exception types, re-implemented over the C ABI.  Weights
// are uploaded to HBM once, at construction (the reference's GPU engine does
// the same, src/model.cu:1491-1513); forward() copies the input in, runs the
// HIP path and copies the result out.
//
// PhiAttention / PhiDecoderLayer (include/layer.h:39-56) are outside the MoE
// hot path and are not provided.
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
}

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

private:
    std::shared_ptr<const moe_dropin::DeviceBuffer> gate_, w1_, w3_, w2_;
    std::size_t experts_ = 0, hidden_ = 0, ff_ = 0;
    int contract_ = MOE_CONTRACT_FMA;
};
