// PhiTinyMoEModel of the drop-in API (include/model.h:10-24 of the
// reference): the whole decoder on the GPU over the C ABI.
//
// generate() packs the batch as the rows of a prefix trie (one row per
// distinct prefix: a shared prefix is computed once, src/model.cu:1624-1680),
// runs every layer over those rows with each node attending over its root
// path, prunes the last layer to the last node of every sequence
// (src/model.cu:1889-1960), and applies the final norm and lm_head to those
// rows only.  generate_decode() is the reference's greedy loop
// (src/model.cu:2061-2101), with the still-running sequences of a step
// batched into one generate().
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "device.h"
#include "layer.h"
#include "model_loader.h"
#include "tensor.h"

class PhiTinyMoEModel {
public:
    // Loads model.embed_tokens.weight, model.layers.{i}.* for every layer
    // the file holds (i = 0, 1, ... while model.layers.{i}.input_layernorm
    // .weight exists), model.norm.{weight,bias} and lm_head.{weight,bias};
    // the vocabulary is lm_head's row count.
    explicit PhiTinyMoEModel(const std::string& model_file);
    ~PhiTinyMoEModel();

    PhiTinyMoEModel(const PhiTinyMoEModel&) = delete;
    PhiTinyMoEModel& operator=(const PhiTinyMoEModel&) = delete;

    // logits [1, vocab] of the last position of input_ids.
    void forward(const std::vector<int>& input_ids, Tensor& logits) const;
    // logits [batch, vocab] of the last position of every sequence, in input order.
    void generate(const std::vector<std::vector<int>>& input_ids, Tensor& logits) const;
    // Greedy decode: logits [batch, max_new_tokens, vocab] (step 0 = the
    // prefill's last-position logits; rows after a sequence's EOS stay 0) and
    // the generated ids (ending at EOS_TOKEN_ID when it is produced).
    void generate_decode(const std::vector<std::vector<int>>& input_ids,
                         std::size_t max_new_tokens, Tensor& logits,
                         std::vector<std::vector<int>>& generated_ids) const;

    std::size_t num_layers() const { return layers_.size(); }
    std::size_t vocab_size() const { return vocab_; }
    std::size_t hidden_size() const { return hidden_; }

private:
    ModelLoader loader_;
    std::shared_ptr<const moe_dropin::DeviceBuffer> embed_, norm_w_, norm_b_, lm_w_, lm_b_;
    std::vector<std::unique_ptr<PhiDecoderLayer>> layers_;
    std::size_t hidden_ = 0, vocab_ = 0, embed_rows_ = 0;
    // Activations and trie arrays, grow-only: generate() of a shape seen
    // before allocates nothing (so, like the reference's generate(), a model
    // is not safe for concurrent calls).
    mutable moe_dropin::Scratch scratch_;
    // Page-locked output reserve (the reference's pinned_out_,
    // include/model.h:123): the first generate() whose logits Tensor is not
    // page-locked and large enough takes it over, so the logits copy runs
    // at full DMA speed, chunk by chunk behind the lm_head.
    static constexpr std::size_t kPinnedOutBytes = std::size_t(256) << 20;
    mutable Tensor pinned_out_;
    struct CopyStream;  // the copy stream and the lm_head chunks' events
    std::unique_ptr<CopyStream> copy_;
};
