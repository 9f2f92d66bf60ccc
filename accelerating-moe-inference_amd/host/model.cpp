#include "model.h"

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <unordered_map>

#include "config.h"
#include "device.h"

namespace {

using moe_dropin::check;
using moe_dropin::DeviceBuffer;

std::shared_ptr<const DeviceBuffer> upload(const Tensor& t) {
    auto b = std::make_shared<DeviceBuffer>(t.size() * sizeof(float));
    b->upload(t.data(), t.size() * sizeof(float));
    return b;
}

enum ModelSlot : std::size_t {
    kX = kSlotModel, kY, kLast, kLastNorm, kLogits, kTok, kPos, kKeys, kOff, kLastIdx, kTailPos,
    kTailBeg, kTailEnd
};

// The prefix trie of a batch (src/model.cu:1624-1680): one node per distinct
// prefix in order of first appearance, with its token, depth and root path.
struct Trie {
    std::vector<int32_t> token, depth, parent, key_off, key_rows, last;
    std::size_t max_len = 0;
};

Trie build_trie(const std::vector<std::vector<int>>& seqs, std::size_t vocab) {
    Trie t;
    std::unordered_map<long long, int32_t> child;
    child.reserve(seqs.size() * 64);
    for (const std::vector<int>& seq : seqs) {
        if (seq.empty()) throw std::invalid_argument("empty input");
        if (seq.size() > apss26::MAX_POSITION_EMBEDDINGS)
            throw std::invalid_argument("sequence is too long");
        int32_t parent = -1;
        for (std::size_t si = 0; si < seq.size(); ++si) {
            const int token = seq[si];
            if (token < 0 || static_cast<std::size_t>(token) >= vocab)
                throw std::invalid_argument("token out of vocabulary");
            const long long key =
                (static_cast<long long>(parent) + 1) * static_cast<long long>(vocab) + token;
            const auto it = child.find(key);
            if (it != child.end()) {
                parent = it->second;
                continue;
            }
            const auto node = static_cast<int32_t>(t.token.size());
            t.token.push_back(token);
            t.parent.push_back(parent);
            t.depth.push_back(static_cast<int32_t>(si));
            child.emplace(key, node);
            parent = node;
        }
        t.last.push_back(parent);
    }
    const std::size_t n = t.token.size();
    t.key_off.assign(n + 1, 0);
    for (std::size_t i = 0; i < n; ++i) t.key_off[i + 1] = t.key_off[i] + t.depth[i] + 1;
    t.key_rows.resize(static_cast<std::size_t>(t.key_off[n]));
    for (std::size_t i = 0; i < n; ++i) {
        int32_t* dst = t.key_rows.data() + t.key_off[i];
        const int32_t p = t.parent[i];
        if (p >= 0)  // the parent's path is this node's minus its last entry
            for (int32_t j = 0; j < t.depth[i]; ++j) dst[j] = t.key_rows[t.key_off[p] + j];
        dst[t.depth[i]] = static_cast<int32_t>(i);
        t.max_len = std::max<std::size_t>(t.max_len, static_cast<std::size_t>(t.depth[i]) + 1);
    }
    return t;
}

}  // namespace

PhiTinyMoEModel::PhiTinyMoEModel(const std::string& model_file) : loader_(model_file) {
    const Tensor emb = loader_.load("model.embed_tokens.weight");
    if (emb.ndim() != 2) throw std::invalid_argument("model.embed_tokens.weight: weight must be 2-D");
    embed_rows_ = emb.size(0);
    hidden_ = emb.size(1);
    embed_ = upload(emb);
    for (std::size_t i = 0;
         loader_.has("model.layers." + std::to_string(i) + ".input_layernorm.weight"); ++i)
        layers_.push_back(std::make_unique<PhiDecoderLayer>(loader_, i));
    auto vec = [&](const std::string& name) {
        const Tensor t = loader_.load(name);
        if (t.size() != hidden_) throw std::invalid_argument(name + ": unexpected weight shape");
        return upload(t);
    };
    norm_w_ = vec("model.norm.weight");
    norm_b_ = vec("model.norm.bias");
    const Tensor lm = loader_.load("lm_head.weight");
    if (lm.ndim() != 2 || lm.size(1) != hidden_)
        throw std::invalid_argument("lm_head.weight: unexpected weight shape");
    vocab_ = lm.size(0);
    lm_w_ = upload(lm);
    if (loader_.has("lm_head.bias")) {
        const Tensor b = loader_.load("lm_head.bias");
        if (b.size() != vocab_) throw std::invalid_argument("lm_head.bias: bias shape");
        lm_b_ = upload(b);
    }
}

PhiTinyMoEModel::~PhiTinyMoEModel() = default;

void PhiTinyMoEModel::forward(const std::vector<int>& input_ids, Tensor& logits) const {
    if (input_ids.empty()) throw std::invalid_argument("empty input");
    generate({input_ids}, logits);
}

void PhiTinyMoEModel::generate(const std::vector<std::vector<int>>& input_ids,
                               Tensor& logits) const {
    if (input_ids.empty()) throw std::runtime_error("generate received an empty input batch");
    const std::size_t batch = input_ids.size(), h = hidden_;
    // tokens index the embedding table too: the smaller of the two bounds
    const Trie t = build_trie(input_ids, std::min(vocab_, embed_rows_));
    const std::size_t rows = t.token.size();

    std::vector<int32_t> tail_pos(batch), tail_beg(batch), tail_end(batch);
    for (std::size_t b = 0; b < batch; ++b) {
        tail_pos[b] = t.depth[t.last[b]];
        tail_beg[b] = t.key_off[t.last[b]];
        tail_end[b] = t.key_off[t.last[b] + 1];
    }
    moe_dropin::Scratch& sc = scratch_;
    const int32_t* d_tok = sc.upload(kTok, t.token.data(), rows);
    const int32_t* d_last = sc.upload(kLastIdx, t.last.data(), batch);
    NodeRows nb;
    nb.rows = rows;
    nb.positions = sc.upload(kPos, t.depth.data(), rows);
    nb.key_rows = sc.upload(kKeys, t.key_rows.data(), t.key_rows.size());
    nb.key_off = sc.upload(kOff, t.key_off.data(), t.key_off.size());
    nb.key_total = t.key_rows.size();
    nb.max_len = t.max_len;
    nb.tail_rows = batch;
    nb.tail_nodes = d_last;
    nb.tail_positions = sc.upload(kTailPos, tail_pos.data(), batch);
    nb.tail_key_beg = sc.upload(kTailBeg, tail_beg.data(), batch);
    nb.tail_key_end = sc.upload(kTailEnd, tail_end.data(), batch);

    moe_ctx* ctx = moe_dropin::context();
    float* x = sc.f32(kX, rows * h);
    float* y = sc.f32(kY, rows * h);
    float* last = sc.f32(kLast, batch * h);
    float* last_n = sc.f32(kLastNorm, batch * h);
    float* out = sc.f32(kLogits, batch * vocab_);
    check(moe_embed(ctx, embed_->as<float>(), d_tok, static_cast<int64_t>(rows),
                    static_cast<int64_t>(h), static_cast<int64_t>(embed_rows_), x, nullptr));
    if (layers_.empty()) {
        check(moe_embed(ctx, x, d_last, static_cast<int64_t>(batch), static_cast<int64_t>(h),
                        static_cast<int64_t>(rows), last, nullptr));
    }
    for (std::size_t l = 0; l < layers_.size(); ++l) {
        const bool tail = l + 1 == layers_.size();
        layers_[l]->forward_nodes(x, tail ? last : y, nb, tail, sc);
        if (!tail) std::swap(x, y);
    }
    check(moe_layer_norm(ctx, last, norm_w_->as<float>(), norm_b_->as<float>(), apss26::NORM_EPS,
                         static_cast<int64_t>(batch), static_cast<int64_t>(h), MOE_CONTRACT_FMA,
                         last_n, nullptr, nullptr, nullptr));
    check(moe_sgemm_nt(ctx, last_n, lm_w_->as<float>(), lm_b_ ? lm_b_->as<float>() : nullptr, out,
                       static_cast<int64_t>(batch), static_cast<int64_t>(vocab_),
                       static_cast<int64_t>(h), nullptr));
    logits = Tensor({batch, vocab_});
    sc.download(kLogits, logits.data(), batch * vocab_ * sizeof(float));
}

void PhiTinyMoEModel::generate_decode(const std::vector<std::vector<int>>& input_ids,
                                      std::size_t max_new_tokens, Tensor& logits,
                                      std::vector<std::vector<int>>& generated_ids) const {
    if (input_ids.empty())
        throw std::runtime_error("generate_decode received an empty input batch");
    if (max_new_tokens == 0) throw std::invalid_argument("max_new_tokens must be positive");
    const std::size_t batch = input_ids.size();
    logits = Tensor({batch, max_new_tokens, vocab_});
    generated_ids.assign(batch, {});
    std::vector<std::vector<int>> prefix = input_ids;
    std::vector<std::size_t> active(batch);
    for (std::size_t b = 0; b < batch; ++b) active[b] = b;
    for (std::size_t step = 0; step < max_new_tokens && !active.empty(); ++step) {
        std::vector<std::vector<int>> rows;
        rows.reserve(active.size());
        for (std::size_t b : active) rows.push_back(prefix[b]);
        Tensor step_logits;
        generate(rows, step_logits);
        std::vector<std::size_t> still;
        for (std::size_t i = 0; i < active.size(); ++i) {
            const std::size_t b = active[i];
            const float* row = step_logits.data() + i * vocab_;
            int next = 0;  // the first maximum, as the reference's scan
            for (std::size_t v = 1; v < vocab_; ++v)
                if (row[v] > row[next]) next = static_cast<int>(v);
            std::copy(row, row + vocab_, logits.data() + (b * max_new_tokens + step) * vocab_);
            generated_ids[b].push_back(next);
            if (next == apss26::EOS_TOKEN_ID) continue;
            prefix[b].push_back(next);
            still.push_back(b);
        }
        active.swap(still);
    }
}
