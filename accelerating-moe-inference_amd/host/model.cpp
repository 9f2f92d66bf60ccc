#include "model.h"

#include <algorithm>
#include <cstdint>
#include <numeric>
#include <stdexcept>
#include <string>

#include <hip/hip_runtime.h>

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
    kTailBeg, kTailEnd, kUTok, kNodeU, kUX
};

// The prefix trie of a batch: one node (one activation row) per distinct
// prefix, so a prefix several sequences share is computed once -- the row set
// of the reference's generate() (src/model.cu:1624-1680); node order does not
// change any row's arithmetic.  Built by sorting: in lexicographic order a
// sequence shares with its predecessor exactly their longest common prefix,
// so one walk over the sorted batch creates the nodes in depth-first order,
// each new node extending the root path the walk holds, which is also the
// node's attention key list.
struct Trie {
    std::vector<int32_t> token, depth;  // per node
    std::vector<int32_t> key_off;       // node i's key list: key_rows[key_off[i] .. key_off[i+1])
    std::vector<int32_t> key_rows;      // root paths, each ending at its own node
    std::vector<int32_t> last;          // per input sequence: the node of its last token
    std::size_t max_len = 0;
};

Trie build_trie(const std::vector<std::vector<int>>& seqs, std::size_t vocab) {
    // validation in input order, so an input raises the reference's error
    for (const std::vector<int>& seq : seqs) {
        if (seq.empty()) throw std::invalid_argument("empty input");
        if (seq.size() > apss26::MAX_POSITION_EMBEDDINGS)
            throw std::invalid_argument("sequence is too long");
        for (const int token : seq)
            if (token < 0 || static_cast<std::size_t>(token) >= vocab)
                throw std::invalid_argument("token out of vocabulary");
    }
    std::vector<std::size_t> order(seqs.size());
    std::iota(order.begin(), order.end(), std::size_t(0));
    std::stable_sort(order.begin(), order.end(),
                     [&](std::size_t a, std::size_t b) { return seqs[a] < seqs[b]; });
    Trie t;
    t.last.assign(seqs.size(), -1);
    t.key_off.push_back(0);
    std::vector<int32_t> walk;  // walk[p]: the node at depth p of the current sequence
    const std::vector<int>* prev = nullptr;
    for (const std::size_t b : order) {
        const std::vector<int>& seq = seqs[b];
        std::size_t shared = 0;
        if (prev != nullptr)
            shared = static_cast<std::size_t>(
                std::mismatch(seq.begin(), seq.end(), prev->begin(), prev->end()).first -
                seq.begin());
        walk.resize(shared);
        for (std::size_t p = shared; p < seq.size(); ++p) {
            walk.push_back(static_cast<int32_t>(t.token.size()));
            t.token.push_back(seq[p]);
            t.depth.push_back(static_cast<int32_t>(p));
            t.key_rows.insert(t.key_rows.end(), walk.begin(), walk.end());
            t.key_off.push_back(static_cast<int32_t>(t.key_rows.size()));
        }
        t.last[b] = walk[seq.size() - 1];
        t.max_len = std::max(t.max_len, seq.size());
        prev = &seq;
    }
    return t;
}

// lm_head row chunks: each chunk's logits go home while the next chunk's
// product runs (src/model.cu:2031-2050 does the same with 4 chunks)
constexpr std::size_t kLmChunks = 4;

}  // namespace

// A non-blocking stream of default priority for the logits copies and one
// event per lm_head chunk, created with the model and destroyed with it.
struct PhiTinyMoEModel::CopyStream {
    hipStream_t stream = nullptr;
    hipEvent_t done[kLmChunks] = {};
    CopyStream() {
        check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        for (hipEvent_t& e : done)
            check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    }
    ~CopyStream() {
        for (hipEvent_t e : done)
            if (e != nullptr) (void)hipEventDestroy(e);
        if (stream != nullptr) (void)hipStreamDestroy(stream);
    }
    CopyStream(const CopyStream&) = delete;
    CopyStream& operator=(const CopyStream&) = delete;
    static void check_hip(hipError_t e, const char* what) {
        if (e != hipSuccess)
            throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    }
};

PhiTinyMoEModel::PhiTinyMoEModel(const std::string& model_file)
    : loader_(model_file),
      pinned_out_({kPinnedOutBytes / sizeof(float)}, Tensor::Alloc::Pinned),
      copy_(std::make_unique<CopyStream>()) {
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
    // The first layer's input norm and q/k/v over the distinct tokens of the
    // nodes (a node's first-layer input is its token's embedding row), in
    // order of first appearance (src/model.cu:1682-1705,1905-1935), when
    // tokens repeat and the first layer is not also the pruned last one.
    NodeRows nb0 = nb;
    if (layers_.size() > 1) {
        std::vector<int32_t> utok, node_u(rows);
        std::vector<int32_t> first(std::min(vocab_, embed_rows_), -1);
        for (std::size_t n = 0; n < rows; ++n) {
            int32_t& u = first[static_cast<std::size_t>(t.token[n])];
            if (u < 0) {
                u = static_cast<int32_t>(utok.size());
                utok.push_back(t.token[n]);
            }
            node_u[n] = u;
        }
        if (utok.size() < rows) {
            const std::size_t U = utok.size();
            float* ux = sc.f32(kUX, U * h);
            check(moe_embed(ctx, embed_->as<float>(), sc.upload(kUTok, utok.data(), U),
                            static_cast<int64_t>(U), static_cast<int64_t>(h),
                            static_cast<int64_t>(embed_rows_), ux, nullptr));
            nb0.urows = U;
            nb0.ux = ux;
            nb0.node_u = sc.upload(kNodeU, node_u.data(), rows);
        }
    }
    for (std::size_t l = 0; l < layers_.size(); ++l) {
        const bool tail = l + 1 == layers_.size();
        layers_[l]->forward_nodes(x, tail ? last : y, l == 0 ? nb0 : nb, tail, sc);
        if (!tail) std::swap(x, y);
    }
    check(moe_layer_norm(ctx, last, norm_w_->as<float>(), norm_b_->as<float>(), apss26::NORM_EPS,
                         static_cast<int64_t>(batch), static_cast<int64_t>(h), MOE_CONTRACT_FMA,
                         last_n, nullptr, nullptr, nullptr));
    // Where the logits land: the caller's Tensor if it is page-locked and
    // large enough, else the model's page-locked reserve (moved into it, as
    // the reference's generate() does), else ordinary host memory.
    const std::size_t n = batch * vocab_;
    const float* lm_b = lm_b_ ? lm_b_->as<float>() : nullptr;
    const bool caller_pinned = logits.alloc() == Tensor::Alloc::Pinned &&
                               logits.capacity() >= n && logits.data() != nullptr;
    if (!caller_pinned && pinned_out_.data() != nullptr && pinned_out_.capacity() >= n)
        logits = std::move(pinned_out_);
    if (logits.alloc() == Tensor::Alloc::Pinned && logits.capacity() >= n &&
        logits.data() != nullptr) {
        logits.reshape_within_capacity({batch, vocab_});
        // lm_head in row chunks; chunk c's copy (on the copy stream, after
        // the chunk's event) overlaps chunk c + 1's product
        const std::size_t chunk = (batch + kLmChunks - 1) / kLmChunks;
        CopyStream& cs = *copy_;
        // every copy enqueued below has ended when this call returns, also
        // when a later launch throws (the copies write into `logits`)
        struct Drain {
            hipStream_t s;
            ~Drain() { (void)hipStreamSynchronize(s); }
        } drain{cs.stream};
        std::size_t c = 0;
        for (std::size_t r0 = 0; r0 < batch; r0 += chunk, ++c) {
            const std::size_t rc = std::min(chunk, batch - r0);
            check(moe_sgemm_nt(ctx, last_n + r0 * h, lm_w_->as<float>(), lm_b, out + r0 * vocab_,
                               static_cast<int64_t>(rc), static_cast<int64_t>(vocab_),
                               static_cast<int64_t>(h), nullptr));
            CopyStream::check_hip(hipEventRecord(cs.done[c], nullptr), "hipEventRecord lm_head");
            CopyStream::check_hip(hipStreamWaitEvent(cs.stream, cs.done[c], 0),
                                  "hipStreamWaitEvent lm_head");
            CopyStream::check_hip(hipMemcpyAsync(logits.data() + r0 * vocab_, out + r0 * vocab_,
                                                 rc * vocab_ * sizeof(float),
                                                 hipMemcpyDeviceToHost, cs.stream),
                                  "hipMemcpyAsync logits");
        }
        CopyStream::check_hip(hipStreamSynchronize(cs.stream), "hipStreamSynchronize logits");
        return;  // (the drain finds the stream idle)
    }
    check(moe_sgemm_nt(ctx, last_n, lm_w_->as<float>(), lm_b, out, static_cast<int64_t>(batch),
                       static_cast<int64_t>(vocab_), static_cast<int64_t>(h), nullptr));
    // pageable output: the caller's Tensor is reused when it holds enough
    // elements; the copy goes through the drop-in's pinned staging
    if (logits.capacity() >= n && logits.data() != nullptr)
        logits.reshape_within_capacity({batch, vocab_});
    else
        logits = Tensor({batch, vocab_});
    auto lock = moe_dropin::io_lock();
    moe_dropin::to_host(logits.data(), out, n * sizeof(float));
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
    Tensor step_logits;  // one buffer for every step (it keeps the page-locked reserve)
    for (std::size_t step = 0; step < max_new_tokens && !active.empty(); ++step) {
        std::vector<std::vector<int>> rows;
        rows.reserve(active.size());
        for (std::size_t b : active) rows.push_back(prefix[b]);
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
