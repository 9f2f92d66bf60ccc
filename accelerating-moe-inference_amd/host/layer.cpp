#include "layer.h"

#include <mutex>
#include <numeric>
#include <stdexcept>

#include "device.h"

namespace {

using moe_dropin::check;
using moe_dropin::DeviceBuffer;

std::shared_ptr<const DeviceBuffer> upload(const Tensor& t) {
    auto b = std::make_shared<DeviceBuffer>(t.size() * sizeof(float));
    b->upload(t.data(), t.size() * sizeof(float));
    return b;
}

// Stacks equally shaped host tensors into one device array [n, ...].
std::shared_ptr<const DeviceBuffer> upload_stacked(const std::vector<Tensor>& ts) {
    const std::size_t each = ts.empty() ? 0 : ts.front().size() * sizeof(float);
    auto b = std::make_shared<DeviceBuffer>(each * ts.size());
    for (std::size_t i = 0; i < ts.size(); ++i) b->upload(ts[i].data(), each, i * each);
    return b;
}

void require_2d(const Tensor& t, std::size_t rows, std::size_t cols, const std::string& what) {
    if (t.ndim() != 2 || t.size(0) != rows || t.size(1) != cols)
        throw std::invalid_argument(what + ": unexpected weight shape");
}

// The RoPE cos/sin of `positions` positions (host libm, moe_rope_table) on
// the device.
std::shared_ptr<const DeviceBuffer> rope_table(std::size_t positions) {
    std::vector<float> t(positions * apss26::HEAD_DIM);
    check(moe_rope_table(apss26::ROPE_THETA, static_cast<int64_t>(apss26::HEAD_DIM),
                         static_cast<int64_t>(positions), t.data()));
    auto b = std::make_shared<DeviceBuffer>(t.size() * sizeof(float));
    b->upload(t.data(), t.size() * sizeof(float));
    return b;
}

// One table of MAX_POSITION_EMBEDDINGS positions shared by every layer.
std::shared_ptr<const DeviceBuffer> shared_rope_table() {
    static std::mutex mu;
    static std::shared_ptr<const DeviceBuffer> table;
    std::lock_guard<std::mutex> lock(mu);
    if (!table) table = rope_table(apss26::MAX_POSITION_EMBEDDINGS);
    return table;
}

// y takes `shape`, reusing its buffer when it holds enough elements (every
// element is overwritten by the caller's copy-out).
void shape_output(Tensor& y, std::vector<std::size_t> shape) {
    std::size_t n = 1;
    for (std::size_t d : shape) n *= d;
    if (y.capacity() >= n && y.data() != nullptr) y.reshape_within_capacity(std::move(shape));
    else y = Tensor(std::move(shape));
}

// Slots of the drop-in's per-call device buffers (moe_dropin::io_scratch).
enum IoSlot : std::size_t { kIoX, kIoY, kIoH, kIoIdx, kIoPerm, kIoOff, kIoQ, kIoK, kIoV, kIoA, kIoN };

void sgemm_nt(const float* a, const DeviceBuffer& w, const std::shared_ptr<const DeviceBuffer>& b,
              float* c, std::size_t m, std::size_t n, std::size_t k) {
    check(moe_sgemm_nt(moe_dropin::context(), a, w.as<float>(), b ? b->as<float>() : nullptr, c,
                       static_cast<int64_t>(m), static_cast<int64_t>(n), static_cast<int64_t>(k),
                       nullptr));
}

// c = a w^T + b + resid, the residual added in the GEMM's store
void sgemm_nt_residual(const float* a, const DeviceBuffer& w,
                       const std::shared_ptr<const DeviceBuffer>& b, const float* resid, float* c,
                       std::size_t m, std::size_t n, std::size_t k) {
    check(moe_sgemm_nt_residual(moe_dropin::context(), a, w.as<float>(),
                                b ? b->as<float>() : nullptr, resid, c, static_cast<int64_t>(m),
                                static_cast<int64_t>(n), static_cast<int64_t>(k), nullptr));
}

}  // namespace

// ------------------------------------------------------------------ Linear
Linear::Linear(const ModelLoader& loader, const std::string& weight, const std::string& bias) {
    const Tensor w = loader.load(weight);
    if (w.ndim() != 2) throw std::invalid_argument(weight + ": weight must be 2-D");
    out_ = w.size(0);
    in_ = w.size(1);
    weight_ = upload(w);
    if (!bias.empty() && loader.has(bias)) {
        const Tensor b = loader.load(bias);
        if (b.size() != out_) throw std::invalid_argument(bias + ": bias shape");
        bias_ = upload(b);
    }
}

void Linear::forward(const Tensor& x, Tensor& y) const {
    if (!weight_) throw std::logic_error("Linear used before construction from weights");
    const std::size_t in = x.size(x.ndim() - 1);
    const std::size_t rows = x.size() / in;
    if (in != in_) throw std::invalid_argument("matmul_transposed shape");
    auto lock = moe_dropin::io_lock();
    moe_dropin::Scratch& io = moe_dropin::io_scratch();
    float* dx = io.f32(kIoX, x.size());
    float* dy = io.f32(kIoY, rows * out_);
    moe_dropin::to_device(dx, x.data(), x.size() * sizeof(float));
    check(moe_sgemm_nt(moe_dropin::context(), dx, weight_->as<float>(),
                       bias_ ? bias_->as<float>() : nullptr, dy, static_cast<int64_t>(rows),
                       static_cast<int64_t>(out_), static_cast<int64_t>(in_), nullptr));
    shape_output(y, {rows, out_});
    moe_dropin::to_host(y.data(), dy, rows * out_ * sizeof(float));
}

// ------------------------------------------------------------------ PhiMLP
PhiMLP::PhiMLP(const ModelLoader& loader, const std::string& prefix) {
    const Tensor w1 = loader.load(prefix + ".w1.weight");
    const Tensor w2 = loader.load(prefix + ".w2.weight");
    const Tensor w3 = loader.load(prefix + ".w3.weight");
    if (w1.ndim() != 2) throw std::invalid_argument(prefix + ".w1.weight: weight must be 2-D");
    ff_ = w1.size(0);
    hidden_ = w1.size(1);
    require_2d(w3, ff_, hidden_, prefix + ".w3.weight");
    require_2d(w2, hidden_, ff_, prefix + ".w2.weight");
    w1_ = upload(w1);
    w2_ = upload(w2);
    w3_ = upload(w3);
}

void PhiMLP::forward(const Tensor& x, Tensor& y) const {
    const std::size_t hidden = x.size(x.ndim() - 1);
    const std::size_t rows = x.size() / hidden;
    if (hidden != hidden_) throw std::invalid_argument("matmul_transposed shape");
    // One expert holding every row: the grouped FFN with E = 1, k = 1.
    std::vector<int32_t> perm(rows);
    std::iota(perm.begin(), perm.end(), 0);
    const int32_t offsets[2] = {0, static_cast<int32_t>(rows)};
    auto lock = moe_dropin::io_lock();
    moe_dropin::Scratch& io = moe_dropin::io_scratch();
    float* dx = io.f32(kIoX, x.size());
    float* dh = io.f32(kIoH, rows * ff_);
    float* dout = io.f32(kIoY, rows * hidden_);
    moe_dropin::to_device(dx, x.data(), x.size() * sizeof(float));
    const int32_t* dperm = io.upload(kIoPerm, perm.data(), rows);
    const int32_t* doff = io.upload(kIoOff, offsets, 2);
    check(moe_expert_ffn_grouped(moe_dropin::context(), dx, dperm, doff, w1_->as<float>(),
                                 w3_->as<float>(), w2_->as<float>(), MOE_ACT_SWIGLU,
                                 static_cast<int64_t>(rows), 1, static_cast<int64_t>(hidden_),
                                 static_cast<int64_t>(ff_), 1, dh, dout, nullptr));
    shape_output(y, x.shape());
    moe_dropin::to_host(y.data(), dout, rows * hidden_ * sizeof(float));
}

// ------------------------------------------------------------------ PhiMoE
PhiMoE::PhiMoE(const ModelLoader& loader, std::size_t layer_idx, int contract)
    : contract_(contract) {
    const std::string base = "model.layers." + std::to_string(layer_idx) + ".block_sparse_moe";
    const Tensor gate = loader.load(base + ".gate.weight");
    if (gate.ndim() != 2) throw std::invalid_argument(base + ".gate.weight: weight must be 2-D");
    experts_ = gate.size(0);
    hidden_ = gate.size(1);
    std::vector<Tensor> w1, w2, w3;
    for (std::size_t e = 0; e < experts_; ++e) {
        const std::string p = base + ".experts." + std::to_string(e);
        w1.push_back(loader.load(p + ".w1.weight"));
        if (e == 0) {
            if (w1[0].ndim() != 2) throw std::invalid_argument(p + ".w1.weight: weight must be 2-D");
            ff_ = w1[0].size(0);
        }
        require_2d(w1.back(), ff_, hidden_, p + ".w1.weight");
        w3.push_back(loader.load(p + ".w3.weight"));
        require_2d(w3.back(), ff_, hidden_, p + ".w3.weight");
        w2.push_back(loader.load(p + ".w2.weight"));
        require_2d(w2.back(), hidden_, ff_, p + ".w2.weight");
    }
    gate_ = upload(gate);
    w1_ = upload_stacked(w1);
    w3_ = upload_stacked(w3);
    w2_ = upload_stacked(w2);
}

void PhiMoE::forward(const Tensor& x, Tensor& y) const { forward(x, y, nullptr); }

void PhiMoE::forward(const Tensor& x, Tensor& y, std::vector<int32_t>* topk_idx) const {
    const std::size_t rows = x.size(0), h = x.size(1);
    if (h != hidden_) throw std::invalid_argument("matmul_transposed shape");
    const std::size_t k = apss26::TOP_K < experts_ ? apss26::TOP_K : experts_;
    auto lock = moe_dropin::io_lock();
    moe_dropin::Scratch& io = moe_dropin::io_scratch();
    float* dx = io.f32(kIoX, x.size());
    float* dy = io.f32(kIoY, rows * hidden_);
    int32_t* didx = io.i32(kIoIdx, rows * k);
    moe_dropin::to_device(dx, x.data(), x.size() * sizeof(float));
    forward_device(dx, dy, rows, MOE_NORM_NONE, nullptr, nullptr, 0, didx);
    shape_output(y, {rows, h});
    moe_dropin::to_host(y.data(), dy, rows * h * sizeof(float));
    if (topk_idx != nullptr) {
        topk_idx->resize(rows * k);
        moe_dropin::to_host(topk_idx->data(), didx, rows * k * sizeof(int32_t));
    }
}

void PhiMoE::forward_device(const float* dx, float* dy, std::size_t rows, int norm,
                            const float* norm_w, const float* norm_b, int residual,
                            int32_t* topk_idx) const {
    const std::size_t k = apss26::TOP_K < experts_ ? apss26::TOP_K : experts_;
    moe_layer_desc desc{};
    desc.T = static_cast<int64_t>(rows);
    desc.d = static_cast<int64_t>(hidden_);
    desc.E = static_cast<int64_t>(experts_);
    desc.k = static_cast<int64_t>(k);
    desc.d_ff = static_cast<int64_t>(ff_);
    desc.act = MOE_ACT_SWIGLU;
    desc.router = MOE_ROUTER_PHI_QUANT;
    desc.quantum = apss26::ROUTER_SCORE_QUANTUM;
    desc.tie_eps = apss26::ROUTER_TIE_EPS;
    desc.contract = contract_;
    desc.norm = norm;
    desc.norm_eps = apss26::NORM_EPS;
    desc.residual = residual;
    moe_layer_weights w{};
    w.gate_w = gate_->as<float>();
    w.w1 = w1_->as<float>();
    w.w3 = w3_->as<float>();
    w.w2 = w2_->as<float>();
    w.norm_w = norm_w;
    w.norm_b = norm_b;
    check(moe_layer_forward(moe_dropin::context(), &desc, &w, dx, dy, topk_idx, nullptr, nullptr));
}

// ------------------------------------------------------------ PhiAttention
// src/layer.cu:105-143: projections with bias, RoPE over the sequence's s
// positions, causal attention within SLIDING_WINDOW, o projection.
PhiAttention::PhiAttention(const ModelLoader& loader, std::size_t layer_idx) {
    const std::string base = "model.layers." + std::to_string(layer_idx) + ".self_attn.";
    const std::size_t qw = apss26::NUM_ATTENTION_HEADS * apss26::HEAD_DIM;
    const std::size_t kw = apss26::NUM_KV_HEADS * apss26::HEAD_DIM;
    const Tensor q = loader.load(base + "q_proj.weight");
    if (q.ndim() != 2) throw std::invalid_argument(base + "q_proj.weight: weight must be 2-D");
    hidden_ = q.size(1);
    auto proj = [&](const std::string& name, std::size_t out, std::size_t in,
                    std::shared_ptr<const DeviceBuffer>& w, std::shared_ptr<const DeviceBuffer>& b) {
        const Tensor wt = name == "q_proj" ? q : loader.load(base + name + ".weight");
        require_2d(wt, out, in, base + name + ".weight");
        w = upload(wt);
        if (loader.has(base + name + ".bias")) {
            const Tensor bt = loader.load(base + name + ".bias");
            if (bt.size() != out) throw std::invalid_argument(base + name + ".bias: bias shape");
            b = upload(bt);
        }
    };
    proj("q_proj", qw, hidden_, wq_, bq_);
    proj("k_proj", kw, hidden_, wk_, bk_);
    proj("v_proj", kw, hidden_, wv_, bv_);
    proj("o_proj", hidden_, qw, wo_, bo_);
    rope_ = shared_rope_table();
    rope_positions_ = apss26::MAX_POSITION_EMBEDDINGS;
}

void PhiAttention::forward_device(const float* dx, float* dy, std::size_t s) const {
    const std::size_t sp = padded_rows(s);
    const std::size_t H = apss26::NUM_ATTENTION_HEADS, KVH = apss26::NUM_KV_HEADS,
                      hd = apss26::HEAD_DIM;
    // the caller holds io_lock()
    moe_dropin::Scratch& io = moe_dropin::io_scratch();
    float* q = io.f32(kIoQ, sp * H * hd);
    float* k = io.f32(kIoK, sp * KVH * hd);
    float* v = io.f32(kIoV, sp * KVH * hd);
    float* a = io.f32(kIoA, sp * H * hd);
    sgemm_nt(dx, *wq_, bq_, q, sp, H * hd, hidden_);
    sgemm_nt(dx, *wk_, bk_, k, sp, KVH * hd, hidden_);
    sgemm_nt(dx, *wv_, bv_, v, sp, KVH * hd, hidden_);
    std::shared_ptr<const DeviceBuffer> table = rope_;
    std::size_t positions = rope_positions_;
    if (s > positions) {
        table = rope_table(s);
        positions = s;
    }
    moe_ctx* ctx = moe_dropin::context();
    // Rows past s come from finite padding rows and sit after every real
    // query, so the causal mask hides them: the padded attention is exact
    // for the rows < s.
    check(moe_rope(ctx, q, k, table->as<float>(),
                   static_cast<int64_t>(positions), 1, static_cast<int64_t>(s), 0,
                   static_cast<int64_t>(H), static_cast<int64_t>(KVH), static_cast<int64_t>(hd),
                   nullptr));
    check(moe_attention(ctx, q, k, v, a, 1,
                        static_cast<int64_t>(sp), static_cast<int64_t>(H),
                        static_cast<int64_t>(KVH), static_cast<int64_t>(hd),
                        static_cast<int64_t>(apss26::SLIDING_WINDOW), nullptr));
    sgemm_nt(a, *wo_, bo_, dy, sp, hidden_, H * hd);
}

void PhiAttention::forward(const Tensor& x, Tensor& y) const {
    if (x.ndim() != 2 || x.size(1) != hidden_) throw std::invalid_argument("matmul_transposed shape");
    const std::size_t s = x.size(0), sp = padded_rows(s);
    if (s == 0) {
        y = Tensor({s, hidden_});
        return;
    }
    auto lock = moe_dropin::io_lock();
    moe_dropin::Scratch& io = moe_dropin::io_scratch();
    float* dx = io.f32(kIoX, sp * hidden_);
    float* dy = io.f32(kIoY, sp * hidden_);
    // the padding rows are zero: finite inputs the causal mask hides
    moe_dropin::zero_device(dx + s * hidden_, (sp - s) * hidden_ * sizeof(float));
    moe_dropin::to_device(dx, x.data(), x.size() * sizeof(float));
    forward_device(dx, dy, s);
    shape_output(y, {s, hidden_});
    moe_dropin::to_host(y.data(), dy, s * hidden_ * sizeof(float));
}

void PhiAttention::forward_nodes(const float* dn, float* dy, const float* resid,
                                 const NodeRows& nb, bool tail, moe_dropin::Scratch& sc) const {
    const std::size_t H = apss26::NUM_ATTENTION_HEADS, KVH = apss26::NUM_KV_HEADS,
                      hd = apss26::HEAD_DIM;
    const std::size_t rows = nb.rows, nq = tail ? nb.tail_rows : rows;
    if (rows == 0 || nq == 0) return;
    moe_ctx* ctx = moe_dropin::context();
    float* k = sc.f32(kSlotK, rows * KVH * hd);
    float* v = sc.f32(kSlotV, rows * KVH * hd);
    float* q = sc.f32(kSlotQ, nq * H * hd);
    float* a = sc.f32(kSlotAttn, nq * H * hd);
    if (nb.urows > 0 && !tail) {
        // the projections of the distinct tokens' rows, then each node's row
        // of them (a row gather, moe_embed over the projected table)
        const std::size_t U = nb.urows;
        float* uq = sc.f32(kSlotUQ, U * H * hd);
        float* uk = sc.f32(kSlotUK, U * KVH * hd);
        float* uv = sc.f32(kSlotUV, U * KVH * hd);
        sgemm_nt(dn, *wq_, bq_, uq, U, H * hd, hidden_);
        sgemm_nt(dn, *wk_, bk_, uk, U, KVH * hd, hidden_);
        sgemm_nt(dn, *wv_, bv_, uv, U, KVH * hd, hidden_);
        const auto R = static_cast<int64_t>(rows), Ui = static_cast<int64_t>(U);
        check(moe_embed(ctx, uq, nb.node_u, R, static_cast<int64_t>(H * hd), Ui, q, nullptr));
        check(moe_embed(ctx, uk, nb.node_u, R, static_cast<int64_t>(KVH * hd), Ui, k, nullptr));
        check(moe_embed(ctx, uv, nb.node_u, R, static_cast<int64_t>(KVH * hd), Ui, v, nullptr));
    } else {
        sgemm_nt(dn, *wk_, bk_, k, rows, KVH * hd, hidden_);
        sgemm_nt(dn, *wv_, bv_, v, rows, KVH * hd, hidden_);
        if (tail) {  // q of the last node of every sequence only
            float* dt = sc.f32(kSlotTailIn, nq * hidden_);
            check(moe_embed(ctx, dn, nb.tail_nodes, static_cast<int64_t>(nq),
                            static_cast<int64_t>(hidden_), static_cast<int64_t>(rows), dt,
                            nullptr));
            sgemm_nt(dt, *wq_, bq_, q, nq, H * hd, hidden_);
        } else {
            sgemm_nt(dn, *wq_, bq_, q, rows, H * hd, hidden_);
        }
    }
    const auto P = static_cast<int64_t>(rope_positions_);
    check(moe_rope_rows(ctx, nullptr, k, rope_->as<float>(), P, nb.positions,
                        static_cast<int64_t>(rows), 0, static_cast<int64_t>(KVH),
                        static_cast<int64_t>(hd), nullptr));
    check(moe_rope_rows(ctx, q, nullptr, rope_->as<float>(), P,
                        tail ? nb.tail_positions : nb.positions, static_cast<int64_t>(nq),
                        static_cast<int64_t>(H), 0, static_cast<int64_t>(hd), nullptr));
    check(moe_attention_paths(ctx, q, k, v, a, static_cast<int64_t>(nq), static_cast<int64_t>(rows), nb.key_rows,
                              tail ? nb.tail_key_beg : nb.key_off,
                              tail ? nb.tail_key_end : nb.key_off + 1,
                              static_cast<int64_t>(nb.max_len),
                              static_cast<int64_t>(nb.key_total), static_cast<int64_t>(H),
                              static_cast<int64_t>(KVH), static_cast<int64_t>(hd),
                              static_cast<int64_t>(apss26::SLIDING_WINDOW), nullptr));
    sgemm_nt_residual(a, *wo_, bo_, resid, dy, nq, hidden_, H * hd);
}

// --------------------------------------------------------- PhiDecoderLayer
// src/layer.cu:145-162: h = x + attention(layer_norm(x)), y = h +
// moe(layer_norm(h)); the second norm and both residual adds of the MoE
// block run inside moe_layer_forward (norm = MOE_NORM_LAYER, residual = 1).
PhiDecoderLayer::PhiDecoderLayer(const ModelLoader& loader, std::size_t layer_idx)
    : attention_(loader, layer_idx), moe_(loader, layer_idx) {
    const std::string base = "model.layers." + std::to_string(layer_idx) + ".";
    const std::size_t h = attention_.hidden();
    if (moe_.hidden() != h) throw std::invalid_argument(base + "block_sparse_moe: width differs");
    auto vec = [&](const std::string& name) {
        const Tensor t = loader.load(base + name);
        if (t.size() != h) throw std::invalid_argument(base + name + ": unexpected weight shape");
        return upload(t);
    };
    in_w_ = vec("input_layernorm.weight");
    in_b_ = vec("input_layernorm.bias");
    post_w_ = vec("post_attention_layernorm.weight");
    post_b_ = vec("post_attention_layernorm.bias");
}

void PhiDecoderLayer::forward(const Tensor& x, Tensor& y) const {
    const std::size_t h = attention_.hidden();
    if (x.ndim() != 2 || x.size(1) != h) throw std::invalid_argument("layer norm shape");
    const std::size_t s = x.size(0), sp = PhiAttention::padded_rows(s);
    if (s == 0) {
        y = Tensor({s, h});
        return;
    }
    auto lock = moe_dropin::io_lock();
    moe_dropin::Scratch& io = moe_dropin::io_scratch();
    float* dx = io.f32(kIoX, sp * h);
    float* dn = io.f32(kIoN, sp * h);
    float* da = io.f32(kIoH, sp * h);
    float* dy = io.f32(kIoY, s * h);
    moe_dropin::zero_device(dx + s * h, (sp - s) * h * sizeof(float));
    moe_dropin::to_device(dx, x.data(), x.size() * sizeof(float));
    moe_ctx* ctx = moe_dropin::context();
    check(moe_layer_norm(ctx, dx, in_w_->as<float>(), in_b_->as<float>(), apss26::NORM_EPS,
                         static_cast<int64_t>(sp), static_cast<int64_t>(h), MOE_CONTRACT_FMA, dn,
                         nullptr, nullptr, nullptr));
    attention_.forward_device(dn, da, s);
    check(moe_add(ctx, da, dx, static_cast<int64_t>(s * h), nullptr));
    moe_.forward_device(da, dy, s, MOE_NORM_LAYER, post_w_->as<float>(), post_b_->as<float>(), 1,
                        nullptr);
    shape_output(y, {s, h});
    moe_dropin::to_host(y.data(), dy, s * h * sizeof(float));
}

// The layer over trie rows; with `tail` (the reference's pruned last layer,
// src/model.cu:1889-1960) the norm, k and v still cover every node, and the
// rest runs on the last node of every sequence.
void PhiDecoderLayer::forward_nodes(const float* dx, float* dy, const NodeRows& nb, bool tail,
                                    moe_dropin::Scratch& sc) const {
    const std::size_t h = attention_.hidden(), rows = nb.rows;
    const std::size_t n = tail ? nb.tail_rows : rows;
    if (rows == 0 || n == 0) return;
    moe_ctx* ctx = moe_dropin::context();
    float* da = sc.f32(kSlotAttnOut, n * h);
    // the input norm: over the distinct tokens' rows when the batch gives
    // them (first layer), else over every node
    const bool distinct = nb.urows > 0 && !tail;
    const std::size_t nrows = distinct ? nb.urows : rows;
    float* dn = sc.f32(distinct ? kSlotUNorm : kSlotNorm, nrows * h);
    check(moe_layer_norm(ctx, distinct ? nb.ux : dx, in_w_->as<float>(), in_b_->as<float>(),
                         apss26::NORM_EPS, static_cast<int64_t>(nrows), static_cast<int64_t>(h),
                         MOE_CONTRACT_FMA, dn, nullptr, nullptr, nullptr));
    // h = x + attention(norm(x)): the residual rows (the tail rows' gathered
    // from x) are added in the o-projection's store
    const float* resid = dx;
    if (tail) {
        float* dr = sc.f32(kSlotTailResid, n * h);
        check(moe_embed(ctx, dx, nb.tail_nodes, static_cast<int64_t>(n), static_cast<int64_t>(h),
                        static_cast<int64_t>(rows), dr, nullptr));
        resid = dr;
    }
    attention_.forward_nodes(dn, da, resid, nb, tail, sc);
    moe_.forward_device(da, dy, n, MOE_NORM_LAYER, post_w_->as<float>(), post_b_->as<float>(), 1,
                        nullptr);
}
