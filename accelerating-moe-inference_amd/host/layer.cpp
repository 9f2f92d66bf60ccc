#include "layer.h"

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
    y = Tensor({rows, out_});
    DeviceBuffer dx(x.size() * sizeof(float)), dy(rows * out_ * sizeof(float));
    dx.upload(x.data(), x.size() * sizeof(float));
    check(moe_sgemm_nt(moe_dropin::context(), dx.as<float>(), weight_->as<float>(),
                       bias_ ? bias_->as<float>() : nullptr, dy.as<float>(),
                       static_cast<int64_t>(rows), static_cast<int64_t>(out_),
                       static_cast<int64_t>(in_), nullptr));
    dy.download(y.data(), rows * out_ * sizeof(float));
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
    DeviceBuffer dx(x.size() * sizeof(float)), dperm(rows * sizeof(int32_t)),
        doff(sizeof(offsets)), dh(rows * ff_ * sizeof(float)), dout(rows * hidden_ * sizeof(float));
    dx.upload(x.data(), x.size() * sizeof(float));
    dperm.upload(perm.data(), rows * sizeof(int32_t));
    doff.upload(offsets, sizeof(offsets));
    check(moe_expert_ffn_grouped(moe_dropin::context(), dx.as<float>(), dperm.as<int32_t>(),
                                 doff.as<int32_t>(), w1_->as<float>(), w3_->as<float>(),
                                 w2_->as<float>(), MOE_ACT_SWIGLU, static_cast<int64_t>(rows), 1,
                                 static_cast<int64_t>(hidden_), static_cast<int64_t>(ff_), 1,
                                 dh.as<float>(), dout.as<float>(), nullptr));
    Tensor out({rows, hidden_});
    dout.download(out.data(), rows * hidden_ * sizeof(float));
    out.reshape(x.shape());
    y = std::move(out);
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
    moe_layer_weights w{};
    w.gate_w = gate_->as<float>();
    w.w1 = w1_->as<float>();
    w.w3 = w3_->as<float>();
    w.w2 = w2_->as<float>();
    DeviceBuffer dx(x.size() * sizeof(float)), dy(rows * hidden_ * sizeof(float)),
        didx(rows * k * sizeof(int32_t));
    dx.upload(x.data(), x.size() * sizeof(float));
    check(moe_layer_forward(moe_dropin::context(), &desc, &w, dx.as<float>(), dy.as<float>(),
                            didx.as<int32_t>(), nullptr, nullptr));
    y = Tensor({rows, h});
    dy.download(y.data(), rows * h * sizeof(float));
    if (topk_idx != nullptr) {
        topk_idx->resize(rows * k);
        didx.download(topk_idx->data(), rows * k * sizeof(int32_t));
    }
}
