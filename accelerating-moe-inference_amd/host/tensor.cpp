// Tensor (host storage) and the GPU-backed tensor_ops of the drop-in API.
#include "tensor.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "device.h"

namespace {

std::size_t count_of(const std::vector<std::size_t>& shape) {
    std::size_t n = 1;
    for (std::size_t d : shape) n *= d;
    return n;
}

}  // namespace

Tensor::Tensor(std::vector<std::size_t> shape, Alloc alloc)
    : shape_(std::move(shape)), alloc_(alloc) {
    const std::size_t n = count_of(shape_);
    if (alloc_ == Alloc::Pinned) {
        void* p = nullptr;
        const hipError_t e = hipHostMalloc(&p, std::max<std::size_t>(n, 1) * sizeof(float),
                                           hipHostMallocDefault);
        if (e != hipSuccess)
            throw std::runtime_error(std::string("hipHostMalloc tensor: ") + hipGetErrorString(e));
        data_ = static_cast<float*>(p);
    } else {
        data_ = new float[std::max<std::size_t>(n, 1)];
    }
    size_ = capacity_ = n;
    std::fill(data_, data_ + n, 0.0f);
}

void Tensor::release() {
    if (data_ == nullptr) return;
    if (alloc_ == Alloc::Pinned) {
        const hipError_t e = hipHostFree(data_);
        if (e != hipSuccess) std::fprintf(stderr, "hipHostFree tensor: %s\n", hipGetErrorString(e));
    } else {
        delete[] data_;
    }
    data_ = nullptr;
    size_ = capacity_ = 0;
}

Tensor::~Tensor() { release(); }

Tensor::Tensor(const Tensor& other) : shape_(other.shape_) {
    if (other.size_ != 0) {
        data_ = new float[other.size_];
        std::copy(other.data_, other.data_ + other.size_, data_);
        size_ = capacity_ = other.size_;
    }
}

Tensor& Tensor::operator=(const Tensor& other) {
    if (this != &other) {
        Tensor copy(other);
        *this = std::move(copy);
    }
    return *this;
}

Tensor::Tensor(Tensor&& other) noexcept
    : shape_(std::move(other.shape_)), data_(other.data_), size_(other.size_),
      capacity_(other.capacity_), alloc_(other.alloc_) {
    other.shape_.clear();
    other.data_ = nullptr;
    other.size_ = other.capacity_ = 0;
}

Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this != &other) {
        release();
        shape_ = std::move(other.shape_);
        data_ = other.data_;
        size_ = other.size_;
        capacity_ = other.capacity_;
        alloc_ = other.alloc_;
        other.shape_.clear();
        other.data_ = nullptr;
        other.size_ = other.capacity_ = 0;
    }
    return *this;
}

std::size_t Tensor::size(std::size_t dim) const {
    if (dim >= shape_.size()) throw std::out_of_range("Tensor dimension");
    return shape_[dim];
}

std::size_t Tensor::index(std::initializer_list<std::size_t> idx) const {
    if (idx.size() != shape_.size()) throw std::invalid_argument("Tensor rank mismatch");
    std::size_t flat = 0;
    std::size_t d = 0;
    for (std::size_t i : idx) {
        if (i >= shape_[d]) throw std::out_of_range("Tensor index");
        flat = flat * shape_[d] + i;
        ++d;
    }
    return flat;
}

float& Tensor::at(std::size_t i) { return data_[index({i})]; }
float& Tensor::at(std::size_t i, std::size_t j) { return data_[index({i, j})]; }
float& Tensor::at(std::size_t i, std::size_t j, std::size_t k) { return data_[index({i, j, k})]; }
float& Tensor::at(std::size_t i, std::size_t j, std::size_t k, std::size_t l) {
    return data_[index({i, j, k, l})];
}
const float& Tensor::at(std::size_t i) const { return data_[index({i})]; }
const float& Tensor::at(std::size_t i, std::size_t j) const { return data_[index({i, j})]; }
const float& Tensor::at(std::size_t i, std::size_t j, std::size_t k) const {
    return data_[index({i, j, k})];
}
const float& Tensor::at(std::size_t i, std::size_t j, std::size_t k, std::size_t l) const {
    return data_[index({i, j, k, l})];
}

void Tensor::reshape(std::vector<std::size_t> shape) {
    if (count_of(shape) != size_) throw std::invalid_argument("reshape changes tensor size");
    shape_ = std::move(shape);
}

void Tensor::reshape_within_capacity(std::vector<std::size_t> shape) {
    const std::size_t n = count_of(shape);
    if (n > capacity_) throw std::invalid_argument("reshape exceeds tensor capacity");
    shape_ = std::move(shape);
    size_ = n;
}

void Tensor::fill(float value) { std::fill(data_, data_ + size_, value); }

namespace tensor_ops {
namespace {

using moe_dropin::check;

// Per-call device copies live in the drop-in's grow-only io slots (no
// allocation once a shape has been seen); the copies go through its pinned
// staging.  Every op holds io_lock() while it uses them.
enum Slot : std::size_t { kA, kB, kC, kD };

float* stage_in(std::size_t slot, const Tensor& t) {
    float* d = moe_dropin::io_scratch().f32(slot, t.size());
    moe_dropin::to_device(d, t.data(), t.size() * sizeof(float));
    return d;
}

void stage_out(Tensor& t, const float* d) {
    moe_dropin::to_host(t.data(), d, t.size() * sizeof(float));
}

void gemm(bool nn, const Tensor& a, const Tensor& b, Tensor& c, const char* what) {
    const std::size_t m = a.size(0), k = a.size(1);
    const std::size_t n = nn ? b.size(1) : b.size(0);
    const std::size_t bk = nn ? b.size(0) : b.size(1);
    if (a.ndim() != 2 || b.ndim() != 2 || c.ndim() != 2 || bk != k || c.size(0) != m ||
        c.size(1) != n)
        throw std::invalid_argument(what);
    auto lock = moe_dropin::io_lock();
    const float* da = stage_in(kA, a);
    const float* db = stage_in(kB, b);
    float* dc = moe_dropin::io_scratch().f32(kC, m * n);
    moe_ctx* ctx = moe_dropin::context();
    const auto M = static_cast<int64_t>(m), N = static_cast<int64_t>(n), K = static_cast<int64_t>(k);
    check(nn ? moe_sgemm_nn(ctx, da, db, nullptr, dc, M, N, K, nullptr)
             : moe_sgemm_nt(ctx, da, db, nullptr, dc, M, N, K, nullptr));
    stage_out(c, dc);
}

}  // namespace

void matmul(const Tensor& a, const Tensor& b, Tensor& c) { gemm(true, a, b, c, "matmul shape"); }

void matmul_transposed(const Tensor& a, const Tensor& b, Tensor& c) {
    gemm(false, a, b, c, "matmul_transposed shape");
}

void mul(const Tensor& a, const Tensor& b, Tensor& c) {
    if (a.size() != b.size() || c.size() != a.size()) throw std::invalid_argument("mul shape");
    auto lock = moe_dropin::io_lock();
    const float* da = stage_in(kA, a);
    const float* db = stage_in(kB, b);
    float* dc = moe_dropin::io_scratch().f32(kC, c.size());
    check(moe_mul(moe_dropin::context(), da, db, dc, static_cast<int64_t>(a.size()), nullptr));
    stage_out(c, dc);
}

void silu(const Tensor& x, Tensor& y) {
    if (x.size() != y.size()) throw std::invalid_argument("silu shape");
    auto lock = moe_dropin::io_lock();
    float* dx = stage_in(kA, x);
    check(moe_silu(moe_dropin::context(), dx, dx, static_cast<int64_t>(x.size()), nullptr));
    stage_out(y, dx);
}

// a[i] += b[i] (src/tensor.cu:150-154).
void add_inplace(Tensor& a, const Tensor& b) {
    if (a.size() != b.size()) throw std::invalid_argument("add shape");
    if (a.size() == 0) return;
    auto lock = moe_dropin::io_lock();
    float* da = stage_in(kA, a);
    const float* db = stage_in(kB, b);
    check(moe_add(moe_dropin::context(), da, db, static_cast<int64_t>(a.size()), nullptr));
    stage_out(a, da);
}

// a[i] += bias[i % h] with h = the last dimension (src/tensor.cu:156-161).
void add_bias_inplace(Tensor& a, const Tensor& bias) {
    if (bias.ndim() != 1 || a.ndim() == 0 || a.size(a.ndim() - 1) != bias.size(0))
        throw std::invalid_argument("bias shape");
    const std::size_t h = bias.size(0);
    if (a.size() == 0) return;
    auto lock = moe_dropin::io_lock();
    float* da = stage_in(kA, a);
    const float* db = stage_in(kB, bias);
    check(moe_add_bias(moe_dropin::context(), da, db, static_cast<int64_t>(a.size() / h),
                       static_cast<int64_t>(h), nullptr));
    stage_out(a, da);
}

// include/tensor.h:67 of the reference declares it; no source defines it.
void softmax_last_dim(const Tensor&, Tensor&) {
    throw std::logic_error(
        "tensor_ops::softmax_last_dim is declared by the reference but never defined");
}
// The post-attention norm in front of the MoE block (src/tensor.cu:175-189):
// bit-identical to the CPU loop built with FMA contraction, the drop-in's
// default (PhiMoE's `contract`).
void layer_norm(const Tensor& x, const Tensor& weight, const Tensor& bias, float eps, Tensor& y) {
    const std::size_t h = x.ndim() > 0 ? x.size(x.ndim() - 1) : 0;
    if (h == 0 || weight.size() != h || bias.size() != h || y.size() != x.size())
        throw std::invalid_argument("layer norm shape");
    const std::size_t rows = x.size() / h;
    auto lock = moe_dropin::io_lock();
    float* dx = stage_in(kA, x);
    const float* dw = stage_in(kB, weight);
    const float* db = stage_in(kC, bias);
    check(moe_layer_norm(moe_dropin::context(), dx, dw, db, eps, static_cast<int64_t>(rows),
                         static_cast<int64_t>(h), MOE_CONTRACT_FMA, dx, nullptr, nullptr,
                         nullptr));
    stage_out(y, dx);
}
// src/tensor.cu:191-210 on the GPU: the cos/sin table comes from the same
// float libm calls (moe_rope_table, on the host), the rotation rounds each
// product on its own, as the reference's loop does.
void apply_rope(Tensor& q, Tensor& k, std::size_t seq_len, std::size_t q_heads,
                std::size_t kv_heads, std::size_t head_dim, float theta) {
    if (q.ndim() != 2 || k.ndim() != 2) throw std::invalid_argument("apply_rope rank");
    if (head_dim % 2 != 0 || q.size(1) != q_heads * head_dim ||
        k.size(1) != kv_heads * head_dim)
        throw std::invalid_argument("apply_rope shape");
    if (seq_len == 0 || head_dim == 0) return;
    if ((q_heads > 0 && seq_len > q.size(0)) || (kv_heads > 0 && seq_len > k.size(0)))
        throw std::out_of_range("Tensor index");
    std::vector<float> table(seq_len * head_dim);
    check(moe_rope_table(theta, static_cast<int64_t>(head_dim), static_cast<int64_t>(seq_len),
                         table.data()));
    auto lock = moe_dropin::io_lock();
    float* dt = moe_dropin::io_scratch().f32(kC, table.size());
    moe_dropin::to_device(dt, table.data(), table.size() * sizeof(float));
    float* dq = stage_in(kA, q);
    float* dk = stage_in(kB, k);
    check(moe_rope(moe_dropin::context(), dq, dk, dt, static_cast<int64_t>(seq_len), 1,
                   static_cast<int64_t>(seq_len), 0, static_cast<int64_t>(q_heads),
                   static_cast<int64_t>(kv_heads), static_cast<int64_t>(head_dim), nullptr));
    stage_out(q, dq);
    stage_out(k, dk);
}

}  // namespace tensor_ops
