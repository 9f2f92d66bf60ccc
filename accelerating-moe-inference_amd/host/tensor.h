// Host tensor and tensor_ops of the drop-in API.
//
// Interface of the reference's include/tensor.h:7-73 (same class, members
// and operator names, same exception types), re-implemented here: Tensor is
// an owning, zero-initialised, row-major fp32 host buffer; the tensor_ops of
// the MoE path run on the GPU through the C ABI (include/moe_amd.h): inputs
// are copied to the device, the HIP kernel runs, the result is copied back.
#pragma once

#include <cstddef>
#include <initializer_list>
#include <string>
#include <vector>

class Tensor {
public:
    // Host: pageable memory.  Pinned: page-locked (hipHostMalloc), for
    // buffers that cross PCIe often; copies of a Tensor are always Host.
    enum class Alloc { Host, Pinned };

    Tensor() = default;
    explicit Tensor(std::vector<std::size_t> shape, Alloc alloc = Alloc::Host);
    ~Tensor();
    Tensor(const Tensor& other);
    Tensor& operator=(const Tensor& other);
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;

    std::size_t ndim() const { return shape_.size(); }
    std::size_t size() const { return size_; }
    std::size_t capacity() const { return capacity_; }
    Alloc alloc() const { return alloc_; }
    std::size_t size(std::size_t dim) const;
    const std::vector<std::size_t>& shape() const { return shape_; }

    float* data() { return data_; }
    const float* data() const { return data_; }
    float& operator[](std::size_t i) { return data_[i]; }
    const float& operator[](std::size_t i) const { return data_[i]; }

    // Bounds-checked element access (std::out_of_range / std::invalid_argument).
    float& at(std::size_t i);
    float& at(std::size_t i, std::size_t j);
    float& at(std::size_t i, std::size_t j, std::size_t k);
    float& at(std::size_t i, std::size_t j, std::size_t k, std::size_t l);
    const float& at(std::size_t i) const;
    const float& at(std::size_t i, std::size_t j) const;
    const float& at(std::size_t i, std::size_t j, std::size_t k) const;
    const float& at(std::size_t i, std::size_t j, std::size_t k, std::size_t l) const;

    void reshape(std::vector<std::size_t> shape);
    // Retarget the buffer at a shape of at most capacity() elements.
    void reshape_within_capacity(std::vector<std::size_t> shape);
    void fill(float value);
    void zero() { fill(0.0f); }

private:
    std::vector<std::size_t> shape_;
    float* data_ = nullptr;
    std::size_t size_ = 0, capacity_ = 0;
    Alloc alloc_ = Alloc::Host;
    void release();
    std::size_t index(std::initializer_list<std::size_t> idx) const;
};

namespace tensor_ops {
// GPU (fp32 MFMA): c[M,N] = a[M,K] b[K,N] and a[M,K] b[N,K]^T.
void matmul(const Tensor& a, const Tensor& b, Tensor& c);
void matmul_transposed(const Tensor& a, const Tensor& b, Tensor& c);
// GPU elementwise, bit-identical to the reference's CPU loops.
void mul(const Tensor& a, const Tensor& b, Tensor& c);
void silu(const Tensor& x, Tensor& y);
// GPU layer norm over the last axis (the MoE block's post-attention norm),
// bit-identical to the reference's CPU loop under FMA contraction.
void layer_norm(const Tensor& x, const Tensor& weight, const Tensor& bias,
                float eps, Tensor& y);
// GPU residual and bias adds, bit-identical to the reference's loops.
void add_inplace(Tensor& a, const Tensor& b);
void add_bias_inplace(Tensor& a, const Tensor& bias);
// Declared by the reference's header but never defined there: throws
// std::logic_error.
void softmax_last_dim(const Tensor& x, Tensor& y);
// GPU RoPE on the first seq_len rows of q [rows, q_heads*head_dim] and k
// [rows, kv_heads*head_dim], cos/sin from the same float libm calls as the
// reference: bit-identical to its loop (each product rounded on its own).
// Rows must be exactly heads*head_dim wide and head_dim even
// (std::invalid_argument otherwise); seq_len past the rows throws
// std::out_of_range, as the reference's at() does.
void apply_rope(Tensor& q, Tensor& k, std::size_t seq_len,
                std::size_t q_heads, std::size_t kv_heads, std::size_t head_dim,
                float theta);
}  // namespace tensor_ops
