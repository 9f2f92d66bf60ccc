#include "device.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>

namespace moe_dropin {
namespace {

void hip(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

struct CtxHolder {
    moe_ctx* ctx = nullptr;
    ~CtxHolder() {
        if (ctx != nullptr) moe_ctx_destroy(ctx);
    }
};

}  // namespace

moe_ctx* context() {
    static CtxHolder holder;
    static std::once_flag once;
    std::call_once(once, [] {
        const char* env = std::getenv("MOE_DEVICE");
        const int device = env != nullptr ? std::atoi(env) : 0;
        moe_ctx* c = nullptr;
        check(moe_ctx_create(device, &c));
        holder.ctx = c;
    });
    if (holder.ctx == nullptr) throw std::runtime_error("moe context unavailable");
    return holder.ctx;
}

void check(int status) {
    if (status == MOE_OK) return;
    const std::string msg = moe_last_error();
    if (status == MOE_ERR_INVALID) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void synchronize() { hip(hipStreamSynchronize(nullptr), "hipStreamSynchronize"); }

DeviceBuffer::DeviceBuffer(std::size_t bytes) : n_(bytes) {
    if (bytes != 0) hip(hipMalloc(&p_, bytes), "hipMalloc");
}

DeviceBuffer::~DeviceBuffer() {
    if (p_ != nullptr) {
        const hipError_t e = hipFree(p_);
        if (e != hipSuccess) std::fprintf(stderr, "hipFree: %s\n", hipGetErrorString(e));
    }
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) {
    o.p_ = nullptr;
    o.n_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
        DeviceBuffer tmp(std::move(*this));
        p_ = o.p_;
        n_ = o.n_;
        o.p_ = nullptr;
        o.n_ = 0;
    }
    return *this;
}

void DeviceBuffer::upload(const void* src, std::size_t bytes, std::size_t offset) {
    if (bytes == 0) return;
    if (offset + bytes > n_) throw std::invalid_argument("device upload out of range");
    hip(hipMemcpy(static_cast<char*>(p_) + offset, src, bytes, hipMemcpyHostToDevice),
        "hipMemcpy H2D");
}

void DeviceBuffer::zero() {
    if (n_ != 0) hip(hipMemset(p_, 0, n_), "hipMemset");
}

void DeviceBuffer::download(void* dst, std::size_t bytes) const {
    if (bytes == 0) return;
    if (bytes > n_) throw std::invalid_argument("device download out of range");
    hip(hipMemcpy(dst, p_, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void* Scratch::get(std::size_t slot, std::size_t bytes) {
    if (slot >= bufs_.size()) bufs_.resize(slot + 1);
    DeviceBuffer& b = bufs_[slot];
    if (b.bytes() < bytes || b.get() == nullptr) {
        const std::size_t grow = std::max(bytes, b.bytes() + b.bytes() / 2);
        b = DeviceBuffer(std::max<std::size_t>(grow, 16));  // frees the old one (synchronising)
    }
    return b.get();
}

void Scratch::download(std::size_t slot, void* dst, std::size_t bytes) const {
    if (slot >= bufs_.size()) throw std::invalid_argument("scratch slot never filled");
    bufs_[slot].download(dst, bytes);
}

const int32_t* Scratch::upload(std::size_t slot, const int32_t* src, std::size_t count) {
    int32_t* p = i32(slot, count);
    bufs_[slot].upload(src, count * sizeof(int32_t));
    return p;
}

}  // namespace moe_dropin
