#include "device.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
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

}  // namespace

// The drop-in's one context, created on first use and never destroyed: a
// destructor of a static would run during process exit, after the HIP
// runtime's own statics may be gone, so hipFree / hipEventDestroy from there
// could crash or hang.  Its workspace is released by the process's end.
moe_ctx* context() {
    static moe_ctx* ctx = nullptr;
    static std::once_flag once;
    std::call_once(once, [] {
        const char* env = std::getenv("MOE_DEVICE");
        const int device = env != nullptr ? std::atoi(env) : 0;
        moe_ctx* c = nullptr;
        check(moe_ctx_create(device, &c));
        ctx = c;
    });
    if (ctx == nullptr) throw std::runtime_error("moe context unavailable");
    return ctx;
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

namespace {

struct Staging {
    std::mutex mu;
    char* host = nullptr;  // pinned, 2 * half bytes
    std::size_t half = 0;
    hipEvent_t done[2] = {nullptr, nullptr};  // the last DMA out of / into each half
    bool pending[2] = {false, false};
    Scratch io;
    // Grow the pinned halves to min(bytes, 32 MiB) each.
    void reserve(std::size_t bytes) {
        constexpr std::size_t kMaxHalf = std::size_t(32) << 20;
        const std::size_t want = std::min(std::max<std::size_t>(bytes, 1 << 16), kMaxHalf);
        if (want <= half) return;
        wait(0);
        wait(1);
        if (host != nullptr) hip(hipHostFree(host), "hipHostFree");
        host = nullptr;
        half = 0;
        hip(hipHostMalloc(reinterpret_cast<void**>(&host), 2 * want, hipHostMallocDefault),
            "hipHostMalloc staging");
        half = want;
        for (hipEvent_t& e : done)
            if (e == nullptr) hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    }
    void wait(int h) {
        if (pending[h]) hip(hipEventSynchronize(done[h]), "hipEventSynchronize");
        pending[h] = false;
    }
};

// Built on first use and never destroyed: a static's destructor would run
// at process exit, after the HIP runtime may have torn down its own state,
// so hipHostFree / hipEventDestroy / hipFree from there could crash or hang.
// The pinned halves, events and device slots are released by the process's
// end instead.
Staging& staging() {
    static Staging& s = *new Staging;
    return s;
}

}  // namespace

std::unique_lock<std::mutex> io_lock() { return std::unique_lock<std::mutex>(staging().mu); }

Scratch& io_scratch() { return staging().io; }

void to_device(void* dst, const void* src, std::size_t bytes) {
    if (bytes == 0) return;
    Staging& st = staging();
    st.reserve(bytes);
    for (std::size_t off = 0, c = 0; off < bytes; off += st.half, ++c) {
        const int h = static_cast<int>(c & 1);
        const std::size_t n = std::min(st.half, bytes - off);
        st.wait(h);  // the DMA that last read this half is done
        char* stage = st.host + h * st.half;
        std::memcpy(stage, static_cast<const char*>(src) + off, n);
        hip(hipMemcpyAsync(static_cast<char*>(dst) + off, stage, n, hipMemcpyHostToDevice, nullptr),
            "hipMemcpyAsync H2D");
        hip(hipEventRecord(st.done[h], nullptr), "hipEventRecord");
        st.pending[h] = true;
    }
}

void zero_device(void* dst, std::size_t bytes) {
    if (bytes != 0) hip(hipMemsetAsync(dst, 0, bytes, nullptr), "hipMemsetAsync");
}

void to_host(void* dst, const void* src, std::size_t bytes) {
    if (bytes == 0) return;
    Staging& st = staging();
    st.reserve(bytes);
    const std::size_t chunks = (bytes + st.half - 1) / st.half;
    auto issue = [&](std::size_t c) {
        const int h = static_cast<int>(c & 1);
        const std::size_t off = c * st.half, n = std::min(st.half, bytes - off);
        st.wait(h);
        hip(hipMemcpyAsync(st.host + h * st.half, static_cast<const char*>(src) + off, n,
                           hipMemcpyDeviceToHost, nullptr),
            "hipMemcpyAsync D2H");
        hip(hipEventRecord(st.done[h], nullptr), "hipEventRecord");
        st.pending[h] = true;
    };
    issue(0);
    for (std::size_t c = 0; c < chunks; ++c) {
        if (c + 1 < chunks) issue(c + 1);  // the next chunk moves while this one is copied out
        const int h = static_cast<int>(c & 1);
        st.wait(h);
        const std::size_t off = c * st.half, n = std::min(st.half, bytes - off);
        std::memcpy(static_cast<char*>(dst) + off, st.host + h * st.half, n);
    }
}

}  // namespace moe_dropin
