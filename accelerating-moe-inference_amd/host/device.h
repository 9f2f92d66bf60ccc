// Internal helpers of the drop-in host layer: the process-wide moe_ctx,
// status-to-exception mapping, and an RAII device buffer.
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <vector>

#include "../../include/moe_amd.h"

namespace moe_dropin {

// The context every drop-in call uses: device $MOE_DEVICE (default 0),
// created on first use, destroyed at exit.
moe_ctx* context();

// MOE_ERR_INVALID -> std::invalid_argument, any other error ->
// std::runtime_error, carrying moe_last_error().
void check(int status);

// Waits for the work the drop-in enqueued (it uses the default stream).
void synchronize();

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;

    void* get() const { return p_; }
    std::size_t bytes() const { return n_; }
    template <class T>
    T* as() const { return static_cast<T*>(p_); }
    void upload(const void* src, std::size_t bytes, std::size_t offset = 0);
    void zero();  // every byte 0 (synchronous)
    void download(void* dst, std::size_t bytes) const;

private:
    void* p_ = nullptr;
    std::size_t n_ = 0;
};

// Grow-only device scratch, one buffer per slot (the reference's Scratch,
// src/model.cu:1294-1324): a slot reallocates only when a call asks for more
// than it holds, so repeated calls of one shape allocate nothing.  Not safe
// for concurrent use.
class Scratch {
public:
    float* f32(std::size_t slot, std::size_t count) {
        return static_cast<float*>(get(slot, count * sizeof(float)));
    }
    int32_t* i32(std::size_t slot, std::size_t count) {
        return static_cast<int32_t*>(get(slot, count * sizeof(int32_t)));
    }
    // Copies count host values into the slot and returns its device copy.
    const int32_t* upload(std::size_t slot, const int32_t* src, std::size_t count);
    // Copies the slot's first `bytes` bytes to the host (synchronous).
    void download(std::size_t slot, void* dst, std::size_t bytes) const;

private:
    std::vector<DeviceBuffer> bufs_;
    void* get(std::size_t slot, std::size_t bytes);
};

// The drop-in's copies of pageable host tensors.  They go through a
// grow-only pinned staging buffer (at most 64 MiB, two halves): the CPU
// copies one chunk into a half while the DMA engine moves the other, on the
// stream the drop-in's kernels use.  to_device returns once every chunk is
// staged (src may be reused; the transfer may still be in flight);
// to_host returns with dst filled.  Callers hold io_lock().
void to_device(void* dst, const void* src, std::size_t bytes);
void to_host(void* dst, const void* src, std::size_t bytes);
// Sets bytes of device memory at dst to 0, on the drop-in's stream.
void zero_device(void* dst, std::size_t bytes);

// The per-call device buffers of the drop-in's inputs and outputs: grow-only
// slots, so repeated calls of one shape allocate nothing.  Callers hold
// io_lock() while they use them.
Scratch& io_scratch();
std::unique_lock<std::mutex> io_lock();

}  // namespace moe_dropin
