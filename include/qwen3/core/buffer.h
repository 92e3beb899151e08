#pragma once

// Owning, move-only byte storage on the host (64-byte aligned) or on a GPU
// (hipMalloc; device blocks of at most 4 MiB are kept for reuse when their
// Buffer is destroyed, in the order of the default stream, up to 64 MiB per
// device).  Unlike hipFree, keeping a block does not wait for the device:
// work on a stream other than the default one that uses a small tensor must
// have finished before the tensor is destroyed.  QWEN3_DEVICE_BLOCK_CACHE=0
// in the environment turns the cache off (every block freed with hipFree, as
// the reference's Buffer does).  Contract pinned by the reference's tests/unit/buffer_cpu_test.cpp
// and buffer_cuda_test.cpp: zero bytes give a null pointer, a moved-from
// buffer is empty, copies check sizes (std::invalid_argument) and ranges
// (std::out_of_range), GPU allocation failures throw std::runtime_error and
// leave the current device unchanged.

#include "qwen3/core/device.h"

#include <cstddef>
#include <cstdint>

namespace qwen3
{
    class Buffer
    {
    public:
        static constexpr std::size_t kCpuAlignment = 64;

        Buffer() noexcept;
        Buffer(std::size_t size_bytes, Device device);
        ~Buffer();

        Buffer(const Buffer &) = delete;
        Buffer &operator=(const Buffer &) = delete;
        Buffer(Buffer &&other) noexcept;
        Buffer &operator=(Buffer &&other) noexcept;

        [[nodiscard]] void *data() noexcept { return data_; }
        [[nodiscard]] const void *data() const noexcept { return data_; }
        [[nodiscard]] std::size_t size_bytes() const noexcept { return size_bytes_; }
        [[nodiscard]] bool empty() const noexcept { return size_bytes_ == 0; }
        [[nodiscard]] const Device &device() const noexcept { return device_; }

    private:
        void release() noexcept;

        void *data_;
        std::size_t size_bytes_;
        Device device_;
    };

    // Device allocations (hipMalloc calls) made by Buffers in this process;
    // a block taken from the reuse cache does not count.
    [[nodiscard]] std::uint64_t device_allocation_count() noexcept;

    // Frees the device blocks kept for reuse (every GPU).
    void release_cached_device_blocks();

    // Whole-buffer copy between any two devices (synchronous).
    void copy_buffer(Buffer &destination, const Buffer &source);

    // Copy of `bytes` bytes from source[source_offset] to destination[destination_offset].
    void copy_buffer(Buffer &destination, std::size_t destination_offset, const Buffer &source,
                     std::size_t source_offset, std::size_t bytes);
} // namespace qwen3
