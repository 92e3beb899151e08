#include "qwen3/core/buffer.h"

#include "qwen3/hip/hip_check.h"

#include <algorithm>
#include <cstdlib>
#include <new>
#include <stdexcept>
#include <utility>

namespace qwen3
{
    namespace
    {
        void *allocate_host(std::size_t bytes)
        {
            const std::size_t rounded = (bytes + Buffer::kCpuAlignment - 1) / Buffer::kCpuAlignment * Buffer::kCpuAlignment;
            void *p = std::aligned_alloc(Buffer::kCpuAlignment, rounded);
            if (p == nullptr)
                throw std::bad_alloc();
            return p;
        }

        void *allocate_device(std::size_t bytes, int index)
        {
            hip::DeviceGuard guard(index);
            void *p = nullptr;
            QWEN3_HIP_CHECK(hipMalloc(&p, bytes));
            guard.restore();
            return p;
        }

        void check_same_or_throw(std::size_t a, std::size_t b)
        {
            if (a != b)
                throw std::invalid_argument("Buffer copy requires buffers of the same size");
        }
    } // namespace

    Buffer::Buffer() noexcept : data_(nullptr), size_bytes_(0), device_(Device::cpu()) {}

    Buffer::Buffer(std::size_t size_bytes, Device device) : data_(nullptr), size_bytes_(0), device_(device)
    {
        if (size_bytes == 0)
            return;
        data_ = device.is_cpu() ? allocate_host(size_bytes) : allocate_device(size_bytes, device.index());
        size_bytes_ = size_bytes;
    }

    Buffer::~Buffer() { release(); }

    Buffer::Buffer(Buffer &&other) noexcept
        : data_(std::exchange(other.data_, nullptr)), size_bytes_(std::exchange(other.size_bytes_, 0)),
          device_(other.device_)
    {
    }

    Buffer &Buffer::operator=(Buffer &&other) noexcept
    {
        if (this != &other)
        {
            release();
            data_ = std::exchange(other.data_, nullptr);
            size_bytes_ = std::exchange(other.size_bytes_, 0);
            device_ = other.device_;
        }
        return *this;
    }

    void Buffer::release() noexcept
    {
        if (data_ == nullptr)
            return;
        if (device_.is_cpu())
            std::free(data_);
        else
            static_cast<void>(hipFree(data_));
        data_ = nullptr;
        size_bytes_ = 0;
    }

    void copy_buffer(Buffer &destination, const Buffer &source)
    {
        check_same_or_throw(destination.size_bytes(), source.size_bytes());
        copy_buffer(destination, 0, source, 0, source.size_bytes());
    }

    void copy_buffer(Buffer &destination, std::size_t destination_offset, const Buffer &source,
                     std::size_t source_offset, std::size_t bytes)
    {
        if (destination_offset > destination.size_bytes() || bytes > destination.size_bytes() - destination_offset ||
            source_offset > source.size_bytes() || bytes > source.size_bytes() - source_offset)
            throw std::out_of_range("Buffer copy range exceeds a buffer");
        if (bytes == 0)
            return;
        auto *dst = static_cast<unsigned char *>(destination.data()) + destination_offset;
        const auto *src = static_cast<const unsigned char *>(source.data()) + source_offset;
        if (destination.device().is_cpu() && source.device().is_cpu())
        {
            std::copy(src, src + bytes, dst);
            return;
        }
        // Unified addressing: the runtime resolves both pointers' devices.
        const int device = source.device().is_cuda() ? source.device().index() : destination.device().index();
        hip::DeviceGuard guard(device);
        QWEN3_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDefault));
        guard.restore();
    }
} // namespace qwen3
