#include "qwen3/core/buffer.h"

#include "qwen3/hip/hip_check.h"
#include "block_cache.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <map>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

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

        std::atomic<std::uint64_t> g_device_allocations{0};
        thread_local int t_fresh_blocks = 0;  // FreshDeviceBlocks scopes open on this thread

        // QWEN3_DEVICE_BLOCK_CACHE=0 in the environment turns the small-block
        // cache off for the process: every device block is then freed with
        // hipFree, which waits for the whole device, as the reference's
        // Buffer does.  Read once, at the first device allocation.
        bool block_cache_enabled()
        {
            static const bool enabled = [] {
                const char *v = std::getenv("QWEN3_DEVICE_BLOCK_CACHE");
                return v == nullptr || std::string(v) != "0";
            }();
            return enabled;
        }

        // Small device blocks are kept when their Buffer is destroyed and
        // handed to the next Buffer of the same size class on that device,
        // so a decode loop that makes and drops the same small tensors every
        // token (token ids, argmax and attention workspaces) stops calling
        // hipMalloc and hipFree, whose free waits for the whole device.  A
        // block is reused in the order of the default stream, where the ops
        // run: work on another stream that reads a tensor must finish before
        // the tensor is destroyed.  Large blocks (weights, activations) are
        // not kept.
        class SmallBlockCache
        {
        public:
            static constexpr std::size_t kMaxBlock = std::size_t{4} << 20;  // larger sizes are not cached
            static constexpr std::size_t kMaxKeptPerDevice = std::size_t{64} << 20;

            static bool cached(std::size_t bytes) { return bytes <= kMaxBlock; }

            // Size class: the next power of two, at least 512 bytes.
            static std::size_t size_class(std::size_t bytes)
            {
                std::size_t c = 512;
                while (c < bytes)
                    c *= 2;
                return c;
            }

            void *take(int device, std::size_t cls)
            {
                std::lock_guard<std::mutex> lock(mutex_);
                if (static_cast<std::size_t>(device) >= kept_.size())
                    return nullptr;
                auto &lists = kept_[static_cast<std::size_t>(device)];
                auto it = lists.free.find(cls);
                if (it == lists.free.end() || it->second.empty())
                    return nullptr;
                void *p = it->second.back();
                it->second.pop_back();
                lists.bytes -= cls;
                return p;
            }

            // Keeps the block; false when the device's kept bytes are at the cap.
            bool keep(int device, std::size_t cls, void *p)
            {
                std::lock_guard<std::mutex> lock(mutex_);
                if (static_cast<std::size_t>(device) >= kept_.size())
                    kept_.resize(static_cast<std::size_t>(device) + 1);
                auto &lists = kept_[static_cast<std::size_t>(device)];
                if (lists.bytes + cls > kMaxKeptPerDevice)
                    return false;
                lists.free[cls].push_back(p);
                lists.bytes += cls;
                return true;
            }

            // Every kept block, per device, removed from the cache.
            std::vector<std::vector<void *>> drain()
            {
                std::lock_guard<std::mutex> lock(mutex_);
                std::vector<std::vector<void *>> out(kept_.size());
                for (std::size_t d = 0; d < kept_.size(); ++d)
                {
                    for (auto &entry : kept_[d].free)
                        out[d].insert(out[d].end(), entry.second.begin(), entry.second.end());
                    kept_[d].free.clear();
                    kept_[d].bytes = 0;
                }
                return out;
            }

        private:
            struct PerDevice
            {
                std::map<std::size_t, std::vector<void *>> free;
                std::size_t bytes = 0;
            };
            std::mutex mutex_;
            std::vector<PerDevice> kept_;
        };

        // Never destroyed: blocks kept at exit go with the process (freeing
        // them from a static destructor could run after the HIP runtime).
        SmallBlockCache &block_cache()
        {
            static SmallBlockCache *cache = new SmallBlockCache;
            return *cache;
        }

        void *allocate_device(std::size_t bytes, int index)
        {
            const bool small = SmallBlockCache::cached(bytes) && block_cache_enabled();
            const std::size_t alloc = small ? SmallBlockCache::size_class(bytes) : bytes;
            if (small && t_fresh_blocks == 0)
                if (void *p = block_cache().take(index, alloc))
                    return p;
            hip::DeviceGuard guard(index);
            void *p = nullptr;
            QWEN3_HIP_CHECK(hipMalloc(&p, alloc));
            g_device_allocations.fetch_add(1, std::memory_order_relaxed);
            guard.restore();
            return p;
        }

        void free_device(void *p, std::size_t bytes, int index) noexcept
        {
            try
            {
                if (SmallBlockCache::cached(bytes) && block_cache_enabled() &&
                    block_cache().keep(index, SmallBlockCache::size_class(bytes), p))
                    return;
            }
            catch (...)
            {
                // no room to record the block: free it instead
            }
            static_cast<void>(hipFree(p));
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
            free_device(data_, size_bytes_, device_.index());
        data_ = nullptr;
        size_bytes_ = 0;
    }

    detail::FreshDeviceBlocks::FreshDeviceBlocks() noexcept { ++t_fresh_blocks; }
    detail::FreshDeviceBlocks::~FreshDeviceBlocks() { --t_fresh_blocks; }

    std::uint64_t device_allocation_count() noexcept { return g_device_allocations.load(std::memory_order_relaxed); }

    void release_cached_device_blocks()
    {
        auto kept = block_cache().drain();
        for (std::size_t d = 0; d < kept.size(); ++d)
        {
            if (kept[d].empty())
                continue;
            hip::DeviceGuard guard(static_cast<int>(d));
            for (void *p : kept[d])
                QWEN3_HIP_CHECK(hipFree(p));
            guard.restore();
        }
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
