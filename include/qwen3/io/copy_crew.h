#pragma once

// A crew of helper threads that splits one large host copy with the calling
// thread (used by the safetensors upload to fill its pinned staging slots
// from mapped files).  A copy is a list of segments; the crew treats them as
// one concatenated byte range and cuts that range into equal parts of whole
// 4 KiB pages, one per thread.  Header-only so the host tests can build it
// under ThreadSanitizer.

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace qwen3::detail
{
    // One piece of a gathered copy: `bytes` bytes from `src` to `dst`.
    struct CopySegment
    {
        void *dst;
        const void *src;
        std::size_t bytes;
    };

    // copy() returns once every part is written, and is called from one
    // thread at a time.
    //
    // Hand-off: the caller stores the job, then bumps `sequence_` under the
    // mutex and wakes the helpers; a helper that finishes its part
    // decrements `remaining_` and the one that reaches zero wakes the
    // caller.  Both sides poll for a short while (a chunk arrives every
    // ~0.1 ms during a load) before they block on a condition variable, so
    // no thread burns a core while the caller waits for a DMA.
    class CopyCrew final
    {
    public:
        explicit CopyCrew(unsigned helpers)
        {
            threads_.reserve(helpers);
            try
            {
                for (unsigned i = 0; i < helpers; ++i)
                    threads_.emplace_back([this, i] { run(i + 1); });
            }
            catch (...)
            {
                stop();
                throw;
            }
        }
        ~CopyCrew() { stop(); }
        CopyCrew(const CopyCrew &) = delete;
        CopyCrew &operator=(const CopyCrew &) = delete;

        [[nodiscard]] std::size_t helpers() const noexcept { return threads_.size(); }

        void copy(void *dst, const void *src, std::size_t bytes)
        {
            const CopySegment one{dst, src, bytes};
            copy(&one, 1);
        }

        void copy(const CopySegment *segments, std::size_t count)
        {
            std::size_t total = 0;
            for (std::size_t i = 0; i < count; ++i)
                total += segments[i].bytes;
            const std::size_t parts = threads_.size() + 1;
            if (parts == 1 || total < kMinSplitBytes)
            {
                for (std::size_t i = 0; i < count; ++i)
                    if (segments[i].bytes != 0)
                        std::memcpy(segments[i].dst, segments[i].src, segments[i].bytes);
                return;
            }
            segments_ = segments;
            count_ = count;
            total_ = total;
            part_ = ((total + parts - 1) / parts + 4095) & ~std::size_t{4095};
            remaining_.store(static_cast<int>(threads_.size()), std::memory_order_relaxed);
            {
                std::lock_guard<std::mutex> lock(mutex_);
                sequence_.fetch_add(1, std::memory_order_release);
            }
            work_.notify_all();
            copy_part(0);
            if (!poll([this] { return remaining_.load(std::memory_order_acquire) == 0; }))
            {
                std::unique_lock<std::mutex> lock(mutex_);
                done_.wait(lock, [this] { return remaining_.load(std::memory_order_acquire) == 0; });
            }
        }

    private:
        static constexpr int kPollRounds = 4096;
        // below this many bytes the caller copies alone (waking the crew costs more)
        static constexpr std::size_t kMinSplitBytes = 256 * 1024;

        static void pause() noexcept
        {
#if defined(__x86_64__)
            __builtin_ia32_pause();
#else
            std::this_thread::yield();
#endif
        }

        template <typename Ready>
        static bool poll(Ready ready)
        {
            for (int i = 0; i < kPollRounds; ++i)
            {
                if (ready())
                    return true;
                pause();
            }
            return ready();
        }

        // Copies bytes [part * part_, (part + 1) * part_) of the concatenated segments.
        void copy_part(std::size_t part) const noexcept
        {
            std::size_t begin = std::min(total_, part_ * part);
            const std::size_t end = std::min(total_, part_ * (part + 1));
            std::size_t base = 0;  // offset of segment i in the concatenation
            for (std::size_t i = 0; i < count_ && begin < end; ++i)
            {
                const CopySegment &s = segments_[i];
                const std::size_t seg_end = base + s.bytes;
                if (begin < seg_end)
                {
                    const std::size_t from = begin - base, to = std::min(end, seg_end) - base;
                    std::memcpy(static_cast<std::byte *>(s.dst) + from, static_cast<const std::byte *>(s.src) + from,
                                to - from);
                    begin = base + to;
                }
                base = seg_end;
            }
        }

        void run(std::size_t part)
        {
            std::uint64_t seen = 0;
            for (;;)
            {
                auto ready = [&] {
                    return sequence_.load(std::memory_order_acquire) != seen || stop_.load(std::memory_order_acquire);
                };
                if (!poll(ready))
                {
                    std::unique_lock<std::mutex> lock(mutex_);
                    work_.wait(lock, ready);
                }
                const std::uint64_t s = sequence_.load(std::memory_order_acquire);
                if (s == seen)
                    return;   // stopped with no new copy
                seen = s;
                copy_part(part);
                if (remaining_.fetch_sub(1, std::memory_order_acq_rel) == 1)
                {
                    { std::lock_guard<std::mutex> lock(mutex_); }
                    done_.notify_one();
                }
            }
        }

        void stop() noexcept
        {
            {
                std::lock_guard<std::mutex> lock(mutex_);
                stop_.store(true, std::memory_order_release);
            }
            work_.notify_all();
            for (auto &t : threads_)
                t.join();
            threads_.clear();
        }

        std::vector<std::thread> threads_;
        std::mutex mutex_;
        std::condition_variable work_, done_;
        std::atomic<std::uint64_t> sequence_{0};
        std::atomic<int> remaining_{0};
        std::atomic<bool> stop_{false};
        const CopySegment *segments_ = nullptr;
        std::size_t count_ = 0;
        std::size_t total_ = 0;
        std::size_t part_ = 0;
    };
} // namespace qwen3::detail
