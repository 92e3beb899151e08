// Pinned, chunked host -> GPU upload (see staged_upload.hpp).
#include "staged_upload.hpp"

#include "../core/block_cache.hpp"
#include "qwen3/hip/hip_check.h"
#include "qwen3/io/copy_crew.h"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace qwen3::io_detail
{
    namespace
    {
        // Where a chunk's bytes go once its slot is on the device's side of
        // the link: `bytes` bytes at slot offset `offset` to `dst`.
        struct Landing
        {
            void *dst;
            std::size_t offset;
            std::size_t bytes;
        };

        unsigned crew_helpers(std::size_t total_bytes)
        {
            if (total_bytes < StagedUpload::kCrewMinBytes)
                return 0;
            const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
            return std::min(StagedUpload::kCopyThreads, hw) - 1;
        }
    } // namespace

    StagedUpload::StagedUpload(int device) : device_(device)
    {
        hip::DeviceGuard guard(device);
        try
        {
            QWEN3_HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
            for (std::size_t s = 0; s < kSlots; ++s)
            {
                QWEN3_HIP_CHECK(hipHostMalloc(&slot_[s], kSlotBytes, hipHostMallocDefault));
                QWEN3_HIP_CHECK(hipEventCreateWithFlags(&slot_done_[s], hipEventDisableTiming));
            }
        }
        catch (...)
        {
            release();
            throw;
        }
    }

    StagedUpload::~StagedUpload() { release(); }

    void StagedUpload::release() noexcept
    {
        int previous = 0;
        const bool restore = hipGetDevice(&previous) == hipSuccess;
        (void)hipSetDevice(device_);
        if (stream_ != nullptr)
            (void)hipStreamSynchronize(stream_);  // no DMA may still read a slot
        for (std::size_t s = 0; s < kSlots; ++s)
        {
            if (slot_done_[s] != nullptr)
                (void)hipEventDestroy(slot_done_[s]);
            if (slot_[s] != nullptr)
                (void)hipHostFree(slot_[s]);
            slot_done_[s] = nullptr;
            slot_[s] = nullptr;
        }
        if (stream_ != nullptr)
            (void)hipStreamDestroy(stream_);
        stream_ = nullptr;
        if (restore)
            (void)hipSetDevice(previous);
    }

    void StagedUpload::run(std::size_t count, std::size_t total_bytes,
                           const std::function<UploadPiece(std::size_t)> &piece)
    {
        hip::DeviceGuard guard(device_);
        // destinations made by piece() are fresh memory, which no work queued
        // on another stream can still be reading
        const qwen3::detail::FreshDeviceBlocks fresh;
        detail::CopyCrew crew(crew_helpers(total_bytes));
        // the slot being filled: host segments to copy into it, and where its bytes land
        std::size_t slot = 0, used = 0;
        std::vector<detail::CopySegment> segments;
        std::vector<Landing> landings;

        const auto send = [&] {
            if (used == 0)
                return;
            if (slot_busy_[slot])
                QWEN3_HIP_CHECK(hipEventSynchronize(slot_done_[slot]));
            crew.copy(segments.data(), segments.size());
            auto *base = static_cast<std::byte *>(slot_[slot]);
            for (const Landing &l : landings)
                QWEN3_HIP_CHECK(hipMemcpyAsync(l.dst, base + l.offset, l.bytes, hipMemcpyHostToDevice, stream_));
            QWEN3_HIP_CHECK(hipEventRecord(slot_done_[slot], stream_));
            slot_busy_[slot] = true;
            segments.clear();
            landings.clear();
            slot = (slot + 1) % kSlots;
            used = 0;
        };

        try
        {
            for (std::size_t i = 0; i < count; ++i)
            {
                const UploadPiece p = piece(i);
                // a large piece starts a slot of its own: its DMAs then stay
                // whole-slot sized and page aligned
                if (p.bytes >= kPackMaxBytes && used != 0)
                    send();
                for (std::size_t done = 0; done < p.bytes;)
                {
                    if (used == kSlotBytes)
                        send();
                    const std::size_t n = std::min(p.bytes - done, kSlotBytes - used);
                    segments.push_back({static_cast<std::byte *>(slot_[slot]) + used, p.src + done, n});
                    landings.push_back({static_cast<std::byte *>(p.dst) + done, used, n});
                    used += n;
                    done += n;
                }
            }
            send();
            QWEN3_HIP_CHECK(hipStreamSynchronize(stream_));
        }
        catch (...)
        {
            (void)hipStreamSynchronize(stream_);
            throw;
        }
        slot_busy_.fill(false);
        guard.restore();
    }

    Tensor copy_out(const SafetensorsFile &file, const SafetensorsTensorInfo &info, Device device,
                    std::string_view name)
    {
        Tensor out = Tensor::empty(info.shape, info.dtype, device);
        if (out.nbytes() != info.size_bytes())
            throw std::logic_error("Tensor size does not match metadata for '" + std::string(name) + "'");
        if (info.size_bytes() == 0)
            return out;
        const std::byte *src = file.data_bytes().data() + info.begin_offset;
        if (device.is_cpu())
        {
            std::memcpy(out.data(), src, info.size_bytes());
            return out;
        }
        hip::DeviceGuard guard(device.index());
        QWEN3_HIP_CHECK(hipMemcpy(out.data(), src, info.size_bytes(), hipMemcpyHostToDevice));
        guard.restore();
        return out;
    }
} // namespace qwen3::io_detail
