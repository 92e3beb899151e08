// Host -> GPU transfer of many tensors through a ring of pinned staging
// slots, shared by SafetensorsLoader and SafetensorsCheckpoint.
//
// The pieces of a batch are treated as one byte stream that is cut into
// slot-sized chunks; a chunk may hold the tail of one tensor and any number
// of small tensors after it (norm weights, biases), so those share a slot
// instead of taking one each, while a large tensor always starts a slot.  A chunk is copied out of the mapped files
// into its slot by a crew of host threads (qwen3::detail::CopyCrew), then
// sent with one async copy per destination piece on the upload's own
// non-blocking stream; a slot is refilled once the event recorded after its
// last copy has completed, so host copies of later chunks overlap the DMA of
// earlier ones.  Destinations are allocated as fresh device memory (never a
// reused block that work queued on the default stream might still read), so
// the upload needs no wait on that stream; such a wait measured 3.5 ms per
// 1.5 GB batch (41 against 46 GB/s).
#pragma once

#include "qwen3/core/device.h"
#include "qwen3/core/tensor.h"
#include "qwen3/io/safetensors_file.h"
#include "qwen3/io/safetensors_metadata.h"

#include <array>
#include <cstddef>
#include <functional>
#include <string_view>

struct ihipStream_t;
struct ihipEvent_t;

namespace qwen3::io_detail
{
    // `bytes` bytes from host memory `src` to device memory `dst`.
    struct UploadPiece
    {
        const std::byte *src;
        void *dst;
        std::size_t bytes;
    };

    class StagedUpload final
    {
    public:
        static constexpr std::size_t kSlots = 3;
        // Small slots: fresh pinned memory faults on its first host write
        // (measured 2.9 GB/s for the first copy into a new buffer, 29 GB/s
        // for the second), so large ones cost more than they save.
        static constexpr std::size_t kSlotBytes = 8ULL << 20;
        // Threads that fill a slot (the caller included), and the batch size
        // from which they are started.
        static constexpr unsigned kCopyThreads = 8;
        static constexpr std::size_t kCrewMinBytes = 32ULL << 20;
        // Pieces below this size share slots with their neighbours; larger
        // ones start a fresh slot.
        static constexpr std::size_t kPackMaxBytes = 1ULL << 20;

        explicit StagedUpload(int device);
        ~StagedUpload();
        StagedUpload(const StagedUpload &) = delete;
        StagedUpload &operator=(const StagedUpload &) = delete;

        [[nodiscard]] int device() const noexcept { return device_; }

        // Moves `count` pieces; piece(i) is asked for when the stream reaches
        // it (the caller allocates the destination there, while earlier
        // chunks are in flight).  Returns once every byte is on the device;
        // on an exception the copies already queued are waited for first.
        void run(std::size_t count, std::size_t total_bytes, const std::function<UploadPiece(std::size_t)> &piece);

    private:
        void release() noexcept;

        int device_;
        ihipStream_t *stream_ = nullptr;
        std::array<void *, kSlots> slot_{};
        std::array<ihipEvent_t *, kSlots> slot_done_{};
        std::array<bool, kSlots> slot_busy_{};
    };

    // One tensor of a mapped safetensors file as a new tensor on `device`
    // (a plain copy; the GPU copy is synchronous).
    [[nodiscard]] Tensor copy_out(const SafetensorsFile &file, const SafetensorsTensorInfo &info, Device device,
                                  std::string_view name);
} // namespace qwen3::io_detail
