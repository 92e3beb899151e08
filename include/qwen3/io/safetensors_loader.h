#pragma once

// Loads tensors of one safetensors file to the host or a GPU (the
// reference's include/qwen3/io/safetensors_loader.h interface).  GPU batches
// go through three pinned 8 MiB staging buffers (hipHostMalloc) on a
// non-blocking stream: each chunk is copied out of the mapped file by up to
// kCopyThreads host threads, and that copy overlaps the DMA of the previous
// chunks.  One host thread copies at about half the host-to-device link's
// rate, so the copy is split; pinned memory costs about 0.25 ms per MiB to
// allocate, so the staging is kept small.

#include "qwen3/core/device.h"
#include "qwen3/core/tensor.h"
#include "qwen3/io/safetensors_file.h"
#include "qwen3/io/safetensors_metadata.h"

#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <string>
#include <string_view>
#include <vector>

struct ihipStream_t;
struct ihipEvent_t;

namespace qwen3
{
    class SafetensorsLoader final
    {
    public:
        explicit SafetensorsLoader(const std::filesystem::path &model_path);
        ~SafetensorsLoader();
        SafetensorsLoader(const SafetensorsLoader &) = delete;
        SafetensorsLoader &operator=(const SafetensorsLoader &) = delete;
        SafetensorsLoader(SafetensorsLoader &&) = delete;
        SafetensorsLoader &operator=(SafetensorsLoader &&) = delete;

        [[nodiscard]] const SafetensorsMetadata &metadata() const noexcept { return metadata_; }
        [[nodiscard]] Tensor load(std::string_view tensor_name, Device target_device) const;
        [[nodiscard]] std::vector<Tensor> load_many(const std::vector<std::string> &tensor_names, Device target_device);

        static constexpr std::size_t kStagingSlotCount = 3;
        static constexpr std::size_t kStagingBufferBytes = 8ULL * 1024ULL * 1024ULL;
        // threads that copy one chunk into staging (the calling thread included)
        static constexpr unsigned kCopyThreads = 8;
        // batches below this many bytes are staged by the calling thread alone
        static constexpr std::size_t kParallelCopyMinBytes = 32ULL * 1024ULL * 1024ULL;

    private:
        void ensure_transfer_resources(int device_index);
        void release_transfer_resources() noexcept;
        [[nodiscard]] const std::byte *source_data(const SafetensorsTensorInfo &info) const noexcept;

        SafetensorsFile file_;
        SafetensorsMetadata metadata_;
        ihipStream_t *stream_ = nullptr;
        std::array<void *, kStagingSlotCount> staging_{};
        std::array<ihipEvent_t *, kStagingSlotCount> events_{};
        int transfer_device_ = -1;
    };
} // namespace qwen3
