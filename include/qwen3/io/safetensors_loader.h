#pragma once

// Loads tensors of one safetensors file to the host or a GPU.  Public
// interface of the reference's include/qwen3/io/safetensors_loader.h.
// load_many() to a GPU streams the batch through pinned staging slots on a
// non-blocking stream, filled by several host threads; the staging is made
// on the first GPU batch and kept for later ones.

#include "qwen3/core/device.h"
#include "qwen3/core/tensor.h"
#include "qwen3/io/safetensors_file.h"
#include "qwen3/io/safetensors_metadata.h"

#include <filesystem>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace qwen3
{
    namespace io_detail
    {
        class StagedUpload;
    }

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
        // One tensor, plain synchronous copy.  Throws std::out_of_range for
        // an unknown name.
        [[nodiscard]] Tensor load(std::string_view tensor_name, Device target_device) const;
        // Results in the order of the names, every one on the device when
        // the call returns; all names are resolved before any byte moves.
        [[nodiscard]] std::vector<Tensor> load_many(const std::vector<std::string> &tensor_names, Device target_device);

    private:
        SafetensorsFile file_;
        SafetensorsMetadata metadata_;
        std::unique_ptr<io_detail::StagedUpload> upload_;
    };
} // namespace qwen3
