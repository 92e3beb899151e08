#pragma once

// A model directory holding either model.safetensors or
// model.safetensors.index.json with its shards.  Public interface of the
// reference's include/qwen3/io/safetensors_checkpoint.h.  Every tensor of
// every shard lives in one table sorted by name; load_many() reads any mix
// of shards through a single staged upload.

#include "qwen3/core/device.h"
#include "qwen3/core/tensor.h"
#include "qwen3/io/safetensors_metadata.h"

#include <cstddef>
#include <filesystem>
#include <string>
#include <string_view>
#include <vector>

namespace qwen3
{
    class SafetensorsCheckpoint final
    {
    public:
        // Throws std::invalid_argument for a missing directory and
        // std::runtime_error for an ambiguous or inconsistent checkpoint.
        explicit SafetensorsCheckpoint(const std::filesystem::path &model_directory);
        SafetensorsCheckpoint(const SafetensorsCheckpoint &) = delete;
        SafetensorsCheckpoint &operator=(const SafetensorsCheckpoint &) = delete;
        SafetensorsCheckpoint(SafetensorsCheckpoint &&) = default;
        SafetensorsCheckpoint &operator=(SafetensorsCheckpoint &&) = default;

        [[nodiscard]] const std::filesystem::path &model_directory() const noexcept { return model_directory_; }
        [[nodiscard]] bool is_sharded() const noexcept { return sharded_; }
        [[nodiscard]] std::size_t shard_count() const noexcept { return shard_files_.size(); }
        [[nodiscard]] std::size_t tensor_count() const noexcept { return table_.size(); }
        [[nodiscard]] bool contains(std::string_view tensor_name) const;
        // Throws std::out_of_range for an unknown name.
        [[nodiscard]] const SafetensorsTensorInfo &tensor_info(std::string_view tensor_name) const;
        [[nodiscard]] Tensor load(std::string_view tensor_name, Device target_device) const;
        // Results in the order of the names; every name is resolved before
        // any byte moves.
        [[nodiscard]] std::vector<Tensor> load_many(const std::vector<std::string> &tensor_names,
                                                    Device target_device) const;

        // One row of the tensor table.
        struct Entry
        {
            std::string name;
            std::size_t shard;
            SafetensorsTensorInfo info;
        };

    private:
        [[nodiscard]] const Entry *find(std::string_view name) const;
        [[nodiscard]] const Entry &find_or_throw(std::string_view name) const;

        std::filesystem::path model_directory_;
        bool sharded_ = false;
        std::vector<std::filesystem::path> shard_files_;
        std::vector<Entry> table_;  // sorted by name
    };
} // namespace qwen3
