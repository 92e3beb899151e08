#pragma once

// Tensor records of a safetensors header (dtype BF16 / F32 / I32, shape,
// data_offsets relative to the data section), checked against the file
// (the reference's include/qwen3/io/safetensors_metadata.h contract).

#include "qwen3/core/dtype.h"
#include "qwen3/core/shape.h"
#include "qwen3/io/safetensors_file.h"

#include <cstddef>
#include <string>
#include <string_view>
#include <unordered_map>

namespace qwen3
{
    struct SafetensorsTensorInfo final
    {
        DType dtype;
        Shape shape;
        std::size_t begin_offset;
        std::size_t end_offset;
        [[nodiscard]] std::size_t size_bytes() const noexcept { return end_offset - begin_offset; }
    };

    class SafetensorsMetadata final
    {
    public:
        // Throws SafetensorsFormatError for malformed JSON or records.
        explicit SafetensorsMetadata(const SafetensorsFile &file);
        [[nodiscard]] std::size_t tensor_count() const noexcept { return tensors_.size(); }
        [[nodiscard]] bool contains(std::string_view name) const;
        // Throws std::out_of_range for an unknown name.
        [[nodiscard]] const SafetensorsTensorInfo &tensor(std::string_view name) const;
        [[nodiscard]] const std::unordered_map<std::string, SafetensorsTensorInfo> &tensors() const noexcept
        {
            return tensors_;
        }

    private:
        std::unordered_map<std::string, SafetensorsTensorInfo> tensors_;
    };
} // namespace qwen3
