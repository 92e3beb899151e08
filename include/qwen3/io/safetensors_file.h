#pragma once

// A .safetensors file: 8-byte little-endian header length, a JSON header
// that starts with '{', then the tensor data (the reference's
// include/qwen3/io/safetensors_file.h contract).

#include "qwen3/io/mapped_file.h"

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <stdexcept>

namespace qwen3
{
    class SafetensorsFormatError final : public std::runtime_error
    {
    public:
        using std::runtime_error::runtime_error;
    };

    class SafetensorsFile final
    {
    public:
        static constexpr std::size_t kLengthPrefixSizeBytes = 8;
        static constexpr std::uint64_t kMaxHeaderSizeBytes = 100'000'000ULL;

        explicit SafetensorsFile(const std::filesystem::path &path);
        SafetensorsFile(const SafetensorsFile &) = delete;
        SafetensorsFile &operator=(const SafetensorsFile &) = delete;
        SafetensorsFile(SafetensorsFile &&) noexcept = default;
        SafetensorsFile &operator=(SafetensorsFile &&) noexcept = default;

        [[nodiscard]] std::size_t file_size_bytes() const noexcept { return mapped_.size_bytes(); }
        [[nodiscard]] std::size_t header_size_bytes() const noexcept { return header_size_; }
        [[nodiscard]] std::size_t data_offset_bytes() const noexcept { return data_offset_; }
        [[nodiscard]] std::size_t data_size_bytes() const noexcept;
        [[nodiscard]] ConstByteView header_bytes() const;
        [[nodiscard]] ConstByteView data_bytes() const;

    private:
        MappedFile mapped_;
        std::size_t header_size_ = 0;
        std::size_t data_offset_ = 0;
    };
} // namespace qwen3
