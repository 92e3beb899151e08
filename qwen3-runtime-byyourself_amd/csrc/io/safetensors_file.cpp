// Framing of a .safetensors file (checks and messages of the reference's
// src/io/safetensors_file.cpp).
#include "qwen3/io/safetensors_file.h"

#include <string>

namespace qwen3
{
    SafetensorsFile::SafetensorsFile(const std::filesystem::path &path) : mapped_(path)
    {
        const std::string text = path.string();
        const ConstByteView bytes = mapped_.bytes();
        if (bytes.size_bytes() < kLengthPrefixSizeBytes)
            throw SafetensorsFormatError("safetensors file is shorter than the 8-byte header length prefix: " + text);
        std::uint64_t length = 0;
        for (std::size_t i = 0; i < kLengthPrefixSizeBytes; ++i)
            length |= static_cast<std::uint64_t>(std::to_integer<unsigned char>(bytes.data()[i])) << (8 * i);
        if (length == 0)
            throw SafetensorsFormatError("safetensors header is empty: " + text);
        if (length > kMaxHeaderSizeBytes)
            throw SafetensorsFormatError("safetensors header exceeds 100,000,000 bytes: " + text);
        if (length > static_cast<std::uint64_t>(bytes.size_bytes() - kLengthPrefixSizeBytes))
            throw SafetensorsFormatError("safetensors header extends beyond the end of the file: " + text);
        header_size_ = static_cast<std::size_t>(length);
        data_offset_ = kLengthPrefixSizeBytes + header_size_;
        if (std::to_integer<unsigned char>(header_bytes().data()[0]) != static_cast<unsigned char>('{'))
            throw SafetensorsFormatError("safetensors header must begin with '{': " + text);
    }

    std::size_t SafetensorsFile::data_size_bytes() const noexcept
    {
        return data_offset_ == 0 ? 0 : mapped_.size_bytes() - data_offset_;
    }

    ConstByteView SafetensorsFile::header_bytes() const
    {
        return data_offset_ == 0 ? ConstByteView{} : mapped_.bytes().subview(kLengthPrefixSizeBytes, header_size_);
    }

    ConstByteView SafetensorsFile::data_bytes() const
    {
        return data_offset_ == 0 ? ConstByteView{} : mapped_.bytes().subview(data_offset_, data_size_bytes());
    }
} // namespace qwen3
