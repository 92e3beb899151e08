#pragma once

// Read-only memory mapping of a file and a bounds-checked byte view of it
// (the reference's include/qwen3/io/mapped_file.h contract).

#include <cstddef>
#include <filesystem>

namespace qwen3
{
    class MappedFile;

    class ConstByteView final
    {
    public:
        ConstByteView() noexcept = default;
        [[nodiscard]] const std::byte *data() const noexcept { return data_; }
        [[nodiscard]] std::size_t size_bytes() const noexcept { return size_bytes_; }
        [[nodiscard]] bool empty() const noexcept { return size_bytes_ == 0; }
        // Throws std::out_of_range when [offset, offset + count) leaves the view.
        [[nodiscard]] ConstByteView subview(std::size_t offset, std::size_t count) const;

    private:
        friend class MappedFile;
        ConstByteView(const std::byte *data, std::size_t size_bytes) noexcept : data_(data), size_bytes_(size_bytes) {}
        const std::byte *data_ = nullptr;
        std::size_t size_bytes_ = 0;
    };

    class MappedFile final
    {
    public:
        // Throws std::system_error if the file cannot be opened, stat'ed or
        // mapped, std::invalid_argument if it is not a regular file.  An empty
        // file maps to an empty view.
        explicit MappedFile(const std::filesystem::path &path);
        ~MappedFile() noexcept;
        MappedFile(const MappedFile &) = delete;
        MappedFile &operator=(const MappedFile &) = delete;
        MappedFile(MappedFile &&other) noexcept;
        MappedFile &operator=(MappedFile &&other) noexcept;

        [[nodiscard]] const std::byte *data() const noexcept { return data_; }
        [[nodiscard]] std::size_t size_bytes() const noexcept { return size_bytes_; }
        [[nodiscard]] bool empty() const noexcept { return size_bytes_ == 0; }
        [[nodiscard]] ConstByteView bytes() const noexcept { return ConstByteView{data_, size_bytes_}; }

    private:
        void unmap() noexcept;
        const std::byte *data_ = nullptr;
        std::size_t size_bytes_ = 0;
    };
} // namespace qwen3
