// Read-only mmap of a file (contract of the reference's
// src/io/mapped_file.cpp: errno-carrying std::system_error for open/fstat/
// mmap failures, std::invalid_argument for a non-regular file, an empty
// view for an empty file).
#include "qwen3/io/mapped_file.h"

#include <cerrno>
#include <fcntl.h>
#include <limits>
#include <stdexcept>
#include <string>
#include <sys/mman.h>
#include <sys/stat.h>
#include <system_error>
#include <unistd.h>
#include <utility>

namespace qwen3
{
    ConstByteView ConstByteView::subview(std::size_t offset, std::size_t count) const
    {
        if (offset > size_bytes_ || count > size_bytes_ - offset)
            throw std::out_of_range("byte subview is out of range");
        return ConstByteView{data_ + offset, count};
    }

    MappedFile::MappedFile(const std::filesystem::path &path)
    {
        const std::string text = path.string();
        const int fd = ::open(text.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0)
            throw std::system_error(errno, std::generic_category(), "open " + text);
        struct stat st
        {
        };
        if (::fstat(fd, &st) != 0)
        {
            const int e = errno;
            ::close(fd);
            throw std::system_error(e, std::generic_category(), "fstat " + text);
        }
        if (!S_ISREG(st.st_mode))
        {
            ::close(fd);
            throw std::invalid_argument("mapped path is not a regular file: " + text);
        }
        if (st.st_size < 0)
        {
            ::close(fd);
            throw std::runtime_error("file has a negative size: " + text);
        }
        if (static_cast<std::uint64_t>(st.st_size) > std::numeric_limits<std::size_t>::max())
        {
            ::close(fd);
            throw std::overflow_error("file is too large for this process: " + text);
        }
        size_bytes_ = static_cast<std::size_t>(st.st_size);
        if (size_bytes_ == 0)
        {
            ::close(fd);
            return;
        }
        void *p = ::mmap(nullptr, size_bytes_, PROT_READ, MAP_PRIVATE, fd, 0);
        const int e = errno;
        ::close(fd);
        if (p == MAP_FAILED)
        {
            size_bytes_ = 0;
            throw std::system_error(e, std::generic_category(), "mmap " + text);
        }
        data_ = static_cast<const std::byte *>(p);
    }

    MappedFile::~MappedFile() noexcept { unmap(); }

    MappedFile::MappedFile(MappedFile &&other) noexcept
        : data_(std::exchange(other.data_, nullptr)), size_bytes_(std::exchange(other.size_bytes_, 0))
    {
    }

    MappedFile &MappedFile::operator=(MappedFile &&other) noexcept
    {
        if (this != &other)
        {
            unmap();
            data_ = std::exchange(other.data_, nullptr);
            size_bytes_ = std::exchange(other.size_bytes_, 0);
        }
        return *this;
    }

    void MappedFile::unmap() noexcept
    {
        if (data_ != nullptr)
            ::munmap(const_cast<std::byte *>(data_), size_bytes_);
        data_ = nullptr;
        size_bytes_ = 0;
    }
} // namespace qwen3
