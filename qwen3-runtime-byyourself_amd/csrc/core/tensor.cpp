#include "qwen3/core/tensor.h"

#include <limits>
#include <stdexcept>
#include <utility>

namespace qwen3
{
    std::size_t checked_nbytes(std::int64_t numel, DType dtype)
    {
        const auto size = static_cast<std::int64_t>(dtype_size(dtype));
        if (numel > std::numeric_limits<std::int64_t>::max() / size)
            throw std::overflow_error("Tensor byte size overflows");
        return static_cast<std::size_t>(numel * size);
    }

    Tensor::Tensor(Shape shape, DType dtype, Buffer buffer) noexcept
        : shape_(std::move(shape)), dtype_(dtype), buffer_(std::move(buffer))
    {
    }

    Tensor Tensor::empty(Shape shape, DType dtype, Device device)
    {
        const std::size_t bytes = checked_nbytes(shape.numel(), dtype);
        Buffer buffer(bytes, device);
        return Tensor(std::move(shape), dtype, std::move(buffer));
    }

    Tensor &Tensor::operator=(Tensor &&other) noexcept
    {
        if (this != &other)
        {
            shape_ = std::move(other.shape_);
            dtype_ = other.dtype_;
            buffer_ = std::move(other.buffer_);
        }
        return *this;
    }

    TensorView Tensor::view() const
    {
        return TensorView(const_cast<void *>(buffer_.data()), dtype_, buffer_.device(), shape_);
    }

    Tensor Tensor::clone() const { return copy_to(device()); }

    Tensor Tensor::copy_to(Device device) const
    {
        Tensor out = Tensor::empty(shape_, dtype_, device);
        copy_buffer(out.buffer_, buffer_);
        return out;
    }

    void Tensor::copy_from(const Tensor &source)
    {
        if (source.shape_ != shape_)
            throw std::invalid_argument("Tensor copy_from requires identical shapes");
        if (source.dtype_ != dtype_)
            throw std::invalid_argument("Tensor copy_from requires identical dtypes");
        copy_buffer(buffer_, source.buffer_);
    }
} // namespace qwen3
