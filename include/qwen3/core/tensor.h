#pragma once

// Owning, move-only, contiguous row-major tensor.  Contract pinned by the
// reference's tests/unit/tensor_cpu_test.cpp and tensor_cuda_test.cpp: not
// default-constructible or copyable, noexcept-movable, data() is null iff the
// tensor has no elements, byte-size overflow throws std::overflow_error,
// copy_from checks shape and dtype (std::invalid_argument), no operation
// changes the current device.

#include "qwen3/core/buffer.h"
#include "qwen3/core/device.h"
#include "qwen3/core/dtype.h"
#include "qwen3/core/shape.h"
#include "qwen3/core/tensor_view.h"

#include <cstddef>
#include <cstdint>

namespace qwen3
{
    class Tensor
    {
    public:
        [[nodiscard]] static Tensor empty(Shape shape, DType dtype, Device device);

        Tensor(const Tensor &) = delete;
        Tensor &operator=(const Tensor &) = delete;
        Tensor(Tensor &&other) noexcept = default;
        Tensor &operator=(Tensor &&other) noexcept;

        [[nodiscard]] void *data() noexcept { return buffer_.data(); }
        [[nodiscard]] const void *data() const noexcept { return buffer_.data(); }
        [[nodiscard]] const Shape &shape() const noexcept { return shape_; }
        [[nodiscard]] DType dtype() const noexcept { return dtype_; }
        [[nodiscard]] const Device &device() const noexcept { return buffer_.device(); }
        [[nodiscard]] std::int64_t numel() const { return shape_.numel(); }
        [[nodiscard]] std::size_t nbytes() const noexcept { return buffer_.size_bytes(); }
        [[nodiscard]] bool is_empty() const noexcept { return shape_.has_zero_dimension(); }

        [[nodiscard]] TensorView view() const;
        [[nodiscard]] Tensor clone() const;
        [[nodiscard]] Tensor copy_to(Device device) const;
        void copy_from(const Tensor &source);

    private:
        Tensor(Shape shape, DType dtype, Buffer buffer) noexcept;

        Shape shape_;
        DType dtype_;
        Buffer buffer_;
    };

    // Bytes of `numel` elements of `dtype`; throws std::overflow_error.
    [[nodiscard]] std::size_t checked_nbytes(std::int64_t numel, DType dtype);
} // namespace qwen3
