#pragma once

// Non-owning strided view.  Contract pinned by the reference's
// tests/unit/tensor_view_test.cpp: contiguous strides by default, transpose
// swaps shape and strides without copying, null data with elements throws
// std::invalid_argument, stride() past the rank throws std::out_of_range,
// nbytes() throws std::overflow_error.

#include "qwen3/core/device.h"
#include "qwen3/core/dtype.h"
#include "qwen3/core/shape.h"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace qwen3
{
    class TensorView
    {
    public:
        TensorView(void *data, DType dtype, Device device, Shape shape);
        TensorView(void *data, DType dtype, Device device, Shape shape, std::vector<std::int64_t> strides);

        [[nodiscard]] void *data() const noexcept { return data_; }
        [[nodiscard]] DType dtype() const noexcept { return dtype_; }
        [[nodiscard]] const Device &device() const noexcept { return device_; }
        [[nodiscard]] const Shape &shape() const noexcept { return shape_; }
        [[nodiscard]] std::size_t rank() const noexcept { return shape_.rank(); }
        [[nodiscard]] std::int64_t numel() const { return shape_.numel(); }
        [[nodiscard]] std::size_t nbytes() const;
        [[nodiscard]] std::int64_t dim(std::size_t axis) const { return shape_[axis]; }
        [[nodiscard]] std::int64_t stride(std::size_t axis) const;
        [[nodiscard]] const std::vector<std::int64_t> &strides() const noexcept { return strides_; }
        [[nodiscard]] bool is_contiguous() const;
        [[nodiscard]] bool is_empty() const { return shape_.has_zero_dimension(); }
        [[nodiscard]] TensorView transpose(std::size_t axis_a, std::size_t axis_b) const;

    private:
        void *data_;
        DType dtype_;
        Device device_;
        Shape shape_;
        std::vector<std::int64_t> strides_;
    };

    // Row-major strides of a shape, in elements.
    [[nodiscard]] std::vector<std::int64_t> contiguous_strides(const Shape &shape);
} // namespace qwen3
