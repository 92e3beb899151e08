#include "qwen3/core/tensor_view.h"

#include "qwen3/core/tensor.h"

#include <stdexcept>
#include <utility>

namespace qwen3
{
    std::vector<std::int64_t> contiguous_strides(const Shape &shape)
    {
        std::vector<std::int64_t> strides(shape.rank());
        std::int64_t s = 1;
        for (std::size_t i = shape.rank(); i-- > 0;)
        {
            strides[i] = s;
            s *= shape[i] == 0 ? 1 : shape[i];
        }
        return strides;
    }

    TensorView::TensorView(void *data, DType dtype, Device device, Shape shape)
        : TensorView(data, dtype, device, shape, contiguous_strides(shape))
    {
    }

    TensorView::TensorView(void *data, DType dtype, Device device, Shape shape, std::vector<std::int64_t> strides)
        : data_(data), dtype_(dtype), device_(device), shape_(std::move(shape)), strides_(std::move(strides))
    {
        if (strides_.size() != shape_.rank())
            throw std::invalid_argument("TensorView stride count must equal the rank");
        for (const std::int64_t s : strides_)
        {
            if (s < 0)
                throw std::invalid_argument("TensorView strides cannot be negative");
        }
        if (data_ == nullptr && !shape_.has_zero_dimension())
            throw std::invalid_argument("TensorView with elements needs non-null data");
    }

    std::size_t TensorView::nbytes() const { return checked_nbytes(shape_.numel(), dtype_); }

    std::int64_t TensorView::stride(std::size_t axis) const
    {
        if (axis >= strides_.size())
            throw std::out_of_range("TensorView stride axis out of range");
        return strides_[axis];
    }

    bool TensorView::is_contiguous() const { return strides_ == contiguous_strides(shape_); }

    TensorView TensorView::transpose(std::size_t axis_a, std::size_t axis_b) const
    {
        if (axis_a >= rank() || axis_b >= rank())
            throw std::out_of_range("TensorView transpose axis out of range");
        std::vector<Shape::Dimension> dims = shape_.dimensions();
        std::vector<std::int64_t> strides = strides_;
        std::swap(dims[axis_a], dims[axis_b]);
        std::swap(strides[axis_a], strides[axis_b]);
        return TensorView(data_, dtype_, device_, Shape(std::move(dims)), std::move(strides));
    }
} // namespace qwen3
