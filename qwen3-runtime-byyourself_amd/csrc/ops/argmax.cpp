// qwen3::ops::argmax_last_dimension over the gfx950 argmax kernel.  Checks,
// their order and exception types follow src/ops/argmax.cu:104-214.
#include "qwen3/ops/argmax.h"

#include "ops_common.hpp"

#include <limits>
#include <utility>
#include <vector>

namespace qwen3::ops
{
    Tensor argmax_last_dimension(const Tensor &input, bool keep_dimension, std::int64_t valid_reduction_size)
    {
        detail::require(input.dtype() == DType::BFloat16, "argmax input must have BFloat16 dtype");
        detail::require(input.device().is_cuda(), "argmax input must be on CUDA");
        detail::require(input.shape().rank() != 0, "argmax input cannot be scalar");
        const std::size_t last = input.shape().rank() - 1;
        const std::int64_t row_stride = input.shape()[last];
        detail::require(row_stride > 0, "argmax reduction dimension must be positive");
        detail::require(row_stride <= std::numeric_limits<std::int32_t>::max(),
                        "argmax reduction dimension exceeds Int32 index range");
        detail::require(valid_reduction_size >= 0 && valid_reduction_size <= row_stride,
                        "valid reduction size is outside the last dimension");
        const std::int64_t search = valid_reduction_size == 0 ? row_stride : valid_reduction_size;
        const std::int64_t rows = input.numel() / row_stride;
        std::vector<Shape::Dimension> dims = input.shape().dimensions();
        if (keep_dimension)
            dims.back() = 1;
        else
            dims.pop_back();
        Tensor output = Tensor::empty(Shape(std::move(dims)), DType::Int32, input.device());
        if (rows == 0)
            return output;
        // few rows are cut into slices searched by separate blocks; the slice results need a workspace
        const std::int64_t ws_bytes = q3k_argmax_workspace_bytes(rows, search);
        Tensor workspace = Tensor::empty(Shape{(ws_bytes + 3) / 4}, DType::Int32, input.device());
        detail::launch_on(input.device(), [&](q3k_stream_t stream) {
            return q3k_argmax_bf16(detail::bf16_ptr(input), static_cast<int32_t *>(output.data()), rows, row_stride,
                                   search, ws_bytes > 0 ? workspace.data() : nullptr, ws_bytes, stream);
        });
        return output;
    }
} // namespace qwen3::ops
