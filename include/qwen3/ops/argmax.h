#pragma once

// Argmax over the last dimension (the reference's include/qwen3/ops/argmax.h
// signature and contract).

#include "qwen3/core/tensor.h"

#include <cstdint>

namespace qwen3::ops
{
    // input BFloat16 [..., N] on the GPU -> Int32 indices [...] (or [..., 1]
    // with keep_dimension).  Only the first valid_reduction_size columns are
    // searched (0 = all N); NaN counts as -inf and ties go to the smaller
    // index.
    [[nodiscard]] Tensor argmax_last_dimension(const Tensor &input, bool keep_dimension = false,
                                               std::int64_t valid_reduction_size = 0);
} // namespace qwen3::ops
