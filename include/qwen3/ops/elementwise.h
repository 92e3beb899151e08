#pragma once

#include "qwen3/core/tensor.h"

namespace qwen3::ops
{
    // destination += source (BFloat16, same shape, same GPU), rounded to bf16.
    // Same signature and contract as the reference's include/qwen3/ops/elementwise.h:13.
    void add_inplace(Tensor &destination, const Tensor &source);

    // silu(gate) * up with silu(x) = x / (1 + exp(-x)); the silu result is
    // rounded to bf16 before the product.  Returns a new tensor.
    // Same signature and contract as the reference's include/qwen3/ops/elementwise.h:21.
    [[nodiscard]] Tensor silu_multiply(const Tensor &gate, const Tensor &up);

    // As above, into a caller-provided output (may be gate or up itself).
    void silu_multiply(const Tensor &gate, const Tensor &up, Tensor &output);
} // namespace qwen3::ops
