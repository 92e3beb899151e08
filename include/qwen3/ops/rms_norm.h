#pragma once

#include "qwen3/core/tensor.h"

namespace qwen3::ops
{
    // RMSNorm over consecutive chunks of weight.size() elements (the last
    // dimension, or packed heads of it: Q [B, S, Hq * D] with a [D] weight).
    // input and weight: BFloat16 on the same GPU; epsilon finite and > 0.
    // Returns a new tensor shaped like input.
    // Same signature and contract as the reference's include/qwen3/ops/rms_norm.h:22.
    [[nodiscard]] Tensor rms_norm(const Tensor &input, const Tensor &weight, float epsilon);

    // As above, into a caller-provided output shaped like input (not aliasing it).
    void rms_norm(const Tensor &input, const Tensor &weight, float epsilon, Tensor &output);
} // namespace qwen3::ops
