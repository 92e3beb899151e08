#pragma once

#include "qwen3/core/tensor.h"

namespace qwen3::ops
{
    // token_ids: Int32, GPU, any non-scalar shape [..].
    // embedding_weight: BFloat16, same GPU, [vocab_size, hidden_size].
    // Returns BFloat16 [.., hidden_size]; ids outside [0, vocab_size) give a zero row.
    // Same signature and contract as the reference's include/qwen3/ops/embedding.h:22.
    [[nodiscard]] Tensor embedding_lookup(const Tensor &token_ids, const Tensor &embedding_weight);

    // As above, into a caller-provided output of shape token_ids.shape + [hidden_size].
    void embedding_lookup(const Tensor &token_ids, const Tensor &embedding_weight, Tensor &output);
} // namespace qwen3::ops
