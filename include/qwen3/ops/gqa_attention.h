#pragma once

// Causal grouped-query attention over KV-cache views (the reference's
// include/qwen3/ops/gqa_attention.h signature and contract).

#include "qwen3/core/tensor.h"
#include "qwen3/core/tensor_view.h"

#include <cstdint>

namespace qwen3::ops
{
    // query [batch, sequence, num_query_heads * head_dim] (BFloat16);
    // key_cache / value_cache [batch, cached_length, num_key_value_heads,
    // head_dim] views (any strides, e.g. KvCache::key_view); cached_length
    // must equal start_position + sequence.  Query position s attends to
    // keys 0 .. start_position + s.  Returns [batch, sequence,
    // num_query_heads * head_dim] (BFloat16).
    [[nodiscard]] Tensor grouped_query_attention(const Tensor &query, const TensorView &key_cache,
                                                 const TensorView &value_cache, std::int32_t num_query_heads,
                                                 std::int64_t start_position);

    // As above, into a caller-provided output shaped like query.
    void grouped_query_attention(const Tensor &query, const TensorView &key_cache, const TensorView &value_cache,
                                 std::int32_t num_query_heads, std::int64_t start_position, Tensor &output);
} // namespace qwen3::ops
