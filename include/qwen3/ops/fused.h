#pragma once

// Fused forms of the decoder layer's non-GEMM op pairs.  Each produces the
// same values as the unfused ops called in the reference's order, with one
// pass over memory instead of two.

#include "qwen3/core/tensor.h"

#include <cstdint>

namespace qwen3::ops
{
    // residual += delta (bf16), then RMSNorm of the updated residual:
    // add_inplace(residual, delta); return rms_norm(residual, weight, eps)
    // (decoder_layer.cpp:78 -> :88, and :94 -> the next layer's :72 or the
    // final norm at model.cpp:146).
    [[nodiscard]] Tensor add_rms_norm(Tensor &residual, const Tensor &delta, const Tensor &weight, float epsilon);

    // As above, into a caller-provided output shaped like residual.
    void add_rms_norm(Tensor &residual, const Tensor &delta, const Tensor &weight, float epsilon, Tensor &output);

    // Per-head RMSNorm of query and key (weights [head_dim]) followed by RoPE,
    // in place: query = rope(rms_norm(query, q_weight)), likewise key
    // (self_attention.cpp:147-152).
    void qk_norm_rope_inplace(Tensor &query, Tensor &key, const Tensor &q_weight, const Tensor &k_weight,
                              float epsilon, const Tensor &rope_cache, std::int32_t num_query_heads,
                              std::int32_t num_key_value_heads, std::int64_t start_position);

    // As above with one Int32 position per token (see apply_rope_inplace).
    void qk_norm_rope_inplace(Tensor &query, Tensor &key, const Tensor &q_weight, const Tensor &k_weight,
                              float epsilon, const Tensor &rope_cache, std::int32_t num_query_heads,
                              std::int32_t num_key_value_heads, const Tensor &positions);
} // namespace qwen3::ops
