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

    // Embedding gather followed by the first layer's input norm:
    // hidden = embedding_lookup(token_ids, embedding_weight);
    // normalized = rms_norm(hidden, norm_weight, epsilon)
    // (model.cpp:118 -> decoder_layer.cpp:72).  The gathered rows are written
    // once and normalised from registers; out-of-range ids give zero rows.
    struct EmbeddingNorm
    {
        Tensor hidden;
        Tensor normalized;
    };
    [[nodiscard]] EmbeddingNorm embedding_rms_norm(const Tensor &token_ids, const Tensor &embedding_weight,
                                                   const Tensor &norm_weight, float epsilon);

    // The final norm of the last token of every sequence only:
    // select_last_token_hidden(rms_norm(hidden_states, weight, epsilon)),
    // hidden_states [B, S, H] -> [B, H] (model.cpp:146 and
    // lm_head.cpp:123-181).  The norm is row-wise, so this equals the
    // reference's full-sequence norm followed by the row copy, bit for bit.
    [[nodiscard]] Tensor rms_norm_last_token(const Tensor &hidden_states, const Tensor &weight, float epsilon);

    // The last layer's MLP residual add carried into that norm: the last row
    // of each sequence of residual gets += delta, and those rows are
    // normalised into [B, H] (decoder_layer.cpp:94 -> model.cpp:146 ->
    // lm_head.cpp:123).  Rows before the last are left as they were: nothing
    // downstream of the final norm reads them.
    [[nodiscard]] Tensor add_rms_norm_last_token(Tensor &residual, const Tensor &delta, const Tensor &weight,
                                                 float epsilon);
} // namespace qwen3::ops
