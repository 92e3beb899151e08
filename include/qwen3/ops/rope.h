#pragma once

#include "qwen3/core/tensor.h"

#include <cstdint>

namespace qwen3::ops
{
    // Float32 table [max_positions, head_dim / 2, 2]: cache[p, i] = (cos, sin)
    // of p * theta^(-2i / head_dim), computed on the host in double.
    // Same signature and result as the reference's include/qwen3/ops/rope.h:16.
    [[nodiscard]] Tensor build_rope_cache(std::int64_t max_positions, std::int32_t head_dim, float rope_theta,
                                          Device device);

    // Rotates query [B, S, Hq * D] and key [B, S, Hkv * D] in place (half-split
    // pairs), token (b, s) at position start_position + s.
    // Same signature and contract as the reference's include/qwen3/ops/rope.h:29.
    void apply_rope_inplace(Tensor &query, Tensor &key, const Tensor &rope_cache, std::int32_t num_query_heads,
                            std::int32_t num_key_value_heads, std::int64_t start_position);

    // As above with one position per token: positions is Int32 [B, S] (or
    // [B * S]) on the same GPU.  A head whose position lies outside the table
    // is set to NaN (positions are not read back to the host).
    void apply_rope_inplace(Tensor &query, Tensor &key, const Tensor &rope_cache, std::int32_t num_query_heads,
                            std::int32_t num_key_value_heads, const Tensor &positions);
} // namespace qwen3::ops
