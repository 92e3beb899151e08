// qwen3::ops::grouped_query_attention over the gfx950 attention kernels.
// Checks, their order and exception types follow
// src/ops/gqa_attention.cu:157-302 of the reference.
#include "qwen3/ops/gqa_attention.h"

#include "ops_common.hpp"

#include <limits>

namespace qwen3::ops
{
    namespace
    {
        void validate(const Tensor &query, const TensorView &key_cache, const TensorView &value_cache,
                      std::int32_t num_query_heads, std::int64_t start_position)
        {
            detail::require(query.dtype() == DType::BFloat16 && key_cache.dtype() == DType::BFloat16 &&
                                value_cache.dtype() == DType::BFloat16,
                            "GQA currently requires bfloat16 tensors");
            detail::require(query.device().is_cuda() && key_cache.device().is_cuda() && value_cache.device().is_cuda(),
                            "GQA tensors must be on CUDA");
            detail::require(query.device() == key_cache.device() && query.device() == value_cache.device(),
                            "GQA tensors must be on the same CUDA device");
            detail::require(query.shape().rank() == 3, "GQA query must have rank 3");
            detail::require(key_cache.shape().rank() == 4 && value_cache.shape().rank() == 4,
                            "GQA cache views must have rank 4");
            detail::require(key_cache.shape() == value_cache.shape(), "GQA key/value cache shapes must match");
            const std::int64_t batch = query.shape()[0];
            const std::int64_t sequence = query.shape()[1];
            const std::int64_t cached = key_cache.shape()[1];
            const std::int64_t kv_heads = key_cache.shape()[2];
            const std::int64_t head_dim = key_cache.shape()[3];
            detail::require(batch > 0 && sequence > 0, "GQA batch and sequence dimensions must be positive");
            detail::require(batch == key_cache.shape()[0], "GQA query/cache batch sizes must match");
            detail::require(num_query_heads > 0 && kv_heads > 0, "GQA head counts must be positive");
            detail::require(num_query_heads % kv_heads == 0, "GQA query heads must be divisible by key/value heads");
            detail::require(head_dim > 0 && head_dim <= 256, "GQA head_dim must be between 1 and 256");
            detail::require(query.shape()[2] == static_cast<std::int64_t>(num_query_heads) * head_dim,
                            "GQA query projection size is incorrect");
            detail::require(start_position >= 0, "GQA start_position cannot be negative");
            detail::require(start_position <= cached && sequence == cached - start_position,
                            "GQA cache length must equal start_position + sequence_length");
            if (batch * sequence * num_query_heads > std::numeric_limits<int>::max())
                throw std::overflow_error("GQA grid is too large");
        }

        void run(const Tensor &query, const TensorView &key_cache, const TensorView &value_cache,
                 std::int32_t num_query_heads, std::int64_t start_position, Tensor &output)
        {
            const std::int64_t ks[4] = {key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
                                        key_cache.stride(3)};
            const std::int64_t vs[4] = {value_cache.stride(0), value_cache.stride(1), value_cache.stride(2),
                                        value_cache.stride(3)};
            const std::int64_t B = query.shape()[0], S = query.shape()[1];
            const auto Hkv = static_cast<std::int32_t>(key_cache.shape()[2]);
            const auto D = static_cast<std::int32_t>(key_cache.shape()[3]);
            // a launch too small for the GPU splits the key range; its slices need a workspace
            const std::int64_t ws_bytes =
                q3k_gqa_attention_workspace_bytes(B, S, num_query_heads, Hkv, D, key_cache.shape()[1]);
            Tensor workspace = Tensor::empty(Shape{(ws_bytes + 3) / 4}, DType::Float32, query.device());
            detail::launch_on(query.device(), [&](q3k_stream_t stream) {
                return q3k_gqa_attention_bf16(
                    detail::bf16_ptr(query), static_cast<const uint16_t *>(key_cache.data()),
                    static_cast<const uint16_t *>(value_cache.data()), detail::bf16_ptr(output), B, S,
                    num_query_heads, Hkv, D, key_cache.shape()[1], start_position, ks, vs,
                    ws_bytes > 0 ? workspace.data() : nullptr, ws_bytes, stream);
            });
        }
    } // namespace

    Tensor grouped_query_attention(const Tensor &query, const TensorView &key_cache, const TensorView &value_cache,
                                   std::int32_t num_query_heads, std::int64_t start_position)
    {
        validate(query, key_cache, value_cache, num_query_heads, start_position);
        Tensor output = Tensor::empty(query.shape(), DType::BFloat16, query.device());
        run(query, key_cache, value_cache, num_query_heads, start_position, output);
        return output;
    }

    void grouped_query_attention(const Tensor &query, const TensorView &key_cache, const TensorView &value_cache,
                                 std::int32_t num_query_heads, std::int64_t start_position, Tensor &output)
    {
        validate(query, key_cache, value_cache, num_query_heads, start_position);
        detail::require(output.dtype() == DType::BFloat16 && output.device() == query.device() &&
                            output.shape() == query.shape(),
                        "GQA output must be BFloat16 on the query's GPU with the query's shape");
        detail::require(output.data() != query.data(), "GQA output cannot alias the query");
        run(query, key_cache, value_cache, num_query_heads, start_position, output);
    }
} // namespace qwen3::ops
