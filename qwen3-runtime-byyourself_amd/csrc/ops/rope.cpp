// qwen3::ops RoPE entry points and the fused Q/K norm + RoPE over the gfx950
// kernels.  Validation follows src/ops/rope.cu:88-211 of the reference (same
// checks, exception types and order); the table comes from the C ABI's host
// builder (the recipe of src/ops/rope.cu:250-303).
#include "qwen3/ops/fused.h"
#include "qwen3/ops/kv_append.h"
#include "qwen3/ops/rope.h"

#include "ops_common.hpp"

#include <cmath>
#include <limits>

namespace qwen3::ops
{
    namespace
    {
        std::int64_t checked_projection_size(std::int32_t num_heads, std::int64_t head_dim)
        {
            if (num_heads <= 0)
                throw std::invalid_argument("RoPE head count must be positive");
            if (head_dim > std::numeric_limits<std::int64_t>::max() / num_heads)
                throw std::overflow_error("RoPE projection size overflow");
            return static_cast<std::int64_t>(num_heads) * head_dim;
        }

        // Everything of src/ops/rope.cu:102-203 (all but the position range).
        void validate_rope_tensors(const Tensor &query, const Tensor &key, const Tensor &cache,
                                   std::int32_t num_query_heads, std::int32_t num_key_value_heads)
        {
            detail::require(query.dtype() == DType::BFloat16 && key.dtype() == DType::BFloat16,
                            "RoPE query and key must use bfloat16");
            detail::require(cache.dtype() == DType::Float32, "RoPE cache must use float32");
            detail::require(query.device().is_cuda() && key.device().is_cuda() && cache.device().is_cuda(),
                            "RoPE tensors must be on the GPU");
            detail::require(query.device() == key.device() && query.device() == cache.device(),
                            "RoPE tensors must be on the same GPU");
            detail::require(query.shape().rank() == 3 && key.shape().rank() == 3, "RoPE query and key must have rank 3");
            detail::require(cache.shape().rank() == 3 && cache.shape()[2] == 2,
                            "RoPE cache shape must be [max_positions, head_dim / 2, 2]");
            detail::require(query.shape()[0] == key.shape()[0] && query.shape()[1] == key.shape()[1],
                            "RoPE query and key batch/sequence dimensions must match");
            const std::int64_t half_dim = cache.shape()[1];
            detail::require(half_dim > 0 && half_dim <= std::numeric_limits<std::int64_t>::max() / 2,
                            "RoPE cache contains an invalid head dimension");
            const std::int64_t head_dim = half_dim * 2;
            const std::int64_t q_size = checked_projection_size(num_query_heads, head_dim);
            const std::int64_t k_size = checked_projection_size(num_key_value_heads, head_dim);
            detail::require(query.shape()[2] == q_size, "RoPE query projection size does not match num_query_heads * head_dim");
            detail::require(key.shape()[2] == k_size, "RoPE key projection size does not match num_key_value_heads * head_dim");
            detail::require(head_dim <= std::numeric_limits<std::int32_t>::max(), "RoPE head dimension is too large");
        }

        void validate_start(const Tensor &query, const Tensor &cache, std::int64_t start_position)
        {
            if (start_position < 0)
                throw std::invalid_argument("RoPE start_position cannot be negative");
            const std::int64_t sequence_length = query.shape()[1];
            const std::int64_t maximum_positions = cache.shape()[0];
            if (start_position > maximum_positions || sequence_length > maximum_positions - start_position)
                throw std::out_of_range("RoPE position range exceeds the cache");
        }

        void validate_positions(const Tensor &query, const Tensor &positions)
        {
            detail::require(positions.dtype() == DType::Int32, "RoPE positions must have Int32 dtype");
            detail::require(positions.device() == query.device(), "RoPE positions must be on the query's GPU");
            detail::require(positions.numel() == query.shape()[0] * query.shape()[1],
                            "RoPE positions must hold one entry per token (batch * sequence)");
        }

        void validate_norm_weights(const Tensor &query, const Tensor &cache, const Tensor &q_weight,
                                   const Tensor &k_weight, float epsilon)
        {
            const std::int64_t head_dim = cache.shape()[1] * 2;
            for (const Tensor *w : {&q_weight, &k_weight})
            {
                detail::require(w->dtype() == DType::BFloat16, "Q/K norm weights must have BFloat16 dtype");
                detail::require(w->device() == query.device(), "Q/K norm weights must be on the query's GPU");
                detail::require(w->shape().rank() == 1 && w->shape()[0] == head_dim,
                                "Q/K norm weights must have shape [head_dim]");
            }
            detail::require(std::isfinite(epsilon) && epsilon > 0.0F, "RMSNorm epsilon must be finite and positive");
        }

        void run_rope(Tensor &query, Tensor &key, const Tensor &cache, std::int32_t hq, std::int32_t hkv,
                      std::int64_t start, const int32_t *positions)
        {
            const std::int64_t B = query.shape()[0], S = query.shape()[1];
            const auto D = static_cast<std::int32_t>(cache.shape()[1] * 2);
            const auto *table = static_cast<const float *>(cache.data());
            const std::int64_t P = cache.shape()[0];
            // query and key in one launch (the reference makes one per tensor,
            // src/ops/rope.cu:326-332); the results are the same bits
            detail::launch_on(query.device(), [&](q3k_stream_t stream) {
                return q3k_rope_qk_bf16(detail::bf16_ptr(query), detail::bf16_ptr(key), B, S, hq, hkv, D, table, P,
                                        start, positions, stream);
            });
        }

        void run_qk_norm_rope(Tensor &query, Tensor &key, const Tensor &q_weight, const Tensor &k_weight, float epsilon,
                              const Tensor &cache, std::int32_t hq, std::int32_t hkv, std::int64_t start,
                              const int32_t *positions)
        {
            const std::int64_t B = query.shape()[0], S = query.shape()[1];
            const auto D = static_cast<std::int32_t>(cache.shape()[1] * 2);
            detail::launch_on(query.device(), [&](q3k_stream_t stream) {
                return q3k_qk_norm_rope_bf16(detail::bf16_ptr(query), detail::bf16_ptr(key), detail::bf16_ptr(q_weight),
                                             detail::bf16_ptr(k_weight), B, S, hq, hkv, D, epsilon,
                                             static_cast<const float *>(cache.data()), cache.shape()[0], start,
                                             positions, stream);
            });
        }
    } // namespace

    Tensor build_rope_cache(std::int64_t max_positions, std::int32_t head_dim, float rope_theta, Device device)
    {
        if (max_positions <= 0)
            throw std::invalid_argument("RoPE max_positions must be positive");
        if (head_dim <= 0 || head_dim % 2 != 0)
            throw std::invalid_argument("RoPE head_dim must be a positive even number");
        if (!std::isfinite(rope_theta) || rope_theta <= 0.0F)
            throw std::invalid_argument("RoPE theta must be finite and positive");
        Tensor host = Tensor::empty(Shape{max_positions, head_dim / 2, 2}, DType::Float32, Device::cpu());
        const int st = q3k_build_rope_cache_f32(static_cast<float *>(host.data()), max_positions, head_dim, rope_theta);
        if (st != Q3K_OK)
            detail::throw_status(st);
        if (device.is_cpu())
            return host;
        return host.copy_to(device);
    }

    void apply_rope_inplace(Tensor &query, Tensor &key, const Tensor &rope_cache, std::int32_t num_query_heads,
                            std::int32_t num_key_value_heads, std::int64_t start_position)
    {
        validate_rope_tensors(query, key, rope_cache, num_query_heads, num_key_value_heads);
        validate_start(query, rope_cache, start_position);
        run_rope(query, key, rope_cache, num_query_heads, num_key_value_heads, start_position, nullptr);
    }

    void apply_rope_inplace(Tensor &query, Tensor &key, const Tensor &rope_cache, std::int32_t num_query_heads,
                            std::int32_t num_key_value_heads, const Tensor &positions)
    {
        validate_rope_tensors(query, key, rope_cache, num_query_heads, num_key_value_heads);
        validate_positions(query, positions);
        run_rope(query, key, rope_cache, num_query_heads, num_key_value_heads, 0,
                 static_cast<const int32_t *>(positions.data()));
    }

    void qk_norm_rope_inplace(Tensor &query, Tensor &key, const Tensor &q_weight, const Tensor &k_weight,
                              float epsilon, const Tensor &rope_cache, std::int32_t num_query_heads,
                              std::int32_t num_key_value_heads, std::int64_t start_position)
    {
        validate_rope_tensors(query, key, rope_cache, num_query_heads, num_key_value_heads);
        validate_norm_weights(query, rope_cache, q_weight, k_weight, epsilon);
        validate_start(query, rope_cache, start_position);
        run_qk_norm_rope(query, key, q_weight, k_weight, epsilon, rope_cache, num_query_heads, num_key_value_heads,
                         start_position, nullptr);
    }

    void qk_norm_rope_inplace(Tensor &query, Tensor &key, const Tensor &q_weight, const Tensor &k_weight,
                              float epsilon, const Tensor &rope_cache, std::int32_t num_query_heads,
                              std::int32_t num_key_value_heads, const Tensor &positions)
    {
        validate_rope_tensors(query, key, rope_cache, num_query_heads, num_key_value_heads);
        validate_norm_weights(query, rope_cache, q_weight, k_weight, epsilon);
        validate_positions(query, positions);
        run_qk_norm_rope(query, key, q_weight, k_weight, epsilon, rope_cache, num_query_heads, num_key_value_heads, 0,
                         static_cast<const int32_t *>(positions.data()));
    }

    void qk_norm_rope_kv_append(Tensor &query, const Tensor &key, const Tensor &value, const Tensor &q_weight,
                                const Tensor &k_weight, float epsilon, const Tensor &rope_cache,
                                std::int32_t num_query_heads, std::int32_t num_key_value_heads,
                                std::int64_t start_position, KvCache &kv_cache, std::int32_t layer_index)
    {
        validate_rope_tensors(query, key, rope_cache, num_query_heads, num_key_value_heads);
        validate_norm_weights(query, rope_cache, q_weight, k_weight, epsilon);
        validate_start(query, rope_cache, start_position);
        detail::require(kv_cache.dtype() == DType::BFloat16, "fused KV append needs a BFloat16 cache");
        const KvCache::AppendTarget target = kv_cache.prepare_append(layer_index, start_position, key, value);
        const std::int64_t B = query.shape()[0], S = query.shape()[1];
        const auto D = static_cast<std::int32_t>(rope_cache.shape()[1] * 2);
        detail::require(D == kv_cache.head_dim() && num_key_value_heads == kv_cache.num_key_value_heads(),
                        "KV cache head layout does not match the key");
        detail::launch_on(query.device(), [&](q3k_stream_t stream) {
            return q3k_qk_norm_rope_kv_append_bf16(
                detail::bf16_ptr(query), detail::bf16_ptr(key), detail::bf16_ptr(value), detail::bf16_ptr(q_weight),
                detail::bf16_ptr(k_weight), B, S, num_query_heads, num_key_value_heads, D, epsilon,
                static_cast<const float *>(rope_cache.data()), rope_cache.shape()[0], start_position, nullptr,
                static_cast<uint16_t *>(target.key_layer), static_cast<uint16_t *>(target.value_layer),
                kv_cache.max_sequence_length(), start_position, stream);
        });
        kv_cache.commit_append(layer_index, start_position, target);
    }
} // namespace qwen3::ops
