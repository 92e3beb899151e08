#include "qwen3/model/non_gemm_layer.h"

#include "qwen3/ops/elementwise.h"
#include "qwen3/ops/fused.h"
#include "qwen3/ops/rms_norm.h"
#include "qwen3/ops/rope.h"

#include <utility>

namespace qwen3
{
    NonGemmLayerOutputs qwen3_non_gemm_layer(const NonGemmLayerTensors &t, const NonGemmLayerWeights &w,
                                             const Tensor &rope_cache, std::int32_t num_query_heads,
                                             std::int32_t num_key_value_heads, std::int64_t start_position,
                                             float rms_norm_eps)
    {
        ops::qk_norm_rope_inplace(t.query, t.key, w.q_norm, w.k_norm, rms_norm_eps, rope_cache, num_query_heads,
                                  num_key_value_heads, start_position);
        Tensor mlp_input = ops::add_rms_norm(t.hidden, t.attention_delta, w.post_attention_layernorm, rms_norm_eps);
        Tensor activation = ops::silu_multiply(t.gate, t.up);
        Tensor next_input = ops::add_rms_norm(t.hidden, t.mlp_delta, w.next_norm, rms_norm_eps);
        return NonGemmLayerOutputs{std::move(mlp_input), std::move(activation), std::move(next_input)};
    }

    NonGemmLayerOutputs qwen3_non_gemm_layer_unfused(const NonGemmLayerTensors &t, const NonGemmLayerWeights &w,
                                                     const Tensor &rope_cache, std::int32_t num_query_heads,
                                                     std::int32_t num_key_value_heads, std::int64_t start_position,
                                                     float rms_norm_eps)
    {
        t.query = ops::rms_norm(t.query, w.q_norm, rms_norm_eps);
        t.key = ops::rms_norm(t.key, w.k_norm, rms_norm_eps);
        ops::apply_rope_inplace(t.query, t.key, rope_cache, num_query_heads, num_key_value_heads, start_position);
        ops::add_inplace(t.hidden, t.attention_delta);
        Tensor mlp_input = ops::rms_norm(t.hidden, w.post_attention_layernorm, rms_norm_eps);
        Tensor activation = ops::silu_multiply(t.gate, t.up);
        ops::add_inplace(t.hidden, t.mlp_delta);
        Tensor next_input = ops::rms_norm(t.hidden, w.next_norm, rms_norm_eps);
        return NonGemmLayerOutputs{std::move(mlp_input), std::move(activation), std::move(next_input)};
    }
} // namespace qwen3
