#pragma once

// The non-GEMM work of one Qwen3 decoder layer, in the order of the
// reference's qwen3_decoder_layer (src/model/decoder_layer.cpp:63-98),
// qwen3_self_attention (src/model/self_attention.cpp:147-152) and qwen3_mlp
// (src/model/mlp.cpp:111).  The projections and attention stay with the
// caller, whose outputs come in through NonGemmLayerTensors.
//
// Fused order (one pass per pair):
//   qk_norm_rope_inplace(query, key)                 q/k norm + RoPE
//   mlp_input  = add_rms_norm(hidden, attention_delta, post_attention_layernorm)
//   activation = silu_multiply(gate, up)
//   next_input = add_rms_norm(hidden, mlp_delta, next_norm)
// where next_norm is the next layer's input_layernorm (or the final norm,
// src/model/model.cpp:146, after the last layer), so the MLP residual add is
// fused with the norm that follows it.

#include "qwen3/core/tensor.h"

#include <cstdint>

namespace qwen3
{
    struct NonGemmLayerWeights
    {
        const Tensor &q_norm;                   // [head_dim]
        const Tensor &k_norm;                   // [head_dim]
        const Tensor &post_attention_layernorm; // [hidden]
        const Tensor &next_norm;                // [hidden]: next layer's input_layernorm or the final norm
    };

    struct NonGemmLayerTensors
    {
        Tensor &hidden;                // [B, S, hidden] residual stream, updated in place
        Tensor &query;                 // [B, S, Hq * head_dim] q_proj output, normalised + rotated in place
        Tensor &key;                   // [B, S, Hkv * head_dim] k_proj output, normalised + rotated in place
        const Tensor &attention_delta; // [B, S, hidden] o_proj output
        const Tensor &gate;            // [B, S, intermediate] gate_proj output
        const Tensor &up;              // [B, S, intermediate] up_proj output
        const Tensor &mlp_delta;       // [B, S, hidden] down_proj output
    };

    struct NonGemmLayerOutputs
    {
        Tensor mlp_input;  // rms_norm(hidden + attention_delta, post_attention_layernorm)
        Tensor activation; // silu(gate) * up
        Tensor next_input; // rms_norm(hidden + attention_delta + mlp_delta, next_norm)
    };

    // The fused chain (four launches).
    [[nodiscard]] NonGemmLayerOutputs qwen3_non_gemm_layer(const NonGemmLayerTensors &tensors,
                                                           const NonGemmLayerWeights &weights, const Tensor &rope_cache,
                                                           std::int32_t num_query_heads, std::int32_t num_key_value_heads,
                                                           std::int64_t start_position, float rms_norm_eps);

    // The same work through the reference's unfused ops, in its order
    // (rms_norm q, rms_norm k, apply_rope_inplace, add_inplace, rms_norm,
    // silu_multiply, add_inplace, rms_norm).  Results equal the fused chain's.
    [[nodiscard]] NonGemmLayerOutputs qwen3_non_gemm_layer_unfused(const NonGemmLayerTensors &tensors,
                                                                   const NonGemmLayerWeights &weights,
                                                                   const Tensor &rope_cache, std::int32_t num_query_heads,
                                                                   std::int32_t num_key_value_heads,
                                                                   std::int64_t start_position, float rms_norm_eps);
} // namespace qwen3
