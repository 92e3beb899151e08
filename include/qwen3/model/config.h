#pragma once

// The dense Qwen3 model's configuration (Hugging Face config.json): the
// sizes the non-GEMM ops take (hidden_size, intermediate_size, head counts,
// head_dim, rms_norm_eps, rope_theta) and the switches the runtime rejects.
// Same struct, defaults, accessors and loader contract as the reference's
// qwen3::ModelConfig (include/qwen3/model/config.h:8-58,
// src/model/config.cpp:145-371): the same required fields, checks in the
// same order, the same exception types and messages.  The JSON is read with
// this library's own parser; only the text after "cannot parse model config
// '<path>': " differs from the reference's (it names this parser's reason and
// byte offset).

#include <cstdint>
#include <filesystem>

namespace qwen3
{
    struct ModelConfig
    {
        std::int32_t vocab_size = 0;
        std::int32_t hidden_size = 0;
        std::int32_t intermediate_size = 0;
        std::int32_t num_hidden_layers = 0;

        std::int32_t num_attention_heads = 0;
        std::int32_t num_key_value_heads = 0;
        std::int32_t head_dim = 0;

        std::int32_t max_position_embeddings = 0;
        float rope_theta = 0.0F;

        float rms_norm_eps = 0.0F;

        std::int32_t bos_token_id = -1;
        std::int32_t eos_token_id = -1;

        bool attention_bias = false;
        bool tie_word_embeddings = false;
        bool use_sliding_window = false;

        // num_attention_heads * head_dim
        [[nodiscard]] std::int64_t q_projection_size() const noexcept;

        // num_key_value_heads * head_dim
        [[nodiscard]] std::int64_t kv_projection_size() const noexcept;

        // num_attention_heads / num_key_value_heads (0 when there are no KV heads)
        [[nodiscard]] std::int32_t query_heads_per_kv_head() const noexcept;

        // Throws std::invalid_argument for a configuration the runtime cannot run.
        void validate() const;
    };

    // Qwen3-0.6B's published values, validated.
    [[nodiscard]] ModelConfig make_qwen3_0_6b_config();

    // Reads and validates a config.json.  Missing or mistyped fields, an
    // unreadable file or malformed JSON: std::runtime_error; a model, dtype
    // or feature the runtime does not run: std::invalid_argument.
    [[nodiscard]] ModelConfig load_model_config(const std::filesystem::path &config_path);
} // namespace qwen3
