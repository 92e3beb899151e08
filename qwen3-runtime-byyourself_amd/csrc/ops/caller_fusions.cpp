// The fusions across the decoder-layer boundary: embedding gather + first
// input norm, and the final norm restricted to each sequence's last token.
// Argument checks keep the reference's messages where the unfused ops have
// them (src/ops/embedding.cu:57-82, src/ops/rms_norm.cu:129-215,
// src/model/lm_head.cpp:43-66).
#include "qwen3/ops/fused.h"

#include "ops_common.hpp"

#include <cmath>
#include <vector>

namespace qwen3::ops
{
    namespace
    {
        void validate_norm_weight(const Tensor &weight, const Tensor &input, std::int64_t hidden, float epsilon)
        {
            detail::require(weight.dtype() == DType::BFloat16, "RMSNorm weight must have BFloat16 dtype");
            detail::require(weight.device() == input.device(), "RMSNorm input and weight must be on the same GPU");
            detail::require(weight.shape().rank() == 1, "RMSNorm weight must be one-dimensional");
            detail::require(weight.shape()[0] == hidden, "RMSNorm weight size must equal the hidden size");
            detail::require(std::isfinite(epsilon) && epsilon > 0.0F, "RMSNorm epsilon must be finite and positive");
        }

        void validate_hidden_states(const Tensor &hidden_states)
        {
            detail::require(hidden_states.dtype() == DType::BFloat16, "LM Head hidden states must be BF16");
            detail::require(hidden_states.device().is_cuda(), "LM Head hidden states must be on CUDA");
            detail::require(hidden_states.shape().rank() == 3,
                            "LM Head hidden states must have shape [batch, sequence, hidden]");
            detail::require(hidden_states.shape()[0] > 0 && hidden_states.shape()[1] > 0 &&
                                hidden_states.shape()[2] > 0,
                            "LM Head hidden-state dimensions must be positive");
        }
    } // namespace

    EmbeddingNorm embedding_rms_norm(const Tensor &token_ids, const Tensor &embedding_weight, const Tensor &norm_weight,
                                     float epsilon)
    {
        detail::require(token_ids.dtype() == DType::Int32, "embedding token_ids must have Int32 dtype");
        detail::require(token_ids.device().is_cuda() && embedding_weight.device().is_cuda(),
                        "embedding currently requires GPU tensors");
        detail::require(token_ids.device() == embedding_weight.device(),
                        "embedding token_ids and weight must be on the same GPU");
        detail::require(token_ids.shape().rank() != 0, "embedding token_ids cannot be scalar");
        detail::require(embedding_weight.shape().rank() == 2,
                        "embedding weight must have shape [vocab_size, hidden_size]");
        detail::require(embedding_weight.shape()[0] > 0 && embedding_weight.shape()[1] > 0,
                        "embedding weight dimensions must be positive");
        detail::require(embedding_weight.dtype() == DType::BFloat16, "embedding weight must have BFloat16 dtype");
        const std::int64_t vocab = embedding_weight.shape()[0];
        const std::int64_t hidden = embedding_weight.shape()[1];
        validate_norm_weight(norm_weight, token_ids, hidden, epsilon);

        std::vector<Shape::Dimension> dims = token_ids.shape().dimensions();
        dims.push_back(hidden);
        const Shape shape(std::move(dims));
        EmbeddingNorm out{Tensor::empty(shape, DType::BFloat16, token_ids.device()),
                          Tensor::empty(shape, DType::BFloat16, token_ids.device())};
        const std::int64_t tokens = token_ids.numel();
        if (tokens == 0)
            return out;
        detail::launch_on(token_ids.device(), [&](q3k_stream_t stream) {
            return q3k_embedding_rms_norm_bf16(static_cast<const int32_t *>(token_ids.data()), tokens,
                                               detail::bf16_ptr(embedding_weight), vocab, hidden,
                                               detail::bf16_ptr(norm_weight), epsilon, detail::bf16_ptr(out.hidden),
                                               detail::bf16_ptr(out.normalized), stream);
        });
        return out;
    }

    Tensor rms_norm_last_token(const Tensor &hidden_states, const Tensor &weight, float epsilon)
    {
        validate_hidden_states(hidden_states);
        const std::int64_t batch = hidden_states.shape()[0];
        const std::int64_t sequence = hidden_states.shape()[1];
        const std::int64_t hidden = hidden_states.shape()[2];
        validate_norm_weight(weight, hidden_states, hidden, epsilon);
        Tensor output = Tensor::empty(Shape{batch, hidden}, DType::BFloat16, hidden_states.device());
        detail::launch_on(hidden_states.device(), [&](q3k_stream_t stream) {
            return q3k_rms_norm_rows_bf16(detail::bf16_ptr(hidden_states), detail::bf16_ptr(weight),
                                          detail::bf16_ptr(output), batch, sequence - 1, sequence, hidden, epsilon,
                                          stream);
        });
        return output;
    }

    Tensor add_rms_norm_last_token(Tensor &residual, const Tensor &delta, const Tensor &weight, float epsilon)
    {
        validate_hidden_states(residual);
        detail::require(delta.dtype() == DType::BFloat16, "add_rms_norm delta must have BFloat16 dtype");
        detail::require(delta.device() == residual.device(), "add_rms_norm delta must be on the residual's GPU");
        detail::require(delta.shape() == residual.shape(), "add_rms_norm requires identical residual and delta shapes");
        const std::int64_t batch = residual.shape()[0];
        const std::int64_t sequence = residual.shape()[1];
        const std::int64_t hidden = residual.shape()[2];
        validate_norm_weight(weight, residual, hidden, epsilon);
        Tensor output = Tensor::empty(Shape{batch, hidden}, DType::BFloat16, residual.device());
        detail::launch_on(residual.device(), [&](q3k_stream_t stream) {
            return q3k_add_rms_norm_rows_bf16(detail::bf16_ptr(residual), detail::bf16_ptr(delta),
                                              detail::bf16_ptr(weight), detail::bf16_ptr(output), batch, sequence - 1,
                                              sequence, hidden, epsilon, stream);
        });
        return output;
    }
} // namespace qwen3::ops
