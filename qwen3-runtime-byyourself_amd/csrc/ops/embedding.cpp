// qwen3::ops::embedding_lookup over the gfx950 gather kernel.
// Validation follows src/ops/embedding.cu:57-82 of the reference (same
// checks, exception types and order), plus a BFloat16 check of the weight
// (the reference reads any weight as bf16).
#include "qwen3/ops/embedding.h"

#include "ops_common.hpp"

#include <utility>
#include <vector>

namespace qwen3::ops
{
    namespace
    {
        void validate(const Tensor &ids, const Tensor &weight)
        {
            detail::require(ids.dtype() == DType::Int32, "embedding token_ids must have Int32 dtype");
            detail::require(ids.device().is_cuda() && weight.device().is_cuda(),
                            "embedding currently requires GPU tensors");
            detail::require(ids.device() == weight.device(),
                            "embedding token_ids and weight must be on the same GPU");
            detail::require(ids.shape().rank() != 0, "embedding token_ids cannot be scalar");
            detail::require(weight.shape().rank() == 2, "embedding weight must have shape [vocab_size, hidden_size]");
            detail::require(weight.shape()[0] > 0 && weight.shape()[1] > 0,
                            "embedding weight dimensions must be positive");
            detail::require(weight.dtype() == DType::BFloat16, "embedding weight must have BFloat16 dtype");
        }

        Shape output_shape(const Tensor &ids, const Tensor &weight)
        {
            std::vector<Shape::Dimension> dims = ids.shape().dimensions();
            dims.push_back(weight.shape()[1]);
            return Shape(std::move(dims));
        }

        void run(const Tensor &ids, const Tensor &weight, Tensor &output)
        {
            const std::int64_t T = ids.numel();
            if (T == 0)
                return;
            detail::launch_on(ids.device(), [&](q3k_stream_t stream) {
                return q3k_embedding_bf16(static_cast<const int32_t *>(ids.data()), T, detail::bf16_ptr(weight),
                                          weight.shape()[0], weight.shape()[1], detail::bf16_ptr(output), stream);
            });
        }
    } // namespace

    Tensor embedding_lookup(const Tensor &token_ids, const Tensor &embedding_weight)
    {
        validate(token_ids, embedding_weight);
        Tensor output = Tensor::empty(output_shape(token_ids, embedding_weight), DType::BFloat16, token_ids.device());
        run(token_ids, embedding_weight, output);
        return output;
    }

    void embedding_lookup(const Tensor &token_ids, const Tensor &embedding_weight, Tensor &output)
    {
        validate(token_ids, embedding_weight);
        detail::require(output.dtype() == DType::BFloat16 && output.device() == token_ids.device(),
                        "embedding output must be BFloat16 on the ids' GPU");
        detail::require(output.shape() == output_shape(token_ids, embedding_weight),
                        "embedding output shape must be token_ids.shape + [hidden_size]");
        run(token_ids, embedding_weight, output);
    }
} // namespace qwen3::ops
