// qwen3::ops::rms_norm and the fused add_rms_norm over the gfx950 kernels.
// Validation follows src/ops/rms_norm.cu:129-215 of the reference (same
// checks, exception types and order).
#include "qwen3/ops/fused.h"
#include "qwen3/ops/rms_norm.h"

#include "ops_common.hpp"

#include <cmath>

namespace qwen3::ops
{
    namespace
    {
        void validate_rms_norm(const Tensor &input, const Tensor &weight, float epsilon)
        {
            detail::require(input.dtype() == DType::BFloat16, "RMSNorm input must have BFloat16 dtype");
            detail::require(weight.dtype() == DType::BFloat16, "RMSNorm weight must have BFloat16 dtype");
            detail::require(input.device().is_cuda() && weight.device().is_cuda(),
                            "RMSNorm currently requires GPU tensors");
            detail::require(input.device() == weight.device(), "RMSNorm input and weight must be on the same GPU");
            detail::require(input.shape().rank() != 0, "RMSNorm input cannot be scalar");
            detail::require(weight.shape().rank() == 1, "RMSNorm weight must be one-dimensional");
            const std::int64_t normalized = weight.shape()[0];
            detail::require(normalized > 0, "RMSNorm normalized size must be positive");
            const std::int64_t packed = input.shape()[input.shape().rank() - 1];
            detail::require(packed > 0, "RMSNorm input last dimension must be positive");
            detail::require(packed % normalized == 0, "RMSNorm input last dimension must be divisible by the weight size");
            detail::require(input.numel() % normalized == 0,
                            "RMSNorm input element count must be divisible by the weight size");
            detail::require(std::isfinite(epsilon) && epsilon > 0.0F, "RMSNorm epsilon must be finite and positive");
        }

        void validate_output(const Tensor &input, const Tensor &output)
        {
            detail::require(output.dtype() == DType::BFloat16 && output.device() == input.device(),
                            "RMSNorm output must be BFloat16 on the input's GPU");
            detail::require(output.shape() == input.shape(), "RMSNorm output must have the input's shape");
            detail::require(output.numel() == 0 || output.data() != input.data(),
                            "RMSNorm output cannot alias its input");
        }

        void run_rms(const Tensor &input, const Tensor &weight, float epsilon, Tensor &output)
        {
            const std::int64_t n = weight.shape()[0];
            const std::int64_t rows = input.numel() / n;
            if (rows == 0)
                return;
            detail::launch_on(input.device(), [&](q3k_stream_t stream) {
                return q3k_rms_norm_bf16(detail::bf16_ptr(input), detail::bf16_ptr(weight), detail::bf16_ptr(output),
                                         rows, n, epsilon, stream);
            });
        }

        void run_add_rms(Tensor &residual, const Tensor &delta, const Tensor &weight, float epsilon, Tensor &output)
        {
            validate_rms_norm(residual, weight, epsilon);
            detail::require(delta.dtype() == DType::BFloat16, "add_rms_norm delta must have BFloat16 dtype");
            detail::require(delta.device() == residual.device(), "add_rms_norm delta must be on the residual's GPU");
            detail::require(delta.shape() == residual.shape(), "add_rms_norm requires identical residual and delta shapes");
            validate_output(residual, output);
            detail::require(output.numel() == 0 || output.data() != delta.data(), "add_rms_norm output cannot alias delta");
            const std::int64_t n = weight.shape()[0];
            const std::int64_t rows = residual.numel() / n;
            if (rows == 0)
                return;
            detail::launch_on(residual.device(), [&](q3k_stream_t stream) {
                return q3k_add_rms_norm_bf16(detail::bf16_ptr(residual), detail::bf16_ptr(delta), detail::bf16_ptr(weight),
                                             detail::bf16_ptr(output), rows, n, epsilon, stream);
            });
        }
    } // namespace

    Tensor rms_norm(const Tensor &input, const Tensor &weight, float epsilon)
    {
        validate_rms_norm(input, weight, epsilon);
        Tensor output = Tensor::empty(input.shape(), input.dtype(), input.device());
        run_rms(input, weight, epsilon, output);
        return output;
    }

    void rms_norm(const Tensor &input, const Tensor &weight, float epsilon, Tensor &output)
    {
        validate_rms_norm(input, weight, epsilon);
        validate_output(input, output);
        run_rms(input, weight, epsilon, output);
    }

    Tensor add_rms_norm(Tensor &residual, const Tensor &delta, const Tensor &weight, float epsilon)
    {
        validate_rms_norm(residual, weight, epsilon);
        Tensor output = Tensor::empty(residual.shape(), residual.dtype(), residual.device());
        run_add_rms(residual, delta, weight, epsilon, output);
        return output;
    }

    void add_rms_norm(Tensor &residual, const Tensor &delta, const Tensor &weight, float epsilon, Tensor &output)
    {
        run_add_rms(residual, delta, weight, epsilon, output);
    }
} // namespace qwen3::ops
