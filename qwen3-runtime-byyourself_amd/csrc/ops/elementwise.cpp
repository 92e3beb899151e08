// qwen3::ops::add_inplace / silu_multiply over the gfx950 kernels.
// Validation follows src/ops/elementwise.cu:69-98 of the reference.
#include "qwen3/ops/elementwise.h"

#include "ops_common.hpp"

#include <string>

namespace qwen3::ops
{
    namespace
    {
        void validate_binary(const Tensor &lhs, const Tensor &rhs, const char *operation)
        {
            const std::string op(operation);
            if (lhs.dtype() != DType::BFloat16 || rhs.dtype() != DType::BFloat16)
                throw std::invalid_argument(op + " requires BFloat16 tensors");
            if (!lhs.device().is_cuda() || !rhs.device().is_cuda())
                throw std::invalid_argument(op + " currently requires GPU tensors");
            if (lhs.device() != rhs.device())
                throw std::invalid_argument(op + " requires tensors on the same device");
            if (lhs.shape() != rhs.shape())
                throw std::invalid_argument(op + " requires identical tensor shapes");
        }

        void run_silu(const Tensor &gate, const Tensor &up, Tensor &output)
        {
            const std::int64_t n = gate.numel();
            if (n == 0)
                return;
            detail::launch_on(gate.device(), [&](q3k_stream_t stream) {
                return q3k_silu_mul_bf16(detail::bf16_ptr(gate), detail::bf16_ptr(up), detail::bf16_ptr(output), n,
                                         stream);
            });
        }
    } // namespace

    void add_inplace(Tensor &destination, const Tensor &source)
    {
        validate_binary(destination, source, "add_inplace");
        const std::int64_t n = destination.numel();
        if (n == 0)
            return;
        detail::launch_on(destination.device(), [&](q3k_stream_t stream) {
            return q3k_add_inplace_bf16(detail::bf16_ptr(destination), detail::bf16_ptr(source), n, stream);
        });
    }

    Tensor silu_multiply(const Tensor &gate, const Tensor &up)
    {
        validate_binary(gate, up, "silu_multiply");
        Tensor output = Tensor::empty(gate.shape(), gate.dtype(), gate.device());
        run_silu(gate, up, output);
        return output;
    }

    void silu_multiply(const Tensor &gate, const Tensor &up, Tensor &output)
    {
        validate_binary(gate, up, "silu_multiply");
        validate_binary(gate, output, "silu_multiply");
        run_silu(gate, up, output);
    }
} // namespace qwen3::ops
