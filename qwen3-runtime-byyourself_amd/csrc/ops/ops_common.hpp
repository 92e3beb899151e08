// Shared plumbing of the qwen3::ops layer: C ABI status -> exception mapping
// and the launch wrapper that makes the tensor's device current, calls the
// kernel on the legacy default stream (as the reference's ops do) and
// restores the previous device, also on error.
#pragma once

#include "q3k_abi.h"
#include "qwen3/core/tensor.h"
#include "qwen3/hip/hip_check.h"

#include <cstdint>
#include <stdexcept>
#include <string>

namespace qwen3::ops::detail
{
    [[noreturn]] inline void throw_status(int status)
    {
        const std::string message = q3k_last_error_string();
        switch (status)
        {
        case Q3K_ERR_INVALID_ARGUMENT: throw std::invalid_argument(message);
        case Q3K_ERR_OUT_OF_RANGE: throw std::out_of_range(message);
        case Q3K_ERR_OVERFLOW: throw std::overflow_error(message);
        default: throw std::runtime_error(message);
        }
    }

    // Runs `launch` (returning a q3k_status) with `device` current.
    template <typename F>
    void launch_on(const Device &device, F &&launch)
    {
        hip::DeviceGuard guard(device.index());
        const int status = launch(static_cast<q3k_stream_t>(nullptr));
        guard.restore();
        if (status != Q3K_OK)
            throw_status(status);
    }

    inline uint16_t *bf16_ptr(Tensor &t) { return static_cast<uint16_t *>(t.data()); }
    inline const uint16_t *bf16_ptr(const Tensor &t) { return static_cast<const uint16_t *>(t.data()); }

    inline void require(bool condition, const char *message)
    {
        if (!condition)
            throw std::invalid_argument(message);
    }
} // namespace qwen3::ops::detail
