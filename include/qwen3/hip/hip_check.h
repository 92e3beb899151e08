#pragma once

// HIP status -> exception, the runtime's error convention (the reference's
// QWEN3_CUDA_CHECK, src/cuda/cuda_check.cpp:8-22): throws std::runtime_error
// naming the failed expression, the HIP error and the location.

#include <hip/hip_runtime_api.h>

namespace qwen3::hip
{
    void check(hipError_t status, const char *expression, const char *file, int line);

    // Makes `device` current for the lifetime of the guard and restores the
    // previous device afterwards (also when an exception leaves the scope).
    class DeviceGuard
    {
    public:
        explicit DeviceGuard(int device);
        ~DeviceGuard();
        DeviceGuard(const DeviceGuard &) = delete;
        DeviceGuard &operator=(const DeviceGuard &) = delete;

        // Restores the previous device now; throws std::runtime_error on failure.
        void restore();

    private:
        int previous_;
        bool changed_;
    };
} // namespace qwen3::hip

#define QWEN3_HIP_CHECK(expression) ::qwen3::hip::check((expression), #expression, __FILE__, __LINE__)
