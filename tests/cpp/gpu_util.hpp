// GPU-side helpers of the C++ tests.
#pragma once

#include "qwen3/core/tensor.h"
#include "qwen3/hip/hip_check.h"
#include "test_util.hpp"

#include <cstring>
#include <vector>

namespace test
{
    template <typename T>
    qwen3::Tensor to_gpu(const std::vector<T> &values, qwen3::Shape shape, qwen3::DType dtype)
    {
        qwen3::Tensor host = qwen3::Tensor::empty(std::move(shape), dtype, qwen3::Device::cpu());
        require(host.nbytes() == values.size() * sizeof(T), "test input size mismatch");
        if (!values.empty())
            std::memcpy(host.data(), values.data(), host.nbytes());
        return host.copy_to(qwen3::Device::cuda(0));
    }

    template <typename T>
    std::vector<T> to_host(const qwen3::Tensor &t)
    {
        qwen3::Tensor host = t.copy_to(qwen3::Device::cpu());
        std::vector<T> out(host.nbytes() / sizeof(T));
        if (!out.empty())
            std::memcpy(out.data(), host.data(), host.nbytes());
        return out;
    }

    inline int current_device()
    {
        int d = -1;
        QWEN3_HIP_CHECK(hipGetDevice(&d));
        return d;
    }

    inline void require_gpu()
    {
        int n = 0;
        QWEN3_HIP_CHECK(hipGetDeviceCount(&n));
        require(n > 0, "no visible GPU");
    }
} // namespace test
