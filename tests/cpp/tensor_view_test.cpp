// TensorView contracts (reference tests/unit/tensor_view_test.cpp).
#include "qwen3/core/tensor_view.h"
#include "test_util.hpp"

#include <cstddef>
#include <limits>

using test::require;
using test::require_throws;

static void body()
{
    float storage[24]{};
    qwen3::TensorView t{storage, qwen3::DType::Float32, qwen3::Device::cpu(), qwen3::Shape{2, 3, 4}};
    require(t.data() == storage && t.rank() == 3 && t.numel() == 24, "view basics");
    require(t.nbytes() == 24 * sizeof(float), "view nbytes");
    require(t.dim(0) == 2 && t.dim(1) == 3 && t.dim(2) == 4, "view dims");
    require(t.stride(0) == 12 && t.stride(1) == 4 && t.stride(2) == 1, "contiguous strides");
    require(t.is_contiguous(), "fresh view is contiguous");
    const auto tr = t.transpose(0, 2);
    require(tr.shape() == (qwen3::Shape{4, 3, 2}), "transposed shape");
    require(tr.stride(0) == 1 && tr.stride(1) == 4 && tr.stride(2) == 12, "transposed strides");
    require(tr.data() == storage && !tr.is_contiguous(), "transpose is a non-contiguous view of the same data");

    std::uint16_t half[8]{};
    qwen3::TensorView b{half, qwen3::DType::BFloat16, qwen3::Device::cpu(), qwen3::Shape{8}};
    require(b.nbytes() == 16, "bf16 nbytes");
    qwen3::TensorView e{nullptr, qwen3::DType::Float32, qwen3::Device::cpu(), qwen3::Shape{2, 0, 4}};
    require(e.is_empty() && e.numel() == 0 && e.nbytes() == 0, "empty view");

    require_throws<std::invalid_argument>(
        [] { qwen3::TensorView v{nullptr, qwen3::DType::Float32, qwen3::Device::cpu(), qwen3::Shape{1}}; (void)v; },
        "null data with elements accepted");
    require_throws<std::invalid_argument>(
        [&] { qwen3::TensorView v{storage, qwen3::DType::Float32, qwen3::Device::cpu(), qwen3::Shape{2, 3}, {3}}; (void)v; },
        "wrong stride rank accepted");
    require_throws<std::invalid_argument>(
        [&] { qwen3::TensorView v{storage, qwen3::DType::Float32, qwen3::Device::cpu(), qwen3::Shape{2, 3}, {3, -1}}; (void)v; },
        "negative stride accepted");
    require_throws<std::out_of_range>([&] { (void)t.stride(3); }, "stride axis out of range accepted");
    std::byte dummy{};
    qwen3::TensorView huge{&dummy, qwen3::DType::Float32, qwen3::Device::cpu(),
                           qwen3::Shape{std::numeric_limits<std::int64_t>::max()}};
    require_throws<std::overflow_error>([&] { (void)huge.nbytes(); }, "nbytes overflow not detected");
}

int main() { return test::run("TensorView test", body); }
