// Tensor contracts on the host (reference tests/unit/tensor_cpu_test.cpp).
#include "qwen3/core/tensor.h"
#include "test_util.hpp"

#include <cstring>
#include <limits>
#include <type_traits>
#include <utility>

static_assert(!std::is_default_constructible_v<qwen3::Tensor>);
static_assert(!std::is_copy_constructible_v<qwen3::Tensor>);
static_assert(!std::is_copy_assignable_v<qwen3::Tensor>);
static_assert(std::is_nothrow_move_constructible_v<qwen3::Tensor>);
static_assert(std::is_nothrow_move_assignable_v<qwen3::Tensor>);

using test::require;
using test::require_throws;

static void body()
{
    using qwen3::DType;
    using qwen3::Shape;
    using qwen3::Tensor;
    const auto cpu = qwen3::Device::cpu();
    Tensor t = Tensor::empty(Shape{2, 3, 4}, DType::Float32, cpu);
    require(t.data() != nullptr && t.device().is_cpu() && t.dtype() == DType::Float32, "empty() basics");
    require(t.shape() == (Shape{2, 3, 4}) && t.numel() == 24 && t.nbytes() == 24 * sizeof(float), "size");
    const auto v = t.view();
    require(v.data() == t.data() && v.shape() == t.shape() && v.dtype() == t.dtype() && v.device() == t.device() &&
                v.is_contiguous(),
            "view of a tensor");
    const auto tr = v.transpose(0, 2);
    require(tr.data() == t.data() && tr.shape() == (Shape{4, 3, 2}) && !tr.is_contiguous(), "transposed view");
    require(t.shape() == (Shape{2, 3, 4}), "transpose does not change the tensor");

    require(Tensor::empty(Shape{8}, DType::BFloat16, cpu).nbytes() == 16, "bf16 bytes");
    Tensor scalar = Tensor::empty(Shape{}, DType::Float32, cpu);
    require(scalar.numel() == 1 && scalar.nbytes() == 4 && scalar.data() != nullptr, "scalar tensor");
    Tensor empty = Tensor::empty(Shape{2, 0, 4}, DType::Float32, cpu);
    require(empty.is_empty() && empty.numel() == 0 && empty.nbytes() == 0 && empty.data() == nullptr, "empty tensor");

    Tensor src = Tensor::empty(Shape{8}, DType::Float32, cpu);
    auto *s = static_cast<float *>(src.data());
    for (int i = 0; i < 8; ++i)
        s[i] = static_cast<float>(i) + 0.5f;
    Tensor c = src.clone();
    require(c.data() != src.data() && std::memcmp(c.data(), src.data(), src.nbytes()) == 0, "clone copies");
    s[0] = 999.0f;
    require(static_cast<const float *>(c.data())[0] == 0.5f, "clone is independent");
    Tensor dst = Tensor::empty(Shape{8}, DType::Float32, cpu);
    dst.copy_from(src);
    require(static_cast<const float *>(dst.data())[0] == 999.0f, "copy_from");
    Tensor wrong_shape = Tensor::empty(Shape{4}, DType::Float32, cpu);
    require_throws<std::invalid_argument>([&] { wrong_shape.copy_from(src); }, "copy_from shape mismatch accepted");
    Tensor wrong_dtype = Tensor::empty(Shape{8}, DType::Int32, cpu);
    require_throws<std::invalid_argument>([&] { wrong_dtype.copy_from(src); }, "copy_from dtype mismatch accepted");
    require_throws<std::overflow_error>(
        [&] { (void)Tensor::empty(Shape{std::numeric_limits<std::int64_t>::max()}, DType::Float32, cpu); },
        "byte-size overflow accepted");
    Tensor host2 = src.copy_to(cpu);
    require(host2.data() != src.data() && std::memcmp(host2.data(), src.data(), 32) == 0, "copy_to host");

    void *p = t.data();
    Tensor moved{std::move(t)};
    require(moved.data() == p, "move keeps storage");
    moved = std::move(moved);
    require(moved.data() == p, "self move keeps storage");
}

int main() { return test::run("CPU Tensor test", body); }
