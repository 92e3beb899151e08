// DType / Device / Shape contracts (reference tests/unit/core_metadata_test.cpp).
#include "qwen3/core/device.h"
#include "qwen3/core/dtype.h"
#include "qwen3/core/shape.h"
#include "test_util.hpp"

#include <limits>

using test::require;
using test::require_throws;

static void body()
{
    require(qwen3::dtype_size(qwen3::DType::Float32) == 4, "float32 size");
    require(qwen3::dtype_size(qwen3::DType::BFloat16) == 2, "bfloat16 size");
    require(qwen3::dtype_size(qwen3::DType::Int32) == 4, "int32 size");
    require(qwen3::dtype_name(qwen3::DType::Int32) == "int32", "int32 name");
    require(qwen3::dtype_name(qwen3::DType::BFloat16) == "bfloat16", "bfloat16 name");

    const qwen3::Device cpu = qwen3::Device::cpu();
    const qwen3::Device gpu = qwen3::Device::cuda(0);
    require(cpu.is_cpu() && !cpu.is_cuda(), "cpu device");
    require(gpu.is_cuda() && gpu.index() == 0, "gpu device");
    require(gpu.to_string() == "cuda: 0", "gpu device name");
    require(cpu.to_string() == "cpu", "cpu device name");
    require(cpu != gpu && gpu == qwen3::Device::cuda(0) && gpu != qwen3::Device::cuda(1), "device equality");
    require_throws<std::invalid_argument>([] { (void)qwen3::Device::cuda(-1); }, "negative gpu index accepted");
    require_throws<std::invalid_argument>([] { (void)qwen3::Device(qwen3::DeviceType::Cpu, 1); }, "cpu index 1 accepted");

    const qwen3::Shape hidden{2, 8, 1024};
    require(hidden.rank() == 3 && hidden[2] == 1024 && hidden.numel() == 2 * 8 * 1024, "shape basics");
    require(hidden.to_string() == "[2, 8, 1024]", "shape to_string");
    require_throws<std::out_of_range>([&] { (void)hidden[3]; }, "shape axis out of range accepted");
    const qwen3::Shape scalar{};
    require(scalar.is_scalar() && scalar.numel() == 1 && scalar.rank() == 0, "scalar shape");
    const qwen3::Shape empty{2, 0, 4};
    require(empty.has_zero_dimension() && empty.numel() == 0, "empty shape");
    require_throws<std::invalid_argument>([] { (void)qwen3::Shape{2, -1, 4}; }, "negative dimension accepted");
    require_throws<std::overflow_error>(
        [] { (void)qwen3::Shape{std::numeric_limits<std::int64_t>::max(), 2}.numel(); }, "numel overflow not detected");
    const std::vector<qwen3::Shape::Dimension> dims{3, 5};
    require(qwen3::Shape(dims) == (qwen3::Shape{3, 5}) && qwen3::Shape(dims).dimensions() == dims, "shape from vector");
}

int main() { return test::run("core metadata test", body); }
