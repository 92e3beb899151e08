// Buffer and Tensor on the GPU (reference tests/unit/buffer_cuda_test.cpp,
// tensor_cuda_test.cpp): device allocation, copies in every direction,
// moves, a failing allocation, and the current device left unchanged.
#include "gpu_util.hpp"

#include <cstdlib>
#include <string>
#include <utility>

using test::require;
using test::require_throws;

static void body()
{
    test::require_gpu();
    const int before = test::current_device();
    int count = 0;
    QWEN3_HIP_CHECK(hipGetDeviceCount(&count));

    const std::size_t n = 1000, bytes = n * sizeof(std::int32_t);
    qwen3::Buffer host_src{bytes, qwen3::Device::cpu()}, host_dst{bytes, qwen3::Device::cpu()};
    auto *s = static_cast<std::int32_t *>(host_src.data());
    for (std::size_t i = 0; i < n; ++i)
        s[i] = static_cast<std::int32_t>(i * 7 - 300);
    qwen3::Buffer gpu{bytes, qwen3::Device::cuda(0)};
    require(gpu.data() != nullptr && gpu.device().is_cuda() && gpu.size_bytes() == bytes, "GPU allocation");
    hipPointerAttribute_t attr{};
    QWEN3_HIP_CHECK(hipPointerGetAttributes(&attr, gpu.data()));
    require(attr.type == hipMemoryTypeDevice && attr.device == 0, "buffer owns device memory of GPU 0");
    qwen3::copy_buffer(gpu, host_src);
    qwen3::copy_buffer(host_dst, gpu);
    require(std::memcmp(host_src.data(), host_dst.data(), bytes) == 0, "host -> GPU -> host");
    qwen3::Buffer gpu2{bytes, qwen3::Device::cuda(0)};
    qwen3::copy_buffer(gpu2, gpu);
    qwen3::Buffer host3{bytes, qwen3::Device::cpu()};
    qwen3::copy_buffer(host3, gpu2);
    require(std::memcmp(host_src.data(), host3.data(), bytes) == 0, "GPU -> GPU");
    void *p = gpu2.data();
    qwen3::Buffer moved{std::move(gpu2)};
    require(moved.data() == p && gpu2.empty(), "GPU buffer move");
    require_throws<std::runtime_error>([&] { qwen3::Buffer bad{16, qwen3::Device::cuda(count)}; }, "invalid GPU accepted");
    static_cast<void>(hipGetLastError());
    require(test::current_device() == before, "failed allocation changed the current device");

    qwen3::Tensor t = qwen3::Tensor::empty(qwen3::Shape{8}, qwen3::DType::Int32, qwen3::Device::cpu());
    for (int i = 0; i < 8; ++i)
        static_cast<std::int32_t *>(t.data())[i] = i * 11 + 3;
    qwen3::Tensor g = t.copy_to(qwen3::Device::cuda(0));
    require(g.device() == qwen3::Device::cuda(0) && g.shape() == t.shape() && g.dtype() == t.dtype(), "Tensor copy_to GPU");
    qwen3::Tensor gc = g.clone();
    require(gc.data() != g.data() && gc.device().is_cuda(), "GPU clone is a new GPU tensor");
    const auto back = test::to_host<std::int32_t>(gc);
    for (int i = 0; i < 8; ++i)
        require(back[i] == i * 11 + 3, "GPU clone content");
    qwen3::Tensor g2 = qwen3::Tensor::empty(qwen3::Shape{8}, qwen3::DType::Int32, qwen3::Device::cuda(0));
    g2.copy_from(g);
    require(test::to_host<std::int32_t>(g2)[7] == 80, "GPU copy_from");
    require(test::current_device() == before, "tensor ops changed the current device");

    // the small-block cache: a block of a size class just freed is reused without hipMalloc; with
    // QWEN3_DEVICE_BLOCK_CACHE=0 every small Buffer calls hipMalloc (and its destruction hipFree)
    const char *env = std::getenv("QWEN3_DEVICE_BLOCK_CACHE");
    const bool cache_on = env == nullptr || std::string(env) != "0";
    {
        qwen3::Buffer warm{3000, qwen3::Device::cuda(0)};
    }
    const std::uint64_t n0 = qwen3::device_allocation_count();
    for (int i = 0; i < 4; ++i)
    {
        qwen3::Buffer small{2500 + static_cast<std::size_t>(i), qwen3::Device::cuda(0)};
        require(small.data() != nullptr, "small device buffer");
    }
    const std::uint64_t made = qwen3::device_allocation_count() - n0;
    require(cache_on ? made == 0 : made == 4,
            std::string("small-block cache ") + (cache_on ? "on" : "off") + ": " + std::to_string(made) +
                " hipMalloc calls for 4 buffers");
}

int main() { return test::run("GPU Buffer/Tensor test", body); }
