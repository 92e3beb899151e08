// Buffer contracts on the host (reference tests/unit/buffer_cpu_test.cpp).
#include "qwen3/core/buffer.h"
#include "qwen3/core/tensor_view.h"
#include "test_util.hpp"

#include <cstdint>
#include <cstring>
#include <type_traits>
#include <utility>

static_assert(!std::is_copy_constructible_v<qwen3::Buffer>);
static_assert(!std::is_copy_assignable_v<qwen3::Buffer>);
static_assert(std::is_nothrow_move_constructible_v<qwen3::Buffer>);
static_assert(std::is_nothrow_move_assignable_v<qwen3::Buffer>);
static_assert(std::is_nothrow_destructible_v<qwen3::Buffer>);

using test::require;
using test::require_throws;

static void body()
{
    qwen3::Buffer def;
    require(def.empty() && def.data() == nullptr && def.device().is_cpu(), "default buffer");
    qwen3::Buffer zero{0, qwen3::Device::cpu()};
    require(zero.empty() && zero.data() == nullptr, "zero-byte buffer");
    for (const std::size_t size : {1, 2, 63, 64, 65, 4097})
    {
        qwen3::Buffer b{size, qwen3::Device::cpu()};
        require(b.data() != nullptr && b.size_bytes() == size, "host allocation");
        require(reinterpret_cast<std::uintptr_t>(b.data()) % qwen3::Buffer::kCpuAlignment == 0, "64-byte alignment");
        std::memset(b.data(), 0x5A, size);
        const auto *bytes = static_cast<const unsigned char *>(b.data());
        for (std::size_t i = 0; i < size; ++i)
            require(bytes[i] == 0x5A, "host buffer read back");
    }
    qwen3::Buffer src{128, qwen3::Device::cpu()};
    void *p = src.data();
    qwen3::Buffer moved{std::move(src)};
    require(moved.data() == p && moved.size_bytes() == 128, "move construction keeps storage");
    require(src.data() == nullptr && src.size_bytes() == 0 && src.empty(), "moved-from buffer is empty");
    qwen3::Buffer a{32, qwen3::Device::cpu()}, b{64, qwen3::Device::cpu()};
    void *pb = b.data();
    a = std::move(b);
    require(a.data() == pb && a.size_bytes() == 64 && b.empty(), "move assignment");
    a = std::move(a);
    require(a.data() == pb && a.size_bytes() == 64, "self move assignment");

    qwen3::Buffer cs{16, qwen3::Device::cpu()}, cd{16, qwen3::Device::cpu()};
    for (int i = 0; i < 16; ++i)
        static_cast<unsigned char *>(cs.data())[i] = static_cast<unsigned char>(i);
    qwen3::copy_buffer(cd, cs);
    require(std::memcmp(cd.data(), cs.data(), 16) == 0, "host copy");
    qwen3::copy_buffer(cd, 4, cs, 8, 8);
    require(static_cast<unsigned char *>(cd.data())[4] == 8 && static_cast<unsigned char *>(cd.data())[11] == 15,
            "ranged host copy");
    require_throws<std::invalid_argument>([&] { qwen3::Buffer w{8, qwen3::Device::cpu()}; qwen3::copy_buffer(w, cs); },
                                          "size mismatch accepted");
    require_throws<std::out_of_range>([&] { qwen3::copy_buffer(cd, 12, cs, 0, 8); }, "out-of-range copy accepted");
    require_throws<std::out_of_range>([&] { qwen3::copy_buffer(cd, 0, cs, 9, 8); }, "out-of-range source accepted");

    qwen3::Buffer storage{24 * sizeof(float), qwen3::Device::cpu()};
    qwen3::TensorView view{storage.data(), qwen3::DType::Float32, storage.device(), qwen3::Shape{2, 3, 4}};
    require(view.nbytes() == storage.size_bytes(), "view over buffer");
}

int main() { return test::run("CPU Buffer test", body); }
