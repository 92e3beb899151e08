// Argument checks of the qwen3::ops layer that need no GPU: every op rejects
// host tensors and wrong dtypes with std::invalid_argument before touching a
// device (reference src/ops/*: validate_* functions), and build_rope_cache
// runs on the host.
#include "qwen3/core/tensor.h"
#include "qwen3/model/kv_cache.h"
#include "qwen3/ops/elementwise.h"
#include "qwen3/ops/embedding.h"
#include "qwen3/ops/fused.h"
#include "qwen3/ops/rms_norm.h"
#include "qwen3/ops/rope.h"
#include "test_util.hpp"

#include <cmath>
#include <limits>

using qwen3::DType;
using qwen3::Shape;
using qwen3::Tensor;
using test::require;
using test::require_throws;

static void body()
{
    const auto cpu = qwen3::Device::cpu();
    Tensor x = Tensor::empty(Shape{2, 3, 8}, DType::BFloat16, cpu);
    Tensor w = Tensor::empty(Shape{8}, DType::BFloat16, cpu);
    Tensor f = Tensor::empty(Shape{2, 3, 8}, DType::Float32, cpu);
    Tensor ids = Tensor::empty(Shape{2, 3}, DType::Int32, cpu);
    Tensor table = Tensor::empty(Shape{5, 8}, DType::BFloat16, cpu);

    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::rms_norm(x, w, 1e-6f); }, "rms_norm host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::rms_norm(f, w, 1e-6f); }, "rms_norm float32 input");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::silu_multiply(x, x); }, "silu host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::silu_multiply(x, f); }, "silu dtype mismatch");
    require_throws<std::invalid_argument>([&] { qwen3::ops::add_inplace(x, x); }, "add host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::embedding_lookup(ids, table); }, "embedding host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::embedding_lookup(table, table); }, "embedding bf16 ids");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::add_rms_norm(x, x, w, 1e-6f); }, "add_rms_norm host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::embedding_rms_norm(ids, table, w, 1e-6f); },
                                          "embedding_rms_norm host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::rms_norm_last_token(x, w, 1e-6f); },
                                          "last-token norm host tensors");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::rms_norm_last_token(f, w, 1e-6f); },
                                          "last-token norm float32 input");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::add_rms_norm_last_token(x, x, w, 1e-6f); },
                                          "last-token add norm host tensors");

    // KvCache constructor checks (src/model/kv_cache.cpp:17-73)
    require_throws<std::invalid_argument>([&] { qwen3::KvCache(0, 1, 4, 1, 8, DType::BFloat16, qwen3::Device::cuda(0)); },
                                          "KV cache with zero layers");
    require_throws<std::invalid_argument>([&] { qwen3::KvCache(1, 1, -4, 1, 8, DType::BFloat16, qwen3::Device::cuda(0)); },
                                          "KV cache with negative capacity");
    require_throws<std::invalid_argument>([&] { qwen3::KvCache(1, 1, 4, 1, 8, DType::Int32, qwen3::Device::cuda(0)); },
                                          "KV cache with int32 dtype");
    require_throws<std::invalid_argument>([&] { qwen3::KvCache(1, 1, 4, 1, 8, DType::BFloat16, cpu); },
                                          "KV cache on the host");

    Tensor cache = qwen3::ops::build_rope_cache(16, 8, 1.0e6f, cpu);
    require(cache.shape() == (Shape{16, 4, 2}) && cache.dtype() == DType::Float32 && cache.device().is_cpu(),
            "host rope cache shape");
    std::vector<float> ref(16 * 8);
    require(q3o_build_rope_cache(16, 8, 1.0e6f, ref.data()) == 0, "oracle table");
    require(std::memcmp(ref.data(), cache.data(), ref.size() * sizeof(float)) == 0, "rope cache equals the oracle's table");
    const auto *c = static_cast<const float *>(cache.data());
    require(c[0] == 1.0f && c[1] == 0.0f, "position 0 is (cos, sin) = (1, 0)");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::build_rope_cache(0, 8, 1e6f, cpu); }, "zero positions");
    require_throws<std::invalid_argument>([&] { (void)qwen3::ops::build_rope_cache(4, 7, 1e6f, cpu); }, "odd head_dim");
    require_throws<std::invalid_argument>(
        [&] { (void)qwen3::ops::build_rope_cache(4, 8, std::numeric_limits<float>::infinity(), cpu); }, "infinite theta");
    Tensor q = Tensor::empty(Shape{1, 3, 16}, DType::BFloat16, cpu);
    Tensor k = Tensor::empty(Shape{1, 3, 8}, DType::BFloat16, cpu);
    require_throws<std::invalid_argument>([&] { qwen3::ops::apply_rope_inplace(q, k, cache, 2, 1, 0); }, "rope host tensors");
    require_throws<std::invalid_argument>([&] { qwen3::ops::apply_rope_inplace(q, k, table, 2, 1, 0); }, "rope bf16 table");
}

int main() { return test::run("ops validation (CPU) test", body); }
