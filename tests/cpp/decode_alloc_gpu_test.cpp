// A decode step's selection and attention calls allocate no device memory
// once warm: Sampler::sample (greedy, GPU top-k, whole-row), the
// sample-into form, argmax_last_dimension and the key-split decode
// attention, counted with qwen3::device_allocation_count() (hipMalloc calls
// made by Buffers).  Also prints the host latency per token of each call.
#include "gpu_util.hpp"
#include "qwen3/generation/sampler.h"
#include "qwen3/ops/argmax.h"
#include "qwen3/ops/gqa_attention.h"

#include <chrono>
#include <cstdio>

using qwen3::DType;
using qwen3::Shape;
using qwen3::Tensor;
using qwen3::generation::Sampler;
using qwen3::generation::SamplingConfig;
using qwen3::generation::SamplingMode;
using test::require;

namespace
{
    template <typename F>
    void steady(const char *what, int steps, F step)
    {
        step();   // warm: buffers made here are kept and reused
        step();
        QWEN3_HIP_CHECK(hipDeviceSynchronize());
        const auto before = qwen3::device_allocation_count();
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; ++i)
            step();
        QWEN3_HIP_CHECK(hipDeviceSynchronize());
        const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / steps;
        const auto made = qwen3::device_allocation_count() - before;
        std::printf("%-44s %8.1f us per call, %llu device allocations in %d calls\n", what, us,
                    static_cast<unsigned long long>(made), steps);
        require(made == 0, std::string(what) + ": device memory allocated per call");
    }

    void body()
    {
        test::require_gpu();
        constexpr std::int64_t V = 151936;
        for (const std::int64_t B : {1, 64})
        {
            Tensor logits = test::to_gpu(test::values(static_cast<std::size_t>(B * V), 11, 3.0F), Shape{B, V},
                                         DType::BFloat16);
            SamplingConfig greedy;
            greedy.mode = SamplingMode::Greedy;
            Sampler g{greedy};
            SamplingConfig topk;   // the reference's defaults: top_k 20, top_p 0.95, temperature 0.6
            Sampler s{topk};
            SamplingConfig whole;
            whole.top_k = 0;
            Sampler w{whole};
            Tensor out = Tensor::empty(Shape{B, 1}, DType::Int32, qwen3::Device::cuda(0));
            const std::string b = " B=" + std::to_string(B);
            steady(("argmax_last_dimension" + b).c_str(), 20, [&] { (void)qwen3::ops::argmax_last_dimension(logits, true); });
            steady(("Sampler greedy" + b).c_str(), 20, [&] { (void)g.sample(logits); });
            steady(("Sampler top_k 20 (GPU candidates)" + b).c_str(), 20, [&] { (void)s.sample(logits); });
            steady(("Sampler top_k 20 into a tensor" + b).c_str(), 20, [&] { s.sample(logits, out); });
            steady(("Sampler top_k 0 (whole rows)" + b).c_str(), B == 1 ? 10 : 2, [&] { w.sample(logits, out); });
        }
        // decode attention over a long cache: the key range is split, with a workspace
        constexpr std::int64_t Hq = 32, Hkv = 8, D = 128, L = 4096;
        Tensor q = test::to_gpu(test::values(Hq * D, 3, 1.0F), Shape{1, 1, Hq * D}, DType::BFloat16);
        Tensor kc = test::to_gpu(test::values(L * Hkv * D, 4, 1.0F), Shape{1, L, Hkv, D}, DType::BFloat16);
        Tensor vc = test::to_gpu(test::values(L * Hkv * D, 5, 1.0F), Shape{1, L, Hkv, D}, DType::BFloat16);
        steady("grouped_query_attention decode B=1 L=4096", 20, [&] {
            (void)qwen3::ops::grouped_query_attention(q, kc.view(), vc.view(), static_cast<std::int32_t>(Hq), L - 1);
        });
    }
} // namespace

int main() { return test::run("decode allocation GPU test", body); }
