// Per-token latency of next-token selection on the GPU, through the C++
// runtime the generation loop calls (src/generation/sampler.cpp:268-313 and
// src/ops/argmax.cu:163-214 of the reference): argmax_last_dimension,
// Sampler greedy, and Sampler with the reference's default sampling
// (temperature 0.6, top_k 20, top_p 0.95), over [B, 151936] bf16 logits at
// B = 1 and 64.  Each call returns its token ids on the GPU; the time is the
// host wall time per call with the device synchronised at the end, i.e. what
// one decode step spends selecting its tokens.  Also reports the device
// allocations made per call once warm (qwen3::device_allocation_count()).
//
// Usage: q3k_decode_select_bench [--calls N]; prints one JSON line.
#include "qwen3/core/buffer.h"
#include "qwen3/core/tensor.h"
#include "qwen3/generation/sampler.h"
#include "qwen3/hip/hip_check.h"
#include "qwen3/ops/argmax.h"

#include <chrono>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <vector>

namespace
{
    qwen3::Tensor random_logits(std::int64_t rows, std::int64_t vocab)
    {
        std::vector<std::uint16_t> host(static_cast<std::size_t>(rows * vocab));
        std::mt19937 g(17);
        std::normal_distribution<float> n(0.0F, 3.0F);
        for (auto &b : host)
        {
            const float v = n(g);
            std::uint32_t w;
            std::memcpy(&w, &v, sizeof w);
            b = static_cast<std::uint16_t>((w + 0x7fffu + ((w >> 16) & 1u)) >> 16);
        }
        qwen3::Tensor cpu = qwen3::Tensor::empty(qwen3::Shape{rows, vocab}, qwen3::DType::BFloat16, qwen3::Device::cpu());
        std::memcpy(cpu.data(), host.data(), cpu.nbytes());
        return cpu.copy_to(qwen3::Device::cuda(0));
    }

    // {microseconds per call, device allocations per call}
    std::pair<double, double> time_calls(int calls, const std::function<void()> &call)
    {
        for (int i = 0; i < 3; ++i)
            call();
        QWEN3_HIP_CHECK(hipDeviceSynchronize());
        const auto allocs = qwen3::device_allocation_count();
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < calls; ++i)
            call();
        QWEN3_HIP_CHECK(hipDeviceSynchronize());
        const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        return {us / calls, static_cast<double>(qwen3::device_allocation_count() - allocs) / calls};
    }
} // namespace

int main(int argc, char **argv)
{
    int calls = 200;
    for (int i = 1; i + 1 < argc; ++i)
        if (std::string(argv[i]) == "--calls")
            calls = std::stoi(argv[++i]);
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1)
    {
        std::fprintf(stderr, "no visible GPU\n");
        return 1;
    }
    try
    {
        constexpr std::int64_t kVocab = 151936;
        std::string json = "{\"unit\": \"us per call\", \"vocab\": " + std::to_string(kVocab) + ", \"calls\": " +
                           std::to_string(calls);
        for (const std::int64_t B : {1, 64})
        {
            qwen3::Tensor logits = random_logits(B, kVocab);
            qwen3::generation::SamplingConfig greedy_cfg;
            greedy_cfg.mode = qwen3::generation::SamplingMode::Greedy;
            qwen3::generation::Sampler greedy{greedy_cfg};
            qwen3::generation::Sampler sampler{qwen3::generation::SamplingConfig{}};
            const auto a = time_calls(calls, [&] { (void)qwen3::ops::argmax_last_dimension(logits, true); });
            const auto g = time_calls(calls, [&] { (void)greedy.sample(logits); });
            const auto s = time_calls(calls, [&] { (void)sampler.sample(logits); });
            char buf[512];
            std::snprintf(buf, sizeof buf,
                          ", \"b%lld\": {\"argmax\": %.2f, \"sampler_greedy\": %.2f, \"sampler_topk20_topp095\": %.2f, "
                          "\"device_allocations_per_call\": %.3f}",
                          static_cast<long long>(B), a.first, g.first, s.first, a.second + g.second + s.second);
            json += buf;
        }
        std::printf("%s}\n", json.c_str());
    }
    catch (const std::exception &e)
    {
        std::fprintf(stderr, "decode select bench failed: %s\n", e.what());
        return 1;
    }
    return 0;
}
