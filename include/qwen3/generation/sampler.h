#pragma once

// Next-token selection from [batch, vocab] logits (the reference's
// include/qwen3/generation/sampler.h interface and behaviour).  Greedy runs
// entirely on the GPU.  Sampling selects the top-k candidates on the GPU and
// finishes on the host with the reference's arithmetic (double-precision
// softmax, top-p, one mt19937_64 draw per row), so the same seed gives the
// same tokens as the reference; top_k = 0 takes the whole row to the host,
// as the reference always does.

#include "qwen3/core/tensor.h"

#include <cstdint>
#include <random>

namespace qwen3::generation
{
    enum class SamplingMode
    {
        Greedy,
        Sample,
    };

    struct SamplingConfig final
    {
        SamplingMode mode = SamplingMode::Sample;
        float temperature = 0.6F;
        std::int32_t top_k = 20;           // 0 disables top-k
        float top_p = 0.95F;               // 1 disables top-p
        std::uint64_t seed = 42;
        std::int64_t valid_vocab_size = 0; // sampled vocabulary prefix; 0 = the whole last dimension
    };

    class Sampler final
    {
    public:
        explicit Sampler(SamplingConfig config);

        // logits BFloat16 [batch, vocab] on the GPU -> Int32 [batch, 1] on the
        // same GPU.
        [[nodiscard]] Tensor sample(const Tensor &logits);

        // Restarts the random sequence: the same seed replays the same draws.
        void reseed(std::uint64_t seed);

        // Largest top_k whose candidates are selected on the GPU (larger ones,
        // or rows whose ties exceed it, take the whole row to the host).
        static constexpr std::int32_t kGpuCandidateCapacity = 1024;

    private:
        SamplingConfig config_;
        std::mt19937_64 random_engine_;
    };
} // namespace qwen3::generation
