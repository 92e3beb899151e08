#pragma once

// Next-token selection from [batch, vocab] logits.  Public interface and
// behaviour of the reference's include/qwen3/generation/sampler.h: greedy
// argmax, or temperature / top-k (ties at the k-th kept) / top-p sampling
// with one mt19937_64 draw per row, so a seed replays the same tokens.
//
// Greedy runs on the GPU.  Sampling selects each row's top-k candidates on
// the GPU; only the candidates cross to the host, where the row is finished
// (top_k = 0, or a row whose ties overflow the candidate capacity, takes the
// whole row to the host).  The device and pinned host buffers a call needs
// are owned by the sampler and reused by later calls; a copied sampler
// starts with none.

#include "qwen3/core/tensor.h"

#include <cstdint>
#include <memory>
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

    namespace detail
    {
        struct SamplerScratch;
    }

    class Sampler final
    {
    public:
        // Throws std::invalid_argument for an invalid configuration.
        explicit Sampler(SamplingConfig config);
        ~Sampler();
        Sampler(const Sampler &other);
        Sampler &operator=(const Sampler &other);
        Sampler(Sampler &&other) noexcept;
        Sampler &operator=(Sampler &&other) noexcept;

        // logits BFloat16 [batch, vocab] on a GPU -> Int32 [batch, 1] on the
        // same GPU.
        [[nodiscard]] Tensor sample(const Tensor &logits);

        // The same into `token_ids` (Int32, [batch, 1], on the logits' GPU):
        // a call allocates no device memory once the sampler has seen a
        // batch of this size.
        void sample(const Tensor &logits, Tensor &token_ids);

        // Restarts the random sequence: the same seed replays the same draws.
        void reseed(std::uint64_t seed);

        // Largest top_k whose candidates are selected on the GPU.
        static constexpr std::int32_t kGpuCandidateCapacity = 1024;

    private:
        SamplingConfig config_;
        std::mt19937_64 random_engine_;
        std::unique_ptr<detail::SamplerScratch> scratch_;
    };
} // namespace qwen3::generation
