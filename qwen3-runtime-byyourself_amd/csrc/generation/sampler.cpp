// qwen3::generation::Sampler.  Checks and the per-row algorithm follow
// src/generation/sampler.cpp of the reference: temperature (:144-158),
// top-k keeping ties at the k-th (:160-190), sort (:192-194), stable
// softmax in double (:196-215), top-p (:217-238), the draw (:240-265) with
// the 53-bit uniform of mt19937_64 (:34-43).  The top-k step runs on the GPU
// (q3k_topk_candidates_bf16); only the candidates cross to the host.
#include "qwen3/generation/sampler.h"

#include "../ops/ops_common.hpp"
#include "qwen3/ops/argmax.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace qwen3::generation
{
    namespace
    {
        struct Candidate final
        {
            double score = 0.0;
            std::int32_t token_id = 0;
        };

        bool better(const Candidate &lhs, const Candidate &rhs)
        {
            if (lhs.score == rhs.score)
                return lhs.token_id < rhs.token_id;
            return lhs.score > rhs.score;
        }

        float bf16_to_float(std::uint16_t value)
        {
            const std::uint32_t bits = static_cast<std::uint32_t>(value) << 16U;
            float result = 0.0F;
            std::memcpy(&result, &bits, sizeof(result));
            return result;
        }

        double next_uniform(std::mt19937_64 &engine)
        {
            return static_cast<double>(engine() >> 11U) * (1.0 / 9007199254740992.0);
        }

        void validate_config(const SamplingConfig &config)
        {
            switch (config.mode)
            {
            case SamplingMode::Greedy: return;
            case SamplingMode::Sample: break;
            default: throw std::invalid_argument("unknown sampling mode");
            }
            if (!std::isfinite(config.temperature) || config.temperature <= 0.0F)
                throw std::invalid_argument("sampling temperature must be finite and positive");
            if (config.top_k < 0)
                throw std::invalid_argument("sampling top_k cannot be negative");
            if (!std::isfinite(config.top_p) || config.top_p <= 0.0F || config.top_p > 1.0F)
                throw std::invalid_argument("sampling top_p must be in the interval (0, 1]");
        }

        void validate_logits(const Tensor &logits)
        {
            if (logits.dtype() != DType::BFloat16)
                throw std::invalid_argument("sampler logits must have BFloat16 dtype");
            if (!logits.device().is_cuda())
                throw std::invalid_argument("sampler logits must be on CUDA");
            if (logits.shape().rank() != 2)
                throw std::invalid_argument("sampler logits must have shape [batch_size, vocab_size]");
            if (logits.shape()[0] <= 0)
                throw std::invalid_argument("sampler batch size must be positive");
            if (logits.shape()[1] <= 0)
                throw std::invalid_argument("sampler vocabulary size must be positive");
        }

        std::int64_t resolve_valid_vocab_size(const Tensor &logits, const SamplingConfig &config)
        {
            if (config.valid_vocab_size < 0)
                throw std::invalid_argument("valid_vocab_size cannot be negative");
            if (config.valid_vocab_size == 0)
                return logits.shape()[1];
            if (config.valid_vocab_size > logits.shape()[1])
                throw std::invalid_argument("valid_vocab_size exceeds logits vocabulary size");
            return config.valid_vocab_size;
        }

        [[noreturn]] void non_finite() { throw std::runtime_error("temperature scaling produced a non-finite score"); }

        // Steps after top-k on a candidate list that already holds every token
        // the reference's top-k keeps (the whole row when top-k is off).
        std::int32_t finish_row(std::vector<Candidate> &candidates, const SamplingConfig &config,
                                std::mt19937_64 &engine)
        {
            if (config.top_k > 0)
            {
                const std::size_t k = std::min(static_cast<std::size_t>(config.top_k), candidates.size());
                if (k < candidates.size())
                {
                    auto kth = candidates.begin() + static_cast<std::ptrdiff_t>(k - 1);
                    std::nth_element(candidates.begin(), kth, candidates.end(), better);
                    const double kth_score = kth->score;
                    candidates.erase(std::remove_if(candidates.begin(), candidates.end(),
                                                    [kth_score](const Candidate &c) { return c.score < kth_score; }),
                                     candidates.end());
                }
            }
            std::sort(candidates.begin(), candidates.end(), better);
            const double maximum = candidates.front().score;
            std::vector<double> weights(candidates.size());
            double total = 0.0;
            for (std::size_t i = 0; i < candidates.size(); ++i)
            {
                weights[i] = std::exp(candidates[i].score - maximum);
                total += weights[i];
            }
            if (!std::isfinite(total) || total <= 0.0)
                throw std::runtime_error("sampler softmax weight sum is invalid");
            const double threshold = static_cast<double>(config.top_p) * total;
            std::size_t retained = candidates.size();
            double retained_weight = 0.0;
            for (std::size_t i = 0; i < candidates.size(); ++i)
            {
                retained_weight += weights[i];
                if (retained_weight >= threshold)
                {
                    retained = i + 1;
                    break;
                }
            }
            const double r = next_uniform(engine) * retained_weight;
            double cumulative = 0.0;
            for (std::size_t i = 0; i < retained; ++i)
            {
                cumulative += weights[i];
                if (r < cumulative)
                    return candidates[i].token_id;
            }
            return candidates[retained - 1].token_id;
        }

        std::vector<Candidate> whole_row(const std::uint16_t *row, std::int64_t n, float temperature)
        {
            std::vector<Candidate> c;
            c.reserve(static_cast<std::size_t>(n));
            for (std::int64_t t = 0; t < n; ++t)
            {
                const float logit = bf16_to_float(row[t]);
                if (!std::isfinite(logit))
                    non_finite();
                c.push_back(Candidate{static_cast<double>(logit) / static_cast<double>(temperature),
                                      static_cast<std::int32_t>(t)});
            }
            return c;
        }

        template <typename T>
        std::vector<T> to_host(const Tensor &t)
        {
            Tensor host = t.copy_to(Device::cpu());
            std::vector<T> out(static_cast<std::size_t>(host.numel()));
            if (!out.empty())
                std::memcpy(out.data(), host.data(), host.nbytes());
            return out;
        }
    } // namespace

    Sampler::Sampler(SamplingConfig config) : config_(config), random_engine_(config.seed) { validate_config(config_); }

    void Sampler::reseed(std::uint64_t seed)
    {
        config_.seed = seed;
        random_engine_.seed(seed);
    }

    Tensor Sampler::sample(const Tensor &logits)
    {
        validate_logits(logits);
        const std::int64_t batch = logits.shape()[0];
        const std::int64_t vocab = logits.shape()[1];
        const std::int64_t valid = resolve_valid_vocab_size(logits, config_);
        if (config_.mode == SamplingMode::Greedy)
            return ops::argmax_last_dimension(logits, true, valid);

        Tensor tokens = Tensor::empty(Shape{batch, 1}, DType::Int32, Device::cpu());
        auto *out = static_cast<std::int32_t *>(tokens.data());
        const bool on_gpu = config_.top_k > 0 && config_.top_k < valid && config_.top_k <= kGpuCandidateCapacity;
        if (on_gpu)
        {
            constexpr std::int32_t cap = kGpuCandidateCapacity;
            Tensor count = Tensor::empty(Shape{batch}, DType::Int32, logits.device());
            Tensor bad = Tensor::empty(Shape{batch}, DType::Int32, logits.device());
            Tensor index = Tensor::empty(Shape{batch, cap}, DType::Int32, logits.device());
            Tensor value = Tensor::empty(Shape{batch, cap}, DType::BFloat16, logits.device());
            // few rows are cut into slices searched by separate blocks; their lists need a workspace
            const std::int64_t ws_bytes = q3k_topk_workspace_bytes(batch, valid, config_.top_k);
            Tensor workspace = Tensor::empty(Shape{(ws_bytes + 3) / 4}, DType::Int32, logits.device());
            ops::detail::launch_on(logits.device(), [&](q3k_stream_t stream) {
                return q3k_topk_candidates_bf16(static_cast<const uint16_t *>(logits.data()), batch, vocab, valid,
                                                config_.top_k, cap, static_cast<int32_t *>(count.data()),
                                                static_cast<int32_t *>(index.data()),
                                                static_cast<uint16_t *>(value.data()),
                                                static_cast<int32_t *>(bad.data()),
                                                ws_bytes > 0 ? workspace.data() : nullptr, ws_bytes, stream);
            });
            const auto counts = to_host<std::int32_t>(count);
            const auto flags = to_host<std::int32_t>(bad);
            const auto ids = to_host<std::int32_t>(index);
            const auto vals = to_host<std::uint16_t>(value);
            std::vector<std::uint16_t> full_row; // a row whose ties overflow the capacity
            for (std::int64_t b = 0; b < batch; ++b)
            {
                if (flags[static_cast<std::size_t>(b)] != 0)
                    non_finite();
                std::vector<Candidate> c;
                const std::int32_t n = counts[static_cast<std::size_t>(b)];
                if (n <= cap)
                {
                    c.reserve(static_cast<std::size_t>(n));
                    for (std::int32_t i = 0; i < n; ++i)
                    {
                        const std::size_t at = static_cast<std::size_t>(b * cap + i);
                        c.push_back(Candidate{static_cast<double>(bf16_to_float(vals[at])) /
                                                  static_cast<double>(config_.temperature),
                                              ids[at]});
                    }
                }
                else
                {
                    full_row.resize(static_cast<std::size_t>(valid));
                    ops::detail::launch_on(logits.device(), [&](q3k_stream_t) {
                        const hipError_t e = hipMemcpy(full_row.data(),
                                                       static_cast<const std::uint16_t *>(logits.data()) + b * vocab,
                                                       static_cast<std::size_t>(valid) * 2, hipMemcpyDeviceToHost);
                        return e == hipSuccess ? Q3K_OK : Q3K_ERR_HIP;
                    });
                    c = whole_row(full_row.data(), valid, config_.temperature);
                }
                out[b] = finish_row(c, config_, random_engine_);
            }
        }
        else
        {
            const auto host = to_host<std::uint16_t>(logits);
            for (std::int64_t b = 0; b < batch; ++b)
            {
                auto c = whole_row(host.data() + b * vocab, valid, config_.temperature);
                out[b] = finish_row(c, config_, random_engine_);
            }
        }
        return tokens.copy_to(logits.device());
    }
} // namespace qwen3::generation
