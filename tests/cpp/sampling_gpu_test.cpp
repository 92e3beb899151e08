// Sampler and argmax on the GPU: the reference's tests
// (tests/unit/argmax_cuda_test.cpp, sampler_cuda_test.cpp) and the sampler's
// GPU top-k path against the oracle's restatement of the reference sampler,
// token for token, fed the same mt19937_64 draws.
#include "gpu_util.hpp"
#include "qwen3/generation/sampler.h"
#include "qwen3/ops/argmax.h"

#include <limits>
#include <random>

using qwen3::DType;
using qwen3::Shape;
using qwen3::Tensor;
using qwen3::generation::Sampler;
using qwen3::generation::SamplingConfig;
using qwen3::generation::SamplingMode;
using test::require;
using test::require_throws;

namespace
{
    Tensor logits_of(const std::vector<float> &values, std::int64_t rows, std::int64_t cols)
    {
        std::vector<uint16_t> b(values.size());
        for (std::size_t i = 0; i < values.size(); ++i)
            b[i] = q3o_bf16_from_f32(values[i]);
        return test::to_gpu(b, Shape{rows, cols}, DType::BFloat16);
    }

    void argmax_reference_test()
    {
        std::vector<float> v(2 * 513, -8.0F);
        v[512] = 12.0F;
        v[513 + 17] = 9.0F;
        v[513 + 500] = 9.0F;
        Tensor x = logits_of(v, 2, 513);
        Tensor compact = qwen3::ops::argmax_last_dimension(x, false);
        Tensor kept = qwen3::ops::argmax_last_dimension(x, true);
        require(compact.shape() == (Shape{2}) && kept.shape() == (Shape{2, 1}), "argmax output shapes");
        require(kept.dtype() == DType::Int32 && kept.device() == qwen3::Device::cuda(0), "argmax dtype and device");
        const auto c = test::to_host<int32_t>(compact), k = test::to_host<int32_t>(kept);
        require(c[0] == 512 && c[1] == 17 && k[0] == 512 && k[1] == 17, "argmax results (ties to the smaller id)");
        const auto p = test::to_host<int32_t>(qwen3::ops::argmax_last_dimension(x, false, 100));
        require(p[0] == 0 && p[1] == 17, "argmax over a valid prefix");
        require_throws<std::invalid_argument>([&] { (void)qwen3::ops::argmax_last_dimension(x, false, 514); },
                                              "valid size past the row accepted");
    }

    void sampler_reference_test()
    {
        Tensor greedy_logits = logits_of({-1, 0, 4, 2, -2, 3, 7, 7, 1, 0}, 2, 5);
        SamplingConfig greedy;
        greedy.mode = SamplingMode::Greedy;
        const auto g = test::to_host<int32_t>(Sampler{greedy}.sample(greedy_logits));
        require(g[0] == 2 && g[1] == 1, "greedy result and tie-breaking");
        SamplingConfig top_one;
        top_one.temperature = 0.6F;
        top_one.top_k = 1;
        top_one.top_p = 1.0F;
        top_one.seed = 122;
        Sampler s1{top_one};
        Tensor t1 = s1.sample(greedy_logits);
        require(t1.shape() == (Shape{2, 1}) && t1.device() == qwen3::Device::cuda(0), "sample output shape");
        const auto o1 = test::to_host<int32_t>(t1);
        require(o1[0] == 2 && o1[1] == 1, "top_k = 1 with seed 122");
        Tensor sampling_logits = logits_of({2, 2, 1, -10}, 1, 4);
        SamplingConfig cfg;
        cfg.temperature = 1.0F;
        cfg.top_k = 3;
        cfg.top_p = 0.8F;
        cfg.seed = 42;
        Sampler s{cfg};
        std::vector<int32_t> first;
        for (int i = 0; i < 16; ++i)
        {
            const auto id = test::to_host<int32_t>(s.sample(sampling_logits))[0];
            require(id == 0 || id == 1, "top-p selected a filtered token");
            first.push_back(id);
        }
        s.reseed(42);
        for (int i = 0; i < 16; ++i)
            require(test::to_host<int32_t>(s.sample(sampling_logits))[0] == first[static_cast<std::size_t>(i)],
                    "reseed replays the sequence");
        require_throws<std::invalid_argument>([] { SamplingConfig c; c.temperature = 0.0F; Sampler x{c}; }, "zero temperature");
        require_throws<std::invalid_argument>([] { SamplingConfig c; c.top_p = 1.5F; Sampler x{c}; }, "top_p above 1");
        require_throws<std::invalid_argument>([] { SamplingConfig c; c.top_k = -1; Sampler x{c}; }, "negative top_k");
        Tensor bad = logits_of({1.0F, std::numeric_limits<float>::infinity(), 0.0F}, 1, 3);
        SamplingConfig k2;
        k2.top_k = 2;
        Sampler sb{k2};
        require_throws<std::runtime_error>([&] { (void)sb.sample(bad); }, "non-finite logit accepted");
        // logits shape and the valid-vocabulary prefix, checked when sampling
        const auto message_is = [](const char *row, auto &&f, const std::string &want) {
            bool caught = false;
            try
            {
                f();
            }
            catch (const std::invalid_argument &e)
            {
                caught = true;
                require(std::string(e.what()) == want, std::string(row) + ": message '" + e.what() + "'");
            }
            require(caught, std::string(row) + ": accepted");
        };
        Sampler plain{SamplingConfig{}};
        const Tensor rank1 = test::to_gpu(std::vector<uint16_t>(3, 0), Shape{3}, DType::BFloat16);
        const Tensor no_rows = Tensor::empty(Shape{0, 3}, DType::BFloat16, qwen3::Device::cuda(0));
        const Tensor no_cols = Tensor::empty(Shape{2, 0}, DType::BFloat16, qwen3::Device::cuda(0));
        message_is("S7 rank", [&] { (void)plain.sample(rank1); }, "sampler logits must have shape [batch_size, vocab_size]");
        message_is("S7 batch", [&] { (void)plain.sample(no_rows); }, "sampler batch size must be positive");
        message_is("S7 vocabulary", [&] { (void)plain.sample(no_cols); }, "sampler vocabulary size must be positive");
        SamplingConfig neg;
        neg.valid_vocab_size = -1;
        Sampler sn{neg};
        message_is("S8 negative prefix", [&] { (void)sn.sample(logits_of({1.0F, 2.0F, 3.0F}, 1, 3)); },
                   "valid_vocab_size cannot be negative");
        SamplingConfig wide;
        wide.valid_vocab_size = 4;
        Sampler sw{wide};
        message_is("S8 prefix past the vocabulary", [&] { (void)sw.sample(logits_of({1.0F, 2.0F, 3.0F}, 1, 3)); },
                   "valid_vocab_size exceeds logits vocabulary size");
    }

    // The GPU top-k path and the whole-row path against the oracle's
    // restatement of the reference sampler, over a real vocabulary.  From 16
    // rows on the candidate rows are finished by a row crew (B = 40 here),
    // with the tie-overflow row among them.
    void sampler_against_oracle(std::int64_t B)
    {
        constexpr std::int64_t V = 151936, valid = 151669;
        std::vector<uint16_t> host(static_cast<std::size_t>(B * V));
        const auto vals = test::values(host.size(), 77, 3.0F);
        host = vals;
        // row 1: many ties at the top (more than the GPU candidate capacity)
        for (std::int64_t i = 0; i < 3000; ++i)
            host[static_cast<std::size_t>(V + i * 37)] = q3o_bf16_from_f32(30.0F);
        Tensor logits = test::to_gpu(host, Shape{B, V}, DType::BFloat16);
        struct Case
        {
            std::int32_t top_k;
            float top_p;
            float temperature;
        };
        for (const Case cs : {Case{20, 0.95F, 0.6F}, Case{1, 1.0F, 1.0F}, Case{1024, 0.5F, 1.3F}, Case{0, 0.9F, 0.7F},
                              Case{50, 1.0F, 0.8F}})
        {
            SamplingConfig cfg;
            cfg.top_k = cs.top_k;
            cfg.top_p = cs.top_p;
            cfg.temperature = cs.temperature;
            cfg.seed = 1234;
            cfg.valid_vocab_size = valid;
            Sampler s{cfg};
            std::mt19937_64 engine(1234);
            for (int step = 0; step < (cs.top_k == 0 ? 2 : 6); ++step)
            {
                const auto got = test::to_host<int32_t>(s.sample(logits));
                for (std::int64_t b = 0; b < B; ++b)
                {
                    const double u = static_cast<double>(engine() >> 11U) * (1.0 / 9007199254740992.0);
                    const int32_t want = q3o_sample_row(host.data() + b * V, valid, cs.temperature, cs.top_k,
                                                        cs.top_p, u);
                    require(got[static_cast<std::size_t>(b)] == want, "sampled token differs from the oracle's");
                }
            }
        }
    }

    // A non-finite logit in row 7 of 20 ends the call; the engine then stands
    // after the draws of rows 0..6, as at the reference's row loop (the draw
    // comes after the scores, src/generation/sampler.cpp:151,232).  Checked
    // through the next call's tokens, for the GPU-candidate path and the
    // whole-row path (both finished by the row crew at 20 rows).
    void sampler_after_nonfinite_row()
    {
        constexpr std::int64_t B = 20, V = 4096;
        const auto good = test::values(static_cast<std::size_t>(B * V), 91, 2.0F);
        std::vector<uint16_t> bad = good;
        bad[static_cast<std::size_t>(7 * V + 123)] = 0x7f80;   // +inf in row 7
        const Tensor good_t = test::to_gpu(good, Shape{B, V}, DType::BFloat16);
        const Tensor bad_t = test::to_gpu(bad, Shape{B, V}, DType::BFloat16);
        for (const std::int32_t top_k : {20, 0})
        {
            SamplingConfig cfg;
            cfg.top_k = top_k;
            cfg.top_p = 0.9F;
            cfg.temperature = 0.8F;
            cfg.seed = 77;
            Sampler s{cfg};
            test::require_throws<std::runtime_error>([&] { (void)s.sample(bad_t); }, "non-finite row accepted");
            const auto got = test::to_host<int32_t>(s.sample(good_t));
            std::mt19937_64 engine(77);
            for (int i = 0; i < 7; ++i)
                (void)engine();
            for (std::int64_t b = 0; b < B; ++b)
            {
                const double u = static_cast<double>(engine() >> 11U) * (1.0 / 9007199254740992.0);
                const int32_t want = q3o_sample_row(good.data() + b * V, V, cfg.temperature, cfg.top_k, cfg.top_p, u);
                require(got[static_cast<std::size_t>(b)] == want,
                        "tokens after a non-finite row: top_k " + std::to_string(top_k));
            }
        }
    }

    void body()
    {
        test::require_gpu();
        const int before = test::current_device();
        argmax_reference_test();
        sampler_reference_test();
        sampler_against_oracle(6);
        sampler_against_oracle(40);
        sampler_after_nonfinite_row();
        require(test::current_device() == before, "a sampling call changed the current device");
    }
} // namespace

int main() { return test::run("GPU sampling test", body); }
