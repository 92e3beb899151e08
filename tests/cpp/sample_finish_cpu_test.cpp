// The sampler's host finish (qwen3::generation::detail::RowFinisher) against
// the oracle's restatement of the reference's per-row sampler
// (q3o_sample_row, src/generation/sampler.cpp:134-265), token for token, for
// the same uniform draw: whole rows (counting-sort path) and shuffled top-k
// candidate lists (the GPU path's input), with heavy ties, signed zeros,
// top_k at and past the row length, top_p = 1, and draws at 0 and near 1.
// Also the sampler's argument rules that need no GPU (configuration, logits
// dtype and device), each with its exception type and message.
#include "../../qwen3-runtime-byyourself_amd/csrc/generation/row_finish.hpp"
#include "qwen3/generation/sampler.h"
#include "test_util.hpp"

#include <algorithm>
#include <limits>
#include <random>

using qwen3::generation::Sampler;
using qwen3::generation::SamplingConfig;
using qwen3::generation::SamplingMode;
using qwen3::generation::detail::DrawRule;
using qwen3::generation::detail::RowFinisher;
using test::require;

namespace
{
    int checked = 0;

    void compare(RowFinisher &f, const std::vector<uint16_t> &row, const DrawRule &rule, double u, std::mt19937 &shuffle,
                 const std::string &what)
    {
        const auto n = static_cast<std::int64_t>(row.size());
        const int32_t want = q3o_sample_row(row.data(), n, rule.temperature, rule.top_k, rule.top_p, u);
        require(want >= 0, what + ": oracle rejected the row");
        const int32_t whole = f.from_row(row.data(), n, rule, u);
        require(whole == want, what + ": whole row gave " + std::to_string(whole) + ", oracle " + std::to_string(want));
        std::vector<int32_t> ids(row.size());
        const int64_t kept = q3o_topk_set(row.data(), n, rule.top_k, ids.data());
        ids.resize(static_cast<std::size_t>(kept));
        std::shuffle(ids.begin(), ids.end(), shuffle);   // the GPU lists candidates in no order
        std::vector<uint16_t> bits(ids.size());
        for (std::size_t i = 0; i < ids.size(); ++i)
            bits[i] = row[static_cast<std::size_t>(ids[i])];
        const int32_t cand = f.from_candidates(bits.data(), ids.data(), static_cast<int32_t>(ids.size()), rule, u);
        require(cand == want, what + ": candidates gave " + std::to_string(cand) + ", oracle " + std::to_string(want));
        checked += 2;
    }

    // The sampler's argument rules that need no GPU, in the order they are
    // checked: the configuration when a Sampler is made (greedy stops after
    // the mode), then the logits' dtype and device.
    template <typename F>
    void rule(const std::string &row, F &&f, const std::string &message)
    {
        bool caught = false;
        try
        {
            f();
        }
        catch (const std::invalid_argument &e)
        {
            caught = true;
            require(std::string(e.what()) == message, row + ": message '" + e.what() + "'");
        }
        require(caught, row + ": no std::invalid_argument");
        ++checked;
    }

    void contract_rows()
    {
        const auto make = [](SamplingConfig c) { Sampler s{c}; };
        const auto with = [](auto edit) {
            SamplingConfig c;
            edit(c);
            return c;
        };
        rule("S1 unknown mode", [&] { make(with([](SamplingConfig &c) { c.mode = static_cast<SamplingMode>(7); })); },
             "unknown sampling mode");
        for (float t : {0.0F, -1.0F, std::numeric_limits<float>::infinity(), std::numeric_limits<float>::quiet_NaN()})
            rule("S2 temperature " + std::to_string(t), [&] { make(with([&](SamplingConfig &c) { c.temperature = t; })); },
                 "sampling temperature must be finite and positive");
        rule("S3 negative top_k", [&] { make(with([](SamplingConfig &c) { c.top_k = -1; })); },
             "sampling top_k cannot be negative");
        for (float p : {0.0F, -0.5F, 1.5F, std::numeric_limits<float>::quiet_NaN()})
            rule("S4 top_p " + std::to_string(p), [&] { make(with([&](SamplingConfig &c) { c.top_p = p; })); },
                 "sampling top_p must be in the interval (0, 1]");
        rule("S order temperature before top_k", [&] {
            make(with([](SamplingConfig &c) { c.temperature = 0.0F; c.top_k = -1; c.top_p = 2.0F; }));
        }, "sampling temperature must be finite and positive");
        // greedy stops after the mode rule: the sampling fields are not read
        make(with([](SamplingConfig &c) { c.mode = SamplingMode::Greedy; c.temperature = 0.0F; c.top_k = -3; c.top_p = 9.0F; }));
        Sampler s{SamplingConfig{}};
        const auto f32 = qwen3::Tensor::empty(qwen3::Shape{2, 8}, qwen3::DType::Float32, qwen3::Device::cpu());
        const auto cpu = qwen3::Tensor::empty(qwen3::Shape{2, 8}, qwen3::DType::BFloat16, qwen3::Device::cpu());
        rule("S5 logits dtype", [&] { (void)s.sample(f32); }, "sampler logits must have BFloat16 dtype");
        rule("S6 logits device", [&] { (void)s.sample(cpu); }, "sampler logits must be on CUDA");
        auto out = qwen3::Tensor::empty(qwen3::Shape{2, 1}, qwen3::DType::Int32, qwen3::Device::cpu());
        rule("S6 logits device, sample into", [&] { s.sample(cpu, out); }, "sampler logits must be on CUDA");
    }

    void body()
    {
        RowFinisher f;
        std::mt19937 shuffle(5);
        std::mt19937_64 draws(99);
        const auto uniform = [&] { return static_cast<double>(draws() >> 11) * 0x1.0p-53; };
        const DrawRule rules[] = {{0.6F, 20, 0.95F}, {1.0F, 1, 1.0F}, {1.3F, 1024, 0.5F}, {0.7F, 0, 0.9F},
                                  {0.8F, 50, 1.0F},  {2.0F, 7, 0.3F},  {0.05F, 200, 0.999F}};
        // random rows of several lengths
        for (std::size_t n : {1u, 2u, 7u, 300u, 5000u, 151669u})
        {
            const auto row = test::values(n, 1000 + n, 3.0F);
            for (const DrawRule &r : rules)
                for (int k = 0; k < (n > 10000 ? 2 : 6); ++k)
                    compare(f, row, r, uniform(), shuffle, "random row n=" + std::to_string(n));
        }
        // heavy ties: few distinct values, signed zeros among them
        {
            std::vector<uint16_t> row(4096);
            std::mt19937 g(3);
            const uint16_t vals[] = {test::bf16(2.0F), test::bf16(1.5F), 0x0000, 0x8000, test::bf16(-1.0F), test::bf16(2.0F)};
            for (auto &v : row)
                v = vals[g() % 6];
            for (const DrawRule &r : rules)
                for (int k = 0; k < 6; ++k)
                    compare(f, row, r, uniform(), shuffle, "tied row");
            for (int32_t kk : {1, 2, 100, 700, 4095, 4096, 5000})
                compare(f, row, DrawRule{1.0F, kk, 0.9F}, uniform(), shuffle, "tied row, top_k " + std::to_string(kk));
        }
        // all logits equal; the maximum at the last token; extreme draws
        {
            std::vector<uint16_t> flat(1000, test::bf16(0.25F));
            std::vector<uint16_t> last = test::values(1000, 8, 1.0F);
            last.back() = test::bf16(40.0F);
            for (double u : {0.0, 0.5, 1.0 - 0x1.0p-53})
                for (const DrawRule &r : rules)
                {
                    compare(f, flat, r, u, shuffle, "flat row");
                    compare(f, last, r, u, shuffle, "peak at the end");
                }
        }
        // non-finite logits are rejected (the reference throws from its temperature loop)
        std::vector<uint16_t> bad = test::values(64, 9, 1.0F);
        bad[40] = 0x7f80;   // +inf
        test::require_throws<std::runtime_error>([&] { (void)f.from_row(bad.data(), 64, rules[0], 0.5); }, "inf accepted");
        bad[40] = 0x7fc1;   // NaN
        test::require_throws<std::runtime_error>([&] { (void)f.from_row(bad.data(), 64, rules[0], 0.5); }, "NaN accepted");
        std::cout << checked << " rows checked against the oracle\n";
        contract_rows();
    }
} // namespace

int main() { return test::run("sampler host finish (CPU) test", body); }
