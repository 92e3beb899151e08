// The sampler's host finish (qwen3::generation::detail::RowFinisher) against
// the oracle's restatement of the reference's per-row sampler
// (q3o_sample_row, src/generation/sampler.cpp:134-265), token for token, for
// the same uniform draw: whole rows (counting-sort path) and shuffled top-k
// candidate lists (the GPU path's input), with heavy ties, signed zeros,
// top_k at and past the row length, top_p = 1, and draws at 0 and near 1.
#include "../../qwen3-runtime-byyourself_amd/csrc/generation/row_finish.hpp"
#include "test_util.hpp"

#include <algorithm>
#include <limits>
#include <random>

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
    }
} // namespace

int main() { return test::run("sampler host finish (CPU) test", body); }
