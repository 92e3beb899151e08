// The host half of sampling one row: from the row's top-k candidates (or
// the whole row) to one token id, given the uniform draw u in [0, 1).
//
// Candidates are ordered by a 16-bit order key of their bf16 logit
// (temperature scaling is monotone, so the key order is the score order; -0
// and +0 share a key, as their scores compare equal), ties by ascending id.
// A whole row is ordered with a counting sort over the 65536 keys, which
// also yields the top-k cut (the bucket where the running count reaches k;
// every logit tied with the k-th is kept).  Then, over the ordered list:
// scores s_i = logit_i / temperature in double, weights w_i = exp(s_i - s_0),
// one array of running sums P_i = P_{i-1} + w_i, the top-p cut at the first
// i with P_i >= top_p * P_last, and the token at the first i with
// u * P_cut < P_i.  The running sums are the ones the reference accumulates
// in its softmax, top-p and draw loops (src/generation/sampler.cpp:196-265),
// added in the same order, so every comparison sees the same doubles and the
// same seed gives the same token.
#pragma once

#include <cstdint>
#include <vector>

namespace qwen3::generation::detail
{
    struct DrawRule
    {
        float temperature;
        std::int32_t top_k;  // <= 0: no cut
        float top_p;
    };

    class RowFinisher final
    {
    public:
        // Candidates as bf16 bits and token ids, in any order: every token
        // of the row whose logit is >= the k-th largest (or the whole row).
        // All logits must be finite.
        std::int32_t from_candidates(const std::uint16_t *bits, const std::int32_t *ids, std::int32_t count,
                                     const DrawRule &rule, double u);

        // A whole row of n logits; throws std::runtime_error for a
        // non-finite one.
        std::int32_t from_row(const std::uint16_t *row, std::int64_t n, const DrawRule &rule, double u);

    private:
        // ordered_[0, n) holds token ids best first; logit(i) their bits
        template <typename Logit>
        std::int32_t draw(std::int64_t n, Logit logit, const DrawRule &rule, double u);

        std::vector<std::uint32_t> buckets_;
        std::vector<std::int32_t> ordered_;
        std::vector<std::uint32_t> keyed_;
        std::vector<std::uint64_t> packed_;
        std::vector<double> running_;
    };
} // namespace qwen3::generation::detail
