// Host finish of one sampled row (see row_finish.hpp).
#include "row_finish.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace qwen3::generation::detail
{
    namespace
    {
        constexpr std::uint32_t kKeys = 1u << 16;

        // Larger key for a larger value; -0 and +0 share the key of +0.
        std::uint32_t order_key(std::uint16_t bits)
        {
            const std::uint32_t b = bits == 0x8000u ? 0u : bits;
            return (b & 0x8000u) != 0 ? (~b & 0xffffu) : (b | 0x8000u);
        }

        bool finite_bf16(std::uint16_t bits) { return (bits & 0x7f80u) != 0x7f80u; }

        float bf16_value(std::uint16_t bits)
        {
            const std::uint32_t w = static_cast<std::uint32_t>(bits) << 16;
            float f;
            std::memcpy(&f, &w, sizeof f);
            return f;
        }

        [[noreturn]] void non_finite() { throw std::runtime_error("temperature scaling produced a non-finite score"); }
    } // namespace

    template <typename Logit>
    std::int32_t RowFinisher::draw(std::int64_t n, Logit logit, const DrawRule &rule, double u)
    {
        const double t = static_cast<double>(rule.temperature);
        running_.resize(static_cast<std::size_t>(n));
        const double top = static_cast<double>(bf16_value(logit(0))) / t;
        double sum = 0.0;
        for (std::int64_t i = 0; i < n; ++i)
        {
            const double s = static_cast<double>(bf16_value(logit(i))) / t;
            sum += std::exp(s - top);
            running_[static_cast<std::size_t>(i)] = sum;
        }
        if (!std::isfinite(sum) || sum <= 0.0)
            throw std::runtime_error("sampler softmax weight sum is invalid");
        const auto first = running_.begin(), last = running_.begin() + n;
        // top-p: the shortest prefix whose weight reaches top_p of the total
        const double threshold = static_cast<double>(rule.top_p) * sum;
        const auto cut = std::lower_bound(first, last, threshold);
        const std::int64_t kept = cut == last ? n : (cut - first) + 1;
        // the draw over the kept prefix: first running sum above u * its weight
        const double r = u * running_[static_cast<std::size_t>(kept - 1)];
        const auto hit = std::upper_bound(first, first + kept, r);
        const std::int64_t pick = hit == first + kept ? kept - 1 : hit - first;
        return ordered_[static_cast<std::size_t>(pick)];
    }

    std::int32_t RowFinisher::from_candidates(const std::uint16_t *bits, const std::int32_t *ids, std::int32_t count,
                                              const DrawRule &rule, double u)
    {
        if (count <= 0)
            throw std::logic_error("sampling row has no candidates");
        // (key, position) packed so that one descending sort gives key order,
        // then ascending id among equal keys
        const auto m = static_cast<std::size_t>(count);
        keyed_.resize(m);
        packed_.resize(m);
        for (std::size_t i = 0; i < m; ++i)
            packed_[i] = (static_cast<std::uint64_t>(order_key(bits[i])) << 32) |
                         (0xffffffffu - static_cast<std::uint32_t>(ids[i]));
        std::sort(packed_.begin(), packed_.end(), [](std::uint64_t a, std::uint64_t b) { return a > b; });
        ordered_.resize(m);
        for (std::size_t i = 0; i < m; ++i)
        {
            ordered_[i] = static_cast<std::int32_t>(0xffffffffu - static_cast<std::uint32_t>(packed_[i]));
            keyed_[i] = static_cast<std::uint32_t>(packed_[i] >> 32);
        }
        // the top-k cut (a no-op for a candidate set that is exactly the top-k set)
        std::int64_t n = count;
        if (rule.top_k > 0 && rule.top_k < count)
        {
            const std::uint32_t kth = keyed_[static_cast<std::size_t>(rule.top_k - 1)];
            while (n > rule.top_k && keyed_[static_cast<std::size_t>(n - 1)] < kth)
                --n;
        }
        // bits of the ordered candidates, by key (the key determines the value
        // up to the sign of zero, which the score ignores)
        return draw(
            n,
            [this](std::int64_t i) {
                const std::uint32_t k = keyed_[static_cast<std::size_t>(i)];
                return static_cast<std::uint16_t>((k & 0x8000u) != 0 ? (k & 0x7fffu) : (~k & 0xffffu));
            },
            rule, u);
    }

    std::int32_t RowFinisher::from_row(const std::uint16_t *row, std::int64_t n, const DrawRule &rule, double u)
    {
        if (n <= 0)
            throw std::logic_error("sampling row is empty");
        buckets_.assign(kKeys, 0u);
        for (std::int64_t t = 0; t < n; ++t)
        {
            if (!finite_bf16(row[t]))
                non_finite();
            ++buckets_[order_key(row[t])];
        }
        // lowest key kept: the bucket where the count from the top reaches k
        std::uint32_t floor_key = 0;
        std::int64_t kept = n;
        if (rule.top_k > 0 && rule.top_k < n)
        {
            std::int64_t seen = 0;
            for (std::uint32_t k = kKeys; k-- > 0;)
            {
                seen += buckets_[k];
                if (seen >= rule.top_k)
                {
                    floor_key = k;
                    kept = seen;
                    break;
                }
            }
        }
        // bucket starts, best key first, then a stable scatter by token id
        std::uint32_t at = 0;
        for (std::uint32_t k = kKeys; k-- > floor_key;)
        {
            const std::uint32_t c = buckets_[k];
            buckets_[k] = at;
            at += c;
        }
        ordered_.resize(static_cast<std::size_t>(kept));
        for (std::int64_t t = 0; t < n; ++t)
        {
            const std::uint32_t k = order_key(row[t]);
            if (k >= floor_key)
                ordered_[buckets_[k]++] = static_cast<std::int32_t>(t);
        }
        return draw(kept, [&](std::int64_t i) { return row[ordered_[static_cast<std::size_t>(i)]]; }, rule, u);
    }
} // namespace qwen3::generation::detail
