// Helpers of the C++ tests: check macros in the style of the reference's
// unit tests (require / require_throws; a failing check throws and main()
// returns EXIT_FAILURE), bf16 helpers, seeded inputs and the oracle band
// comparison.
#pragma once

#include "q3k_oracle.h"

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace test
{
    inline void require(bool condition, const std::string &message)
    {
        if (!condition)
            throw std::runtime_error(message);
    }

    template <typename Exception, typename F>
    void require_throws(F &&f, const std::string &message)
    {
        bool caught = false;
        try
        {
            f();
        }
        catch (const Exception &)
        {
            caught = true;
        }
        require(caught, message);
    }

    inline uint16_t bf16(float v) { return q3o_bf16_from_f32(v); }
    inline float f32(uint16_t v) { return q3o_f32_from_bf16(v); }

    // Deterministic values in roughly N(0, scale) (sum of uniforms), rounded to bf16.
    inline std::vector<uint16_t> values(std::size_t n, uint64_t seed, float scale = 1.0f, float offset = 0.0f)
    {
        std::vector<uint16_t> out(n);
        uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
        for (std::size_t i = 0; i < n; ++i)
        {
            float acc = 0.0f;
            for (int k = 0; k < 4; ++k)
            {
                s ^= s << 13;
                s ^= s >> 7;
                s ^= s << 17;
                acc += static_cast<float>(s >> 40) / static_cast<float>(1ull << 24);
            }
            out[i] = bf16(offset + scale * (acc - 2.0f) * 1.7320508f);
        }
        return out;
    }

    // Every element inside the oracle band widened by one bf16 ulp.
    inline void require_band(const std::vector<uint16_t> &got, const std::vector<uint16_t> &primary,
                             const std::vector<uint16_t> &lo, const std::vector<uint16_t> &hi, const std::string &what)
    {
        require(got.size() == primary.size(), what + ": size mismatch");
        int64_t stats[8];
        q3o_compare_band(got.data(), primary.data(), lo.data(), hi.data(), static_cast<int64_t>(got.size()), stats);
        if (stats[1] != 0)
        {
            const int64_t i = stats[2];
            throw std::runtime_error(what + ": " + std::to_string(stats[1]) + " elements outside the 1-ulp band, first at " +
                                     std::to_string(i) + " got " + std::to_string(f32(got[i])) + " expected " +
                                     std::to_string(f32(primary[i])));
        }
    }

    inline int run(const char *name, void (*body)())
    {
        try
        {
            body();
            std::cout << name << " passed.\n";
            return EXIT_SUCCESS;
        }
        catch (const std::exception &error)
        {
            std::cerr << name << " failed: " << error.what() << '\n';
            return EXIT_FAILURE;
        }
    }
} // namespace test
