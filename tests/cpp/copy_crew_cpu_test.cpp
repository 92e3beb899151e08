// The staging copy crew of the safetensors loader (qwen3::detail::CopyCrew):
// every byte lands for sizes around the 4 KiB part boundaries, for 0 to 7
// helpers, over many copies per crew, and crews start and stop cleanly.
// Also built under ThreadSanitizer by the sanitizer test.
#include "qwen3/io/copy_crew.h"
#include "test_util.hpp"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace
{
    void body()
    {
        std::vector<std::uint8_t> src(1024u * 1024u + 4099u), dst(src.size()), want(src.size());
        std::uint32_t s = 12345u;
        for (auto &b : src)
        {
            s = s * 1664525u + 1013904223u;
            b = static_cast<std::uint8_t>(s >> 24);
        }
        const std::size_t sizes[] = {0, 1, 4095, 4096, 4097, 3 * 4096 + 5, 8 * 4096, 65536 + 3, src.size()};
        for (unsigned helpers : {0u, 1u, 3u, 7u})
        {
            qwen3::detail::CopyCrew crew(helpers);
            test::require(crew.helpers() == helpers, "helper count");
            for (int round = 0; round < 3; ++round)
                for (std::size_t n : sizes)
                {
                    const std::size_t offset = (round * 977u) % 61u;   // unaligned source and destination
                    const std::size_t len = std::min(n, src.size() - offset);
                    std::fill(dst.begin(), dst.end(), std::uint8_t{0xAB});
                    std::fill(want.begin(), want.end(), std::uint8_t{0xAB});
                    std::memcpy(want.data() + offset, src.data() + offset, len);
                    crew.copy(dst.data() + offset, src.data() + offset, len);
                    test::require(std::memcmp(dst.data(), want.data(), dst.size()) == 0,
                                  "a " + std::to_string(len) + "-byte copy at offset " + std::to_string(offset) +
                                      " with " + std::to_string(helpers) + " helpers");
                }
        }
        for (int i = 0; i < 20; ++i)   // crews that never copy still stop
            qwen3::detail::CopyCrew idle(3);
    }
} // namespace

int main() { return test::run("copy crew CPU test", body); }
