// The sampler's row crew (csrc/generation/row_crew.hpp): every part of a run
// runs exactly once, run returns only after all parts are done, an exception
// from any part reaches the caller and leaves the crew usable, and the crew
// serves many runs with varying part counts.  Also built under
// ThreadSanitizer by tests/test_cpp_sanitizers.py.
#include "../../qwen3-runtime-byyourself_amd/csrc/generation/row_crew.hpp"
#include "test_util.hpp"

#include <atomic>
#include <stdexcept>
#include <vector>

using qwen3::generation::detail::RowCrew;
using test::require;

namespace
{
    void body()
    {
        RowCrew crew;
        std::vector<int> hits(RowCrew::kMaxParts, 0);
        long long total = 0;
        for (int round = 0; round < 2000; ++round)
        {
            const int parts = 1 + round % RowCrew::kMaxParts;
            std::vector<int> seen(RowCrew::kMaxParts, 0);
            crew.run(parts, [&](int part) { seen[static_cast<std::size_t>(part)] += 1; });
            for (int p = 0; p < RowCrew::kMaxParts; ++p)
                require(seen[static_cast<std::size_t>(p)] == (p < parts ? 1 : 0), "a part ran other than once");
            total += parts;
        }
        require(total == 5000, "part count");
        // the caller's part and a helper's part each throw; the first error reaches the caller
        for (int thrower : {0, 1, 3})
        {
            std::atomic<int> ran{0};
            bool caught = false;
            try
            {
                crew.run(4, [&](int part) {
                    ran.fetch_add(1);
                    if (part == thrower)
                        throw std::runtime_error("part failed");
                });
            }
            catch (const std::runtime_error &)
            {
                caught = true;
            }
            require(caught, "a part's exception was lost");
            require(ran.load() == 4, "run returned before every part had run");
        }
        // usable after an exception; more parts than the crew has are capped
        std::atomic<int> ran{0};
        crew.run(9, [&](int) { ran.fetch_add(1); });
        require(ran.load() == RowCrew::kMaxParts, "parts capped at the crew's maximum");
        // a crew that never started a helper, and one destroyed right after a run
        {
            RowCrew idle;
        }
        {
            RowCrew brief;
            std::atomic<int> n{0};
            brief.run(4, [&](int) { n.fetch_add(1); });
            require(n.load() == 4, "brief crew");
        }
        std::cout << "row crew checked\n";
    }
} // namespace

int main() { return test::run("row crew (CPU) test", body); }
