// The grid decisions of the kernel launchers (csrc/kernels/launch_limits.hpp)
// at their boundaries.  One dispatch holds at most 2^32 - 1 work-items per
// grid dimension; each fast kernel must be chosen only while its grid stays
// within that, and its launcher takes the grid-stride kernel (or, for
// attention, reports Q3K_ERR_OVERFLOW) past it.  The arithmetic must not
// overflow for any int64 count.
#include "../../qwen3-runtime-byyourself_amd/csrc/kernels/launch_limits.hpp"
#include "test_util.hpp"

#include <cstdint>
#include <limits>

using test::require;

namespace
{
    constexpr int64_t kMaxItems = 4294967295LL;   // 2^32 - 1
    constexpr int64_t kMax256 = kMaxItems / 256;  // 16777215 blocks of 256 threads

    void body()
    {
        using namespace q3k;
        const int64_t big = std::numeric_limits<int64_t>::max();

        // the limit itself
        require(launch_fits(1, 256) && launch_fits(kMax256, 256), "largest 256-thread grid rejected");
        require(kMax256 * 256 <= kMaxItems && (kMax256 + 1) * 256 > kMaxItems, "boundary arithmetic");
        require(!launch_fits(kMax256 + 1, 256), "grid of 2^32 work-items accepted");
        require(launch_fits(kMaxItems / 1024, 1024) && !launch_fits(kMaxItems / 1024 + 1, 1024), "1024-thread boundary");
        require(launch_fits(kMaxItems, 1), "one-thread boundary");
        require(!launch_fits(0, 256) && !launch_fits(-1, 256) && !launch_fits(big, 256) && !launch_fits(4, 0),
                "empty, negative or huge grid accepted");

        require(blocks_for(0, 4) == 0 && blocks_for(1, 4) == 1 && blocks_for(4, 4) == 1 && blocks_for(5, 4) == 2,
                "blocks_for rounding");
        require(blocks_for(big, 2) == big / 2 + 1 && blocks_for(big, 1) == big, "blocks_for overflows");

        // element-wise: 8 elements a lane, 256 lanes a block (the default), `unroll` vectors a lane
        for (int unroll : {1, 2, 4})
        {
            const int64_t per_block = 8LL * 256 * unroll;
            const int64_t last = per_block * kMax256;
            require(binary_vec_blocks(1, unroll) == 1 && binary_vec_blocks(7, unroll) == 1, "short input: one block");
            require(binary_vec_fits(last, unroll), "largest element-wise grid rejected");
            require(binary_vec_fits(last + 7, unroll), "the partial vector after the last lane needs no block");
            require(!binary_vec_fits(last + 8, unroll), "element-wise grid past 2^32 work-items accepted");
            require(!binary_vec_fits(big, unroll), "huge element-wise input accepted");
        }
        // the large launches' one-wave blocks: the same 2^32 work-item limit
        {
            const int64_t max64 = static_cast<int64_t>(UINT32_MAX) / 64;
            const int64_t last = 8LL * 64 * max64;
            require(binary_vec_blocks(last, 1, 64) == max64, "one-wave block count");
            require(binary_vec_fits(last, 1, 64) && binary_vec_fits(last + 7, 1, 64), "largest one-wave grid rejected");
            require(!binary_vec_fits(last + 8, 1, 64), "one-wave grid past 2^32 work-items accepted");
            require(binary_vec_blocks(1, 1, 64) == 1, "short input: one one-wave block");
        }

        // embedding: 1, 2 or 4 waves a token in four-wave blocks
        require(kEmbeddingBlock == 256 && kEmbeddingVectorsPerLane == 2, "embedding geometry");
        require(embedding_waves_per_token(128) == 1 && embedding_waves_per_token(129) == 2 &&
                    embedding_waves_per_token(256) == 2 && embedding_waves_per_token(257) == 4 &&
                    embedding_waves_per_token(512) == 4 && embedding_waves_per_token(1) == 1,
                "embedding waves per token");
        for (int wpt : {1, 2, 4})
        {
            const int64_t tokens = 4 * kMax256 / wpt;
            require(embedding_vec_fits(tokens, wpt) && !embedding_vec_fits(tokens + 1, wpt),
                    "embedding boundary, waves per token " + std::to_string(wpt));
            require(!embedding_vec_fits(big, wpt), "huge embedding accepted");
        }

        // RMSNorm: rows in lane groups (one-wave blocks by default, four-wave
        // blocks where a launch asks for them), or one row a block of 1..8 waves
        require(kRmsRowsBlock == 64, "rms rows geometry");
        const int64_t max64 = kMaxItems / 64;
        for (int group : {1, 2, 4, 8, 16, 32, 64})
        {
            const int64_t rows = static_cast<int64_t>(64 / group) * max64;
            require(rms_rows_fit(rows, group) && !rms_rows_fit(rows + 1, group),
                    "rms rows boundary, group " + std::to_string(group));
            const int64_t rows256 = static_cast<int64_t>(256 / group) * kMax256;
            require(rms_rows_fit(rows256, group, 256) && !rms_rows_fit(rows256 + 1, group, 256),
                    "rms rows boundary (four-wave blocks), group " + std::to_string(group));
        }
        for (int waves = 1; waves <= 8; ++waves)
        {
            const int64_t rows = kMaxItems / (64LL * waves);
            require(rms_block_fits(rows, waves) && !rms_block_fits(rows + 1, waves),
                    "rms block boundary, waves " + std::to_string(waves));
        }
        require(!rms_rows_fit(big, 1) && !rms_block_fits(big, 1), "huge row count accepted");

        // RoPE heads: four (token, head) rows a wave, four waves a block
        require(kRopeHeadsPerWave == 4 && kRopeWavesPerBlock == 4, "rope geometry");
        const int64_t rope_rows = 16 * kMax256;   // 268435440
        require(rope_heads_fit(rope_rows / 8, 8) && rope_heads_fit(rope_rows / 40, 40), "largest rope grid rejected");
        require(!rope_heads_fit(8388608, 32), "rope grid of 2^32 work-items accepted (2^28 rows)");
        require(rope_heads_fit(8388607, 32), "rope rows just under the limit rejected");
        require(!rope_heads_fit(big, 64) && !rope_heads_fit(1LL << 40, 64) && !rope_heads_fit(1, 0) &&
                    !rope_heads_fit(-1, 8),
                "huge, empty-head or negative rope input accepted");
        std::cout << "launch limits checked\n";
    }
} // namespace

int main() { return test::run("launch limits (CPU) test", body); }
