// Launch geometry of the kernels and the grid limit of one dispatch, kept
// free of HIP so that host-side tests can check the dispatch decisions.
//
// The dispatch packet holds the grid size in work-items, 32 bits per
// dimension, so blocks x threads-per-block must stay below 2^32.  Each
// launcher asks the helper of its kernel family whether the fast kernel's
// grid fits; when it does not, the launcher takes the family's grid-stride
// kernel, whose grid is capped and which loops over any count.
#pragma once

#include <stdint.h>

namespace q3k
{
    constexpr int kWave = 64;

    // Blocks of 256 threads (four waves) unless stated otherwise.
    constexpr int kBlock = 256;

    // A launch that writes at most this many bytes is small (a decode step):
    // its kernels take their small-launch shapes and store policy.  Config 3's
    // decode launches write 0.5-1.5 MB; config 2's (T = 512) Q/K norm + RoPE
    // and SwiGLU write 3 MB and run faster in their large-launch shapes (the
    // config-2 chain replayed from a HIP graph: 12.4 against 13.65 us per step
    // with a 4 MiB bound; a 1 MiB bound slowed the decode step by 0.3 us).
    constexpr int64_t kSmallLaunchBytes = int64_t{2} << 20;

    // Whether `blocks` blocks of `threads` threads fit one dispatch.
    inline bool launch_fits(int64_t blocks, int64_t threads)
    {
        return threads > 0 && blocks > 0 && blocks <= static_cast<int64_t>(UINT32_MAX) / threads;
    }

    // Blocks for `units` units of work, `per_block` a block.
    inline int64_t blocks_for(int64_t units, int64_t per_block) { return units / per_block + (units % per_block != 0); }

    // Element-wise vector kernels: 8 elements a lane, `unroll` vectors a
    // lane, one block for an input of fewer than 8 elements.
    inline int64_t binary_vec_blocks(int64_t n, int unroll, int block = kBlock)
    {
        const int64_t blocks = blocks_for(n / 8, static_cast<int64_t>(block) * unroll);
        return blocks > 0 ? blocks : 1;
    }
    inline bool binary_vec_fits(int64_t n, int unroll, int block = kBlock)
    {
        return launch_fits(binary_vec_blocks(n, unroll, block), block);
    }

    // Embedding gather: blocks of four waves, 1, 2 or 4 waves a token (rows
    // of up to 128, 256 or more 128-bit vectors), kEmbeddingVectorsPerLane
    // vectors a lane per pass over the row.
    constexpr int kEmbeddingBlock = 4 * kWave;
    constexpr int kEmbeddingVectorsPerLane = 2;
    inline int embedding_waves_per_token(int64_t nvec)
    {
        const int64_t per_wave = static_cast<int64_t>(kWave) * kEmbeddingVectorsPerLane;
        return nvec > 2 * per_wave ? 4 : nvec > per_wave ? 2 : 1;
    }
    inline bool embedding_vec_fits(int64_t tokens, int waves_per_token)
    {
        return tokens >= 0 && tokens <= INT64_MAX / 4 &&
               launch_fits(blocks_for(tokens * waves_per_token, kEmbeddingBlock / kWave), kEmbeddingBlock);
    }

    // RMSNorm, several rows a block: groups of `group` lanes, one row each.
    // Narrow RMSNorm rows: a group of `group` lanes a row, `block` lanes a
    // block (kRmsRowsBlock unless a launch asks for more).
    constexpr int kRmsRowsBlock = kWave;
    inline bool rms_rows_fit(int64_t rows, int group, int block = kRmsRowsBlock)
    {
        return launch_fits(blocks_for(rows, block / group), block);
    }
    // RMSNorm, one row a block of `waves` waves.
    inline bool rms_block_fits(int64_t rows, int waves) { return launch_fits(rows, static_cast<int64_t>(waves) * kWave); }

    // RoPE / Q-K norm + RoPE over (token, head) rows of 128 elements: 16
    // lanes a head, so four heads a wave at one head per lane group, the
    // most waves any head grouping launches.  The kernel also indexes rows
    // with 32-bit wave-uniform arithmetic, hence rows < 2^31.
    constexpr int kRopeHeadsPerWave = kWave / 16;
    constexpr int kRopeWavesPerBlock = 4;
    constexpr int kRopeBlock = kRopeWavesPerBlock * kWave;
    inline bool rope_heads_fit(int64_t tokens, int64_t heads)
    {
        if (tokens < 0 || heads <= 0 || tokens > (int64_t{1} << 31) / heads)
            return false;
        const int64_t rows = tokens * heads;
        return rows < (int64_t{1} << 31) &&
               launch_fits(blocks_for(blocks_for(rows, kRopeHeadsPerWave), kRopeWavesPerBlock), kRopeBlock);
    }
} // namespace q3k
