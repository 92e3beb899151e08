// Which kernel, and which instance of it, the RoPE / Q-K norm + RoPE and the
// attention launchers take for a given shape, as host functions free of HIP.
// The launchers call these and nothing else to decide, so a host test can
// check every decision (each head layout of the Qwen3 family and of its
// tensor-parallel shards) without a GPU.
#pragma once

#include "launch_limits.hpp"

namespace q3k
{
    // ---- RoPE and Q/K norm + RoPE over [tokens, heads, 128] rows ------------

    constexpr int kRopeHeadDim = 128;
    // Below this many (token, head) rows (kSmallLaunchBytes of 256-byte rows)
    // a launch is small (decode): one head per lane group, so more and
    // shorter waves fill more CUs, and write-through stores.
    constexpr int64_t kRopeSmallLaunchRows = kSmallLaunchBytes / (2 * kRopeHeadDim);

    struct RopePlan
    {
        bool fast = false; // rope_heads_kernel; otherwise the generic kernels
        int hg_q = 1;      // heads per lane of Q's waves (1, 2 or 4)
        int hg_k = 1;      // heads per lane of K's waves
        int any_heads = 0; // bit 0 (Q) / bit 1 (K): head count not a multiple of 4, rows per lane group
        bool small = false; // a small launch: write-through stores
    };

    // Waves over a tensor's rows, hg heads per lane; the last one partial when
    // the head count is not a multiple of 4 hg.
    inline int64_t rope_waves(int64_t tokens, int32_t heads, int hg)
    {
        return blocks_for(tokens * heads, static_cast<int64_t>(kRopeHeadsPerWave) * hg);
    }

    // 4 heads per lane when the head count allows it (32 or 64 query heads),
    // else 2 (8 KV heads), else 1.
    inline int rope_heads_per_lane(int32_t heads) { return heads % 16 == 0 ? 4 : heads % 8 == 0 ? 2 : 1; }

    // Every tensor's rows below 2^31 and the grid of the most waves the
    // launcher makes (one head per lane group) within one dispatch.
    inline bool rope_grid_ok(int64_t tokens, int32_t hq, int32_t hk)
    {
        if (!rope_heads_fit(tokens, hq) || (hk > 0 && !rope_heads_fit(tokens, hk)) || !rope_heads_fit(tokens, hq + hk))
            return false;
        const int64_t waves = rope_waves(tokens, hq, 1) + rope_waves(tokens, hk, 1);
        return launch_fits(blocks_for(waves, kRopeWavesPerBlock), kRopeBlock);
    }

    // hk = 0 for one tensor (q3k_rope_bf16).  aligned: every tensor, the table
    // and the norm weights 16-byte aligned.  A head count that is not a
    // multiple of 4 takes one row per lane group, with per-row tokens and
    // positions.  (Two or four such rows per lane group, every load first,
    // did not pay at config 4's tensor-parallel-8 shards: Q/K norm + RoPE at
    // 4/1 heads 7.0 and 8.1 us against 7.2 us with one row, at 8/1 heads
    // 11.3 and 12.1 us against 10.0 us.)
    inline RopePlan plan_rope(int64_t tokens, int32_t hq, int32_t hk, int32_t head_dim, bool aligned)
    {
        RopePlan p;
        if (head_dim != kRopeHeadDim || !aligned || hq <= 0 || hk < 0 || !rope_grid_ok(tokens, hq, hk))
            return p;
        p.fast = true;
        const bool small = tokens * (static_cast<int64_t>(hq) + hk) < kRopeSmallLaunchRows;
        p.small = small;
        p.any_heads = (hq % kRopeHeadsPerWave != 0 ? 1 : 0) | (hk > 0 && hk % kRopeHeadsPerWave != 0 ? 2 : 0);
        if (p.any_heads != 0)
            return p;
        p.hg_q = small ? 1 : rope_heads_per_lane(hq);
        p.hg_k = small ? 1 : (hk == 0 ? p.hg_q : rope_heads_per_lane(hk));
        return p;
    }

    // ---- grouped-query attention ---------------------------------------------

    constexpr int kAttHeadDim = 128;
    constexpr int kAttKeyTile = 64;               // keys per pipeline step
    constexpr int kAttWavesPerBlock = 4;          // waves of a matrix-core block
    constexpr int kAttColsPerWave = 32;           // (position, head) columns of a wave
    constexpr int kAttMaxSplits = 64;             // key slices the combine kernel merges
    // Below this many blocks the grid leaves CUs idle and the key range is
    // split; a slice keeps at least two tiles, or one for a decode step (one
    // query position), whose slices of up to two tiles run as one-wave blocks:
    // the four-wave block computes one position in one wave, so each slice
    // then takes a wave of its own instead of a block (B 1 x 4096 keys: 8.7
    // against 10.3 us; from B 4 the four-wave blocks, which share each tile's
    // loads, are as fast or faster).
    constexpr int64_t kAttSplitTargetBlocks = 512;
    constexpr int32_t kAttMinSplitKeys = 2 * kAttKeyTile;
    constexpr int32_t kAttMinDecodeSplitKeys = kAttKeyTile;
    constexpr int32_t kAttMaxOneWaveSplitKeys = 2 * kAttKeyTile;

    struct AttnSplit
    {
        int32_t splits = 1;
        int32_t split_keys = INT32_MAX;
        int64_t bytes = 0; // workspace: unnormalised O^T, max and sum of each slice, fp32
    };

    inline AttnSplit plan_attention_split(int64_t B, int64_t S, int32_t Hq, int32_t Hkv, int64_t cached)
    {
        AttnSplit p;
        const int32_t G = Hq / Hkv;
        const int64_t cols = S * G, block_cols = static_cast<int64_t>(kAttColsPerWave) * kAttWavesPerBlock;
        const int64_t blocks = B * Hkv * blocks_for(cols, block_cols);
        const int32_t min_keys = S == 1 ? kAttMinDecodeSplitKeys : kAttMinSplitKeys;
        if (blocks >= kAttSplitTargetBlocks || cached < 2 * static_cast<int64_t>(min_keys))
            return p;
        int64_t want = blocks_for(kAttSplitTargetBlocks, blocks);
        const int64_t most = cached / min_keys;
        if (want > most)
            want = most;
        if (want > kAttMaxSplits)
            want = kAttMaxSplits;
        if (want < 2)
            return p;
        const int64_t keys = blocks_for(blocks_for(cached, want), kAttKeyTile) * kAttKeyTile;
        p.splits = static_cast<int32_t>(blocks_for(cached, keys));
        p.split_keys = static_cast<int32_t>(keys);
        if (p.splits < 2)
            return AttnSplit{};
        p.bytes = static_cast<int64_t>(p.splits) * B * S * Hq * (kAttHeadDim + 2) * 4;
        return p;
    }

    struct AttnPlan
    {
        bool mfma = false;   // attn_mfma_kernel; otherwise attn_generic_kernel
        int g_instance = 0;  // the compiled group size (1, 2, 4, 8, 16, 32), or 0: taken at run time
        int waves = kAttWavesPerBlock; // waves per block (1: one-wave decode slices)
        AttnSplit split;     // splits > 1: the key range is split and attn_combine_kernel merges
    };

    // ks / vs: element strides (batch, position, head, dim) of the K / V
    // views.  aligned: q, k and v 16-byte aligned and out 8-byte aligned.
    // workspace_bytes: what the caller passes (0 without a workspace), and
    // whether that workspace is 16-byte aligned.
    inline AttnPlan plan_attention(int64_t B, int64_t S, int32_t Hq, int32_t Hkv, int32_t D, int64_t start,
                                   const int64_t ks[4], const int64_t vs[4], bool aligned, int64_t workspace_bytes,
                                   bool workspace_aligned)
    {
        AttnPlan p;
        if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0)
            return p;
        const int32_t G = Hq / Hkv;
        // tile loads use 32-bit byte offsets of up to kAttKeyTile rows
        const int64_t row_limit = (INT32_MAX - 2 * kAttHeadDim) / (2 * kAttKeyTile);
        p.mfma = G >= 1 && G <= kAttColsPerWave && D == kAttHeadDim && start + S <= INT32_MAX && ks[1] <= row_limit &&
                 vs[1] <= row_limit && ks[3] == 1 && vs[3] == 1 && ks[0] % 8 == 0 && ks[1] % 8 == 0 &&
                 ks[2] % 8 == 0 && vs[0] % 8 == 0 && vs[1] % 8 == 0 && vs[2] % 8 == 0 && aligned;
        if (!p.mfma)
            return p;
        p.g_instance = (G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32) ? G : 0;
        const AttnSplit split = plan_attention_split(B, S, Hq, Hkv, start + S);
        if (split.splits > 1 && split.splits <= kAttMaxSplits && workspace_bytes >= split.bytes && workspace_aligned)
            p.split = split;
        if (p.split.splits > 1 && S == 1 && p.split.split_keys <= kAttMaxOneWaveSplitKeys)
            p.waves = 1;
        return p;
    }
} // namespace q3k
