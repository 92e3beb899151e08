// The kernel choices of the RoPE / Q-K norm + RoPE and attention launchers
// (csrc/kernels/dispatch.hpp), decided on the host: every head layout of the
// Qwen3 family, and of one rank of its 8-way tensor-parallel shards, must take
// the fast kernels (rope_heads_kernel; the matrix-core attention kernel with
// the compiled group size where there is one), the generic kernels only the
// shapes they exist for (head_dim other than 128, unaligned or strided
// tensors), and decode-sized launches their small-launch shapes.
#include "../../qwen3-runtime-byyourself_amd/csrc/kernels/dispatch.hpp"
#include "test_util.hpp"

#include <string>

using test::require;

namespace
{
    struct Heads
    {
        int32_t hq, hkv;
    };
    // Qwen3 0.6B/1.7B, 4B/8B, 14B, 32B; one rank of 8-way tensor parallelism of each
    constexpr Heads kFamily[] = {{16, 8}, {32, 8}, {40, 8}, {64, 8}, {2, 1}, {4, 1}, {5, 1}, {8, 1}};

    std::string tag(const Heads &h) { return std::to_string(h.hq) + "/" + std::to_string(h.hkv); }

    void rope_cases()
    {
        using namespace q3k;
        for (const Heads &h : kFamily)
        {
            for (const int64_t tokens : {int64_t{8192}, int64_t{512}, int64_t{64}, int64_t{1}})
            {
                const std::string what = "Q/K norm + RoPE " + tag(h) + " tokens " + std::to_string(tokens);
                const RopePlan p = plan_rope(tokens, h.hq, h.hkv, 128, true);
                require(p.fast, what + ": generic kernels chosen");
                const int any = (h.hq % 4 != 0 ? 1 : 0) | (h.hkv % 4 != 0 ? 2 : 0);
                require(p.any_heads == any, what + ": rows per lane group only for head counts not a multiple of 4");
                const bool small = tokens * (h.hq + h.hkv) < kRopeSmallLaunchRows;
                if (any != 0)
                {
                    require(p.hg_q == 1 && p.hg_k == 1, what + ": one head per lane group");
                    continue;
                }
                const int want_q = small ? 1 : (h.hq % 16 == 0 ? 4 : h.hq % 8 == 0 ? 2 : 1);
                const int want_k = small ? 1 : (h.hkv % 16 == 0 ? 4 : h.hkv % 8 == 0 ? 2 : 1);
                require(p.hg_q == want_q && p.hg_k == want_k, what + ": heads per lane");
                // apply_rope_inplace's single launch over Q and K, and one tensor alone
                const RopePlan r = plan_rope(tokens, h.hq, 0, 128, true);
                require(r.fast && r.hg_k == r.hg_q, what + ": one-tensor RoPE");
            }
        }
        // config 4 (8B prefill): 4 heads per lane for the 32 query heads, 2 for the 8 KV heads;
        // config 3 (decode, 64 tokens): one head per lane group
        const RopePlan c4 = plan_rope(8192, 32, 8, 128, true);
        require(c4.fast && c4.hg_q == 4 && c4.hg_k == 2 && c4.any_heads == 0, "config 4 instance");
        const RopePlan c3 = plan_rope(64, 32, 8, 128, true);
        require(c3.fast && c3.small && c3.hg_q == 1 && c3.hg_k == 1, "config 3 instance");
        // config 2 (0.6B prefill, 512 tokens, 16 + 8 heads: 3 MB written) takes the large-launch shapes
        const RopePlan c2 = plan_rope(512, 16, 8, 128, true);
        require(c2.fast && !c2.small && c2.hg_q == 4 && c2.hg_k == 2, "config 2 instance");
        // the generic kernels: head_dim 64, an unaligned tensor or table, rows past 2^31
        require(!plan_rope(8192, 32, 8, 64, true).fast, "head_dim 64 took the fast kernel");
        require(!plan_rope(8192, 32, 8, 128, false).fast, "unaligned tensors took the fast kernel");
        // the grid of one head per lane group: 10 waves a token at 32/8 heads, four waves a block, at most
        // 2^32 - 1 work-items: 6710886 tokens fit, one more does not
        require(plan_rope(6710886, 32, 8, 128, true).fast, "the largest grid rejected");
        require(!plan_rope(6710887, 32, 8, 128, true).fast, "a grid past one dispatch took the fast kernel");
        require(!plan_rope((int64_t{1} << 31) / 32, 32, 0, 128, true).fast, "rows past 2^31 took the fast kernel");
    }

    void attention_cases()
    {
        using namespace q3k;
        for (const Heads &h : kFamily)
        {
            const int32_t G = h.hq / h.hkv;
            const int want_g = (G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32) ? G : 0;
            // prefill (B 4 x 2048, cache [B, L, Hkv, D]) and a decode step over 4096 cached keys
            for (const bool decode : {false, true})
            {
                const int64_t B = decode ? 1 : 4, S = decode ? 1 : 2048, start = decode ? 4095 : 0, L = start + S;
                const int64_t st[4] = {L * h.hkv * 128, h.hkv * 128, 128, 1};
                const std::string what = std::string(decode ? "decode " : "prefill ") + tag(h);
                const AttnSplit split = plan_attention_split(B, S, h.hq, h.hkv, L);
                const AttnPlan p = plan_attention(B, S, h.hq, h.hkv, 128, start, st, st, true, split.bytes, true);
                require(p.mfma, what + ": generic kernel chosen");
                require(p.g_instance == want_g, what + ": group-size instance");
                require(p.split.splits == split.splits, what + ": the workspace the library asks for splits the keys");
                if (decode)
                {
                    require(p.split.splits > 1, what + ": a one-sequence decode step is not split");
                    require(p.waves == (p.split.split_keys <= kAttMaxOneWaveSplitKeys ? 1 : kAttWavesPerBlock),
                            what + ": one-wave slices");
                    // without a workspace: one unsplit launch
                    const AttnPlan n = plan_attention(B, S, h.hq, h.hkv, 128, start, st, st, true, 0, false);
                    require(n.mfma && n.split.splits == 1 && n.waves == kAttWavesPerBlock, what + ": unsplit form");
                }
                else
                {
                    require(split.bytes == 0 || h.hkv == 1, what + ": prefill of 4 x 2048 split");
                }
            }
        }
        const int64_t st[4] = {2048 * 8 * 128, 8 * 128, 128, 1};
        // the generic kernel: head_dim 64, unit-stride dims missing, unaligned rows, too many query heads per KV head
        const int64_t st64[4] = {2048 * 8 * 64, 8 * 64, 64, 1};
        require(!plan_attention(4, 2048, 32, 8, 64, 0, st64, st64, true, 0, false).mfma, "head_dim 64 on matrix cores");
        const int64_t strided[4] = {2048 * 8 * 256, 8 * 256, 256, 2};
        require(!plan_attention(4, 2048, 32, 8, 128, 0, strided, strided, true, 0, false).mfma, "dim stride 2");
        require(!plan_attention(4, 2048, 32, 8, 128, 0, st, st, false, 0, false).mfma, "unaligned pointers");
        const int64_t odd[4] = {2048 * 8 * 128 + 4, 8 * 128, 128, 1};
        require(!plan_attention(4, 2048, 32, 8, 128, 0, odd, st, true, 0, false).mfma, "16-byte-unaligned batch stride");
        require(!plan_attention(1, 64, 64, 1, 128, 0, st, st, true, 0, false).mfma, "group size 64");
        // a workspace that is too small or unaligned leaves the decode step unsplit
        const int64_t dst[4] = {4096 * 8 * 128, 8 * 128, 128, 1};
        const AttnSplit need = plan_attention_split(1, 1, 32, 8, 4096);
        require(need.splits > 1, "decode split plan");
        require(plan_attention(1, 1, 32, 8, 128, 4095, dst, dst, true, need.bytes - 1, true).split.splits == 1,
                "a short workspace used");
        require(plan_attention(1, 1, 32, 8, 128, 4095, dst, dst, true, need.bytes, false).split.splits == 1,
                "an unaligned workspace used");
    }

    void body()
    {
        rope_cases();
        attention_cases();
    }
} // namespace

int main() { return test::run("dispatch decisions test", body); }
