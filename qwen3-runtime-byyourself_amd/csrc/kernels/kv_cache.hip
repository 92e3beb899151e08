// KV-cache append for gfx950: the current K and V projections [B, S, row]
// go to rows start .. start + S - 1 of every batch row of one layer's
// [batch_cap, seq_cap, row] cache (src/model/kv_cache.cpp:76-204, which does
// it with two cudaMemcpy2DAsync calls).  When a token's K and V rows fit one
// block (2 x row <= 256 words), thread t copies word t of K/V for kRowsPerBlock
// consecutive tokens, all loads before the stores; wider rows take a strided
// loop, one token at a time.  Words are 16 bytes when the row and every
// pointer allow, narrower otherwise.  Bytes are copied unchanged, so the
// kernel serves bf16 and fp32 caches alike.
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        constexpr int kNtmKv = 3;
        constexpr int kRowsPerBlock = 4;

        template <int NTM, typename W>
        __device__ __forceinline__ void copy_word(W *dst, const W *src)
        {
            if constexpr (sizeof(W) == 16)
                store8<nt_store(NTM)>(dst, load8<nt_load(NTM)>(src));
            else
                *dst = *src;
        }

        // Token rows t = b * S + s, strided over the grid; words_per_row is
        // the row size in W units.
        template <typename W>
        __global__ __launch_bounds__(kBlock) void kv_append_kernel(const W *__restrict__ k, const W *__restrict__ v,
                                                                   W *__restrict__ kc, W *__restrict__ vc,
                                                                   int64_t tokens, int64_t seq, int64_t seq_cap,
                                                                   int64_t start, int64_t words_per_row)
        {
            for (int64_t token = blockIdx.x; token < tokens; token += gridDim.x)
            {
                const int64_t b = token / seq;
                const int64_t dst_row = b * seq_cap + start + (token - b * seq);
                const W *ks = k + token * words_per_row;
                const W *vs = v + token * words_per_row;
                W *kd = kc + dst_row * words_per_row;
                W *vd = vc + dst_row * words_per_row;
                for (int64_t i = threadIdx.x; i < 2 * words_per_row; i += kBlock)
                {
                    if (i < words_per_row)
                        copy_word<kNtmKv>(kd + i, ks + i);
                    else
                        copy_word<kNtmKv>(vd + (i - words_per_row), vs + (i - words_per_row));
                }
            }
        }

        // 2 * words_per_row <= kBlock: thread t owns word t of the K row (t <
        // words_per_row) or of the V row; the block's tokens tok0 .. tok0 +
        // kRowsPerBlock - 1 are loaded first, then stored.  The destination row
        // (batch b, position start + s) steps from tok0's without a division.
        template <typename W>
        __global__ __launch_bounds__(kBlock) void kv_append_rows_kernel(const W *__restrict__ k, const W *__restrict__ v,
                                                                        W *__restrict__ kc, W *__restrict__ vc,
                                                                        int64_t tokens, int64_t seq, int64_t seq_cap,
                                                                        int64_t start, int64_t words_per_row)
        {
            const int t = threadIdx.x;
            const bool active = t < 2 * words_per_row;
            const bool is_v = t >= words_per_row;
            const int64_t w = is_v ? t - words_per_row : t;
            const W *src = (is_v ? v : k) + w;
            W *dst = (is_v ? vc : kc) + w;
            for (int64_t tok0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock; tok0 < tokens;
                 tok0 += static_cast<int64_t>(gridDim.x) * kRowsPerBlock)
            {
                W val[kRowsPerBlock];
#pragma unroll
                for (int u = 0; u < kRowsPerBlock; ++u)
                    if (active && tok0 + u < tokens)
                    {
                        if constexpr (sizeof(W) == 16)
                            val[u] = load8<nt_load(kNtmKv)>(src + (tok0 + u) * words_per_row);
                        else
                            val[u] = src[(tok0 + u) * words_per_row];
                    }
                int64_t b = tok0 / seq, s = tok0 - b * seq;
#pragma unroll
                for (int u = 0; u < kRowsPerBlock; ++u)
                {
                    if (active && tok0 + u < tokens)
                    {
                        W *d = dst + (b * seq_cap + start + s) * words_per_row;
                        if constexpr (sizeof(W) == 16)
                            store8<nt_store(kNtmKv)>(d, val[u]);
                        else
                            *d = val[u];
                    }
                    if (++s == seq)
                    {
                        s = 0;
                        ++b;
                    }
                }
            }
        }

        template <typename W>
        void launch_words(const void *k, const void *v, void *kc, void *vc, int64_t tokens, int64_t seq,
                          int64_t seq_cap, int64_t start, int64_t row_bytes, hipStream_t stream)
        {
            const int64_t words = row_bytes / static_cast<int64_t>(sizeof(W));
            if (2 * words <= kBlock)
            {
                const int64_t blocks = (tokens + kRowsPerBlock - 1) / kRowsPerBlock;
                const int64_t grid = blocks < (int64_t{1} << 20) ? blocks : (int64_t{1} << 20);
                kv_append_rows_kernel<W><<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, stream>>>(
                    static_cast<const W *>(k), static_cast<const W *>(v), static_cast<W *>(kc),
                    static_cast<W *>(vc), tokens, seq, seq_cap, start, words);
                return;
            }
            const int64_t grid = tokens < (int64_t{1} << 20) ? tokens : (int64_t{1} << 20);
            kv_append_kernel<W><<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, stream>>>(
                static_cast<const W *>(k), static_cast<const W *>(v), static_cast<W *>(kc), static_cast<W *>(vc),
                tokens, seq, seq_cap, start, words);
        }

        // The widest word that divides the row and every pointer.
        int word_bytes(const void *k, const void *v, const void *kc, const void *vc, int64_t row_bytes)
        {
            for (int w : {16, 4, 2})
                if (row_bytes % w == 0 && aligned_to(k, w) && aligned_to(v, w) && aligned_to(kc, w) &&
                    aligned_to(vc, w))
                    return w;
            return 1;
        }
    } // namespace

    int validate_kv_append(const void *k, const void *v, const void *kc, const void *vc, int64_t B, int64_t S,
                           int64_t row_bytes, int64_t seq_cap, int64_t start)
    {
        if (B < 0 || S < 0)
            return set_error(Q3K_ERR_INVALID_ARGUMENT, "KV cache input batch and sequence sizes cannot be negative");
        if (row_bytes <= 0 || seq_cap <= 0)
            return set_error(Q3K_ERR_INVALID_ARGUMENT, "KV cache row size and sequence capacity must be positive");
        if (start < 0 || start > seq_cap || S > seq_cap - start)
            return set_error(Q3K_ERR_OUT_OF_RANGE, "KV cache append exceeds sequence capacity");
        if (B > 0 && (seq_cap > INT64_MAX / B || row_bytes > INT64_MAX / (B * seq_cap)))
            return set_error(Q3K_ERR_OVERFLOW, "KV cache layer size overflows");
        if (B > 0 && S > 0 && (k == nullptr || v == nullptr || kc == nullptr || vc == nullptr))
            return set_error(Q3K_ERR_INVALID_ARGUMENT, "KV cache append received a null pointer");
        return Q3K_OK;
    }

    void launch_kv_append(const void *k, const void *v, void *kc, void *vc, int64_t B, int64_t S, int64_t row_bytes,
                          int64_t seq_cap, int64_t start, hipStream_t stream)
    {
        const int64_t tokens = B * S;
        if (tokens == 0)
            return;
        switch (word_bytes(k, v, kc, vc, row_bytes))
        {
        case 16: launch_words<Vec8>(k, v, kc, vc, tokens, S, seq_cap, start, row_bytes, stream); break;
        case 4: launch_words<uint32_t>(k, v, kc, vc, tokens, S, seq_cap, start, row_bytes, stream); break;
        case 2: launch_words<uint16_t>(k, v, kc, vc, tokens, S, seq_cap, start, row_bytes, stream); break;
        default: launch_words<uint8_t>(k, v, kc, vc, tokens, S, seq_cap, start, row_bytes, stream); break;
        }
    }
} // namespace q3k

extern "C" int q3k_kv_append(const void *key, const void *value, void *key_cache, void *value_cache, int64_t B,
                             int64_t S, int64_t row_bytes, int64_t seq_cap, int64_t start, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_kv_append(key, value, key_cache, value_cache, B, S, row_bytes, seq_cap, start))
        return st;
    if (B == 0 || S == 0)
        return Q3K_OK;
    launch_kv_append(key, value, key_cache, value_cache, B, S, row_bytes, seq_cap, start,
                     reinterpret_cast<hipStream_t>(stream));
    return check_launch("kv_cache_append");
}
