// Embedding gather for gfx950: out[t, :] = table[ids[t], :], a zero row for
// ids outside [0, V) (src/ops/embedding.cu:38-45).  Bit-exact copy.
//
// Fast path (H % 8 == 0, 16-byte aligned): one wave per token.  The id is
// wave-uniform (scalar load); each lane moves VPT 128-bit vectors, all loads
// issued before the stores, so a wave keeps VPT KiB of the row in flight.
// Rows longer than 64 * VPT vectors are covered by a loop.  Other shapes
// take a scalar kernel (one block per token, as the reference).
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        constexpr int kTokensPerBlock = kEmbeddingTokensPerBlock;
        constexpr int kVpt = 8;
        constexpr int kNtm = 2;  // measured: plain loads (random rows), non-temporal stores

        template <int NTM>
        __global__ __launch_bounds__(kEmbeddingBlock) void embedding_vec_kernel(
            const int32_t *__restrict__ ids, int64_t tokens,
            const Vec8 *__restrict__ table, int64_t vocab, int64_t nvec,
            Vec8 *__restrict__ out)
        {
            const int lane = threadIdx.x % kWave;
            const int64_t token = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + threadIdx.x / kWave;
            if (token >= tokens)
                return;
            const int32_t id = __builtin_amdgcn_readfirstlane(ids[token]);
            Vec8 *dst = out + token * nvec;
            if (id < 0 || static_cast<int64_t>(id) >= vocab)
            {
                const Vec8 zero = {{0u, 0u, 0u, 0u}};
                for (int64_t j = lane; j < nvec; j += kWave)
                    store8<nt_store(NTM)>(dst + j, zero);
                return;
            }
            const Vec8 *src = table + static_cast<int64_t>(id) * nvec;
            for (int64_t j0 = 0; j0 < nvec; j0 += static_cast<int64_t>(kWave) * kVpt)
            {
                Vec8 v[kVpt];
#pragma unroll
                for (int i = 0; i < kVpt; ++i)
                {
                    const int64_t j = j0 + lane + i * kWave;
                    if (j < nvec)
                        v[i] = load8<nt_load(NTM)>(src + j);
                }
#pragma unroll
                for (int i = 0; i < kVpt; ++i)
                {
                    const int64_t j = j0 + lane + i * kWave;
                    if (j < nvec)
                        store8<nt_store(NTM)>(dst + j, v[i]);
                }
            }
        }

        __global__ __launch_bounds__(kBlock) void embedding_scalar_kernel(
            const int32_t *ids, int64_t tokens, const uint16_t *table, int64_t vocab, int64_t hidden,
            uint16_t *out)
        {
            for (int64_t token = blockIdx.x; token < tokens; token += gridDim.x)
            {
                const int32_t id = ids[token];
                uint16_t *dst = out + token * hidden;
                const bool valid = id >= 0 && static_cast<int64_t>(id) < vocab;
                const uint16_t *src = table + (valid ? static_cast<int64_t>(id) * hidden : 0);
                for (int64_t c = threadIdx.x; c < hidden; c += blockDim.x)
                    dst[c] = valid ? src[c] : uint16_t{0};
            }
        }
    } // namespace
} // namespace q3k

extern "C" int q3k_embedding_bf16(const int32_t *ids, int64_t T, const uint16_t *table, int64_t V,
                                  int64_t H, uint16_t *out, q3k_stream_t stream)
{
    using namespace q3k;
    if (T < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding token count cannot be negative");
    if (V <= 0 || H <= 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding weight dimensions must be positive");
    if (T == 0)
        return Q3K_OK;
    if (ids == nullptr || table == nullptr || out == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding received a null pointer");
    if (!aligned_to(ids, 4) || !aligned_to(table, 2) || !aligned_to(out, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding pointers must be aligned to their element size");
    if (V > INT64_MAX / H || T > INT64_MAX / H)
        return set_error(Q3K_ERR_OVERFLOW, "embedding size overflows");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (H % 8 == 0 && aligned16(table) && aligned16(out) && embedding_vec_fits(T))
    {
        const dim3 grid(static_cast<unsigned>(blocks_for(T, kTokensPerBlock)));
        embedding_vec_kernel<kNtm><<<grid, dim3(kEmbeddingBlock), 0, s>>>(
            ids, T, reinterpret_cast<const Vec8 *>(table), V, H / 8, reinterpret_cast<Vec8 *>(out));
    }
    else
    {
        const int64_t grid = T < 65535 ? T : 65535;
        embedding_scalar_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, s>>>(ids, T, table, V, H, out);
    }
    return check_launch("embedding_lookup");
}
