// RoPE (half-split pairs) and fused per-head Q/K RMSNorm + RoPE for gfx950.
//
// Fast path (head_dim 128, heads % 4 == 0, 16-byte aligned): a head of 128
// bf16 is 256 bytes = 16 lanes x one 128-bit vector, so a wave holds four
// heads of one token.  Lane l of a head holds elements 8(l%16) .. +7; the
// RoPE partner of element p (p < 64) is p + 64, which sits in lane l ^ 8 of
// the same 16-lane row and is fetched with one DPP row_ror:8 per dword (no
// LDS).  Token and position are wave-uniform (scalar math).  The fused
// kernel reduces the 128-element sum of squares over the 16 lanes with DPP,
// normalises, rounds to bf16 (twice, as rms_norm does), then rotates the
// rounded values: Q and K make a single round trip through HBM.
//
// Generic path: one thread per pair (any even head_dim), and for the fused
// op the generic RMSNorm followed by the generic RoPE.
//
// Arithmetic follows src/ops/rope.cu:64-84: c, s from the fp32 table,
// x1' = RNE(x1*c - x2*s), x2' = RNE(x2*c + x1*s), products and sum each
// rounded to fp32 (no contraction).
#include "q3k_common.hpp"

namespace q3k
{
    // Declared in rms_norm.hip: the generic RMSNorm used by the fused op's
    // fallback path.
    int launch_rms_generic(uint16_t *x, const uint16_t *w, int64_t rows, int64_t n, float eps, hipStream_t stream);

    namespace
    {
        constexpr int kHeadDim = 128;
        constexpr int kHalf = kHeadDim / 2;
        constexpr int kHeadsPerWave = kWave / 16;
        constexpr int kWavesPerBlock = kBlock / kWave;
        constexpr uint32_t kNanPair = 0x7fc07fc0u;

        struct RopeShape
        {
            int64_t tokens;   // B * S
            int64_t seq;      // S
            int64_t table_positions;
            int64_t start;
            const int32_t *positions;
            const float *cache;
        };

        // Position of a token: positions[t] or start + t % S; -1 when outside the table.
        __device__ __forceinline__ int64_t token_position(const RopeShape &rs, int64_t token)
        {
            int64_t pos;
            if (rs.positions != nullptr)
                pos = rs.positions[token];
            else
                pos = rs.start + token % rs.seq;
            return (pos >= 0 && pos < rs.table_positions) ? pos : -1;
        }

        // Rotate the eight values held by this lane.  own: this lane's values;
        // partner: the values of lane ^ 8.  First-half lanes compute
        // x1*c - x2*s, second-half lanes x2*c + x1*s.
        __device__ __forceinline__ Vec8 rotate8(const Vec8 &own, const Vec8 &partner, const float *cs, bool first_half)
        {
            const uint32_t sign = first_half ? 0x80000000u : 0u;
            Vec8 r;
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const float c0 = cs[4 * k + 0], s0 = __uint_as_float(__float_as_uint(cs[4 * k + 1]) ^ sign);
                const float c1 = cs[4 * k + 2], s1 = __uint_as_float(__float_as_uint(cs[4 * k + 3]) ^ sign);
                const float a0 = bf_lo(own.d[k]) * c0;
                const float b0 = bf_lo(partner.d[k]) * s0;
                const float a1 = bf_hi(own.d[k]) * c1;
                const float b1 = bf_hi(partner.d[k]) * s1;
                r.d[k] = pack_rne(a0 + b0, a1 + b1);
            }
            return r;
        }

        __device__ __forceinline__ Vec8 partner_of(const Vec8 &v)
        {
            Vec8 p;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                p.d[k] = dpp_u<kDppRowRor8>(v.d[k]);
            return p;
        }

        // One wave = four consecutive heads of one token.  Waves [0, q_waves)
        // cover q (heads_q per token), the rest k (heads_k per token).
        template <bool NORM>
        __global__ __launch_bounds__(kBlock) void rope_heads_kernel(
            uint16_t *__restrict__ q, uint16_t *__restrict__ k,
            const uint16_t *__restrict__ qw, const uint16_t *__restrict__ kw,
            int32_t heads_q, int32_t heads_k, int64_t q_waves, int64_t total_waves,
            RopeShape rs, float eps)
        {
            const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock +
                                 __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
            if (wave >= total_waves)
                return;
            const int lane16 = threadIdx.x % 16;
            const bool first_half = lane16 < 8;

            const bool is_q = wave < q_waves;
            const int64_t head0 = (is_q ? wave : wave - q_waves) * kHeadsPerWave;
            const int32_t heads = is_q ? heads_q : heads_k;
            uint16_t *base = is_q ? q : k;
            const int64_t token = head0 / heads;
            const int64_t pos = token_position(rs, token);

            Vec8 *hv = reinterpret_cast<Vec8 *>(base) + (head0 + (threadIdx.x % kWave) / 16) * (kHeadDim / 8) + lane16;
            Vec8 x = *hv;
            Vec8 wv;
            if constexpr (NORM)
                wv = reinterpret_cast<const Vec8 *>(is_q ? qw : kw)[lane16];

            if (pos < 0)
            {
                const Vec8 nan = {{kNanPair, kNanPair, kNanPair, kNanPair}};
                *hv = nan;
                return;
            }

            const F4 *crow = reinterpret_cast<const F4 *>(rs.cache + (pos * kHalf + (lane16 % 8) * 8) * 2);
            float cs[16];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const F4 t = crow[i];
                cs[4 * i + 0] = t.v[0];
                cs[4 * i + 1] = t.v[1];
                cs[4 * i + 2] = t.v[2];
                cs[4 * i + 3] = t.v[3];
            }

            if constexpr (NORM)
            {
                const float total = group_sum<16>(sum_sq8(x));
                x = norm_scale8(x, wv, inverse_rms(total, static_cast<float>(kHeadDim), eps));
            }
            *hv = rotate8(x, partner_of(x), cs, first_half);
        }

        // Generic RoPE: one thread per (token, head, pair), any even head_dim.
        __global__ __launch_bounds__(kBlock) void rope_generic_kernel(
            uint16_t *x, int32_t heads, int64_t head_dim, int64_t pairs_total, RopeShape rs)
        {
            const int64_t half = head_dim / 2;
            const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
            for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; idx < pairs_total; idx += stride)
            {
                const int64_t pair = idx % half;
                const int64_t head_linear = idx / half;            // token * heads + head
                const int64_t token = head_linear / heads;
                uint16_t *head_ptr = x + head_linear * head_dim;
                const int64_t pos = token_position(rs, token);
                if (pos < 0)
                {
                    head_ptr[pair] = 0x7fc0;
                    head_ptr[pair + half] = 0x7fc0;
                    continue;
                }
                const float c = rs.cache[(pos * half + pair) * 2];
                const float s = rs.cache[(pos * half + pair) * 2 + 1];
                const float x1 = bf_to_f(head_ptr[pair]);
                const float x2 = bf_to_f(head_ptr[pair + half]);
                const float a = x1 * c;
                const float b = x2 * s;
                const float e = x2 * c;
                const float f = x1 * s;
                head_ptr[pair] = f_to_bf(a - b);
                head_ptr[pair + half] = f_to_bf(e + f);
            }
        }

        bool fast_ok(const void *x, const float *cache, int32_t heads, int32_t head_dim)
        {
            return head_dim == kHeadDim && heads % kHeadsPerWave == 0 && aligned16(x) && aligned16(cache);
        }

        void launch_generic_rope(uint16_t *x, int32_t heads, int32_t head_dim, const RopeShape &rs, hipStream_t stream)
        {
            const int64_t pairs = rs.tokens * heads * (head_dim / 2);
            if (pairs == 0)
                return;
            const int64_t want = (pairs + kBlock - 1) / kBlock;
            const int64_t grid = want < 65536 ? want : 65536;
            rope_generic_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, stream>>>(
                x, heads, head_dim, pairs, rs);
        }

        // Validation shared by both entry points (src/ops/rope.cu:102-211 and
        // the positions form).
        int validate_rope(const void *q, int64_t B, int64_t S, int32_t heads, int32_t D, const float *cache,
                          int64_t P, int64_t start, const int32_t *positions)
        {
            if (B < 0 || S < 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE batch and sequence sizes cannot be negative");
            if (heads <= 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE head count must be positive");
            if (D <= 0 || D % 2 != 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE cache contains an invalid head dimension");
            if (P <= 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE cache must have at least one position");
            if (B > 0 && S > 0 && (q == nullptr || cache == nullptr))
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE received a null pointer");
            if (!aligned_to(q, 2) || !aligned_to(cache, 4) || !aligned_to(positions, 4))
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE pointers must be aligned to their element size");
            if (positions == nullptr)
            {
                if (start < 0)
                    return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE start_position cannot be negative");
                if (start > P || S > P - start)
                    return set_error(Q3K_ERR_OUT_OF_RANGE, "RoPE position range exceeds the cache");
            }
            if (B > 0 && S > INT64_MAX / B)
                return set_error(Q3K_ERR_OVERFLOW, "RoPE token count overflows");
            const int64_t tokens = B * S;
            if (tokens > 0 && static_cast<int64_t>(heads) * D > INT64_MAX / tokens)
                return set_error(Q3K_ERR_OVERFLOW, "RoPE projection size overflow");
            return Q3K_OK;
        }

        int64_t waves_for(int64_t tokens, int32_t heads) { return tokens * heads / kHeadsPerWave; }
    } // namespace
} // namespace q3k

extern "C" int q3k_rope_bf16(uint16_t *x, int64_t B, int64_t S, int32_t heads, int32_t D,
                             const float *cache, int64_t P, int64_t start,
                             const int32_t *positions, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_rope(x, B, S, heads, D, cache, P, start, positions))
        return st;
    const int64_t tokens = B * S;
    if (tokens == 0)
        return Q3K_OK;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const RopeShape rs{tokens, S, P, start, positions, cache};
    const int64_t waves = waves_for(tokens, heads);
    const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    if (fast_ok(x, cache, heads, D) && blocks < (int64_t{1} << 31))
    {
        rope_heads_kernel<false><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s>>>(
            x, x, nullptr, nullptr, heads, heads, waves, waves, rs, 0.0f);
    }
    else
    {
        launch_generic_rope(x, heads, D, rs, s);
    }
    return check_launch("apply_rope");
}

extern "C" int q3k_qk_norm_rope_bf16(uint16_t *q, uint16_t *k, const uint16_t *qw, const uint16_t *kw,
                                     int64_t B, int64_t S, int32_t Hq, int32_t Hkv, int32_t D, float eps,
                                     const float *cache, int64_t P, int64_t start,
                                     const int32_t *positions, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_rope(q, B, S, Hq, D, cache, P, start, positions))
        return st;
    if (const int st = validate_rope(k, B, S, Hkv, D, cache, P, start, positions))
        return st;
    if (!(eps > 0.0f) || eps == __builtin_huge_valf())
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm epsilon must be finite and positive");
    const int64_t tokens = B * S;
    if (tokens == 0)
        return Q3K_OK;
    if (qw == nullptr || kw == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "Q/K norm weight pointer is null");
    if (!aligned_to(qw, 2) || !aligned_to(kw, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "Q/K norm weights must be 2-byte aligned");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const RopeShape rs{tokens, S, P, start, positions, cache};
    const int64_t q_waves = waves_for(tokens, Hq);
    const int64_t total = q_waves + waves_for(tokens, Hkv);
    const int64_t blocks = (total + kWavesPerBlock - 1) / kWavesPerBlock;
    if (fast_ok(q, cache, Hq, D) && fast_ok(k, cache, Hkv, D) && aligned16(qw) && aligned16(kw) && blocks < (int64_t{1} << 31))
    {
        rope_heads_kernel<true><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s>>>(
            q, k, qw, kw, Hq, Hkv, q_waves, total, rs, eps);
        return check_launch("qk_norm_rope");
    }
    // Unfused fallback: per-head RMSNorm in place, then RoPE.
    int st = launch_rms_generic(q, qw, tokens * Hq, D, eps, s);
    if (st == Q3K_OK)
        st = launch_rms_generic(k, kw, tokens * Hkv, D, eps, s);
    if (st != Q3K_OK)
        return st;
    launch_generic_rope(q, Hq, D, rs, s);
    launch_generic_rope(k, Hkv, D, rs, s);
    return check_launch("qk_norm_rope (generic)");
}
