// RoPE (half-split pairs) and fused per-head Q/K RMSNorm + RoPE for gfx950.
//
// Fast path (head_dim 128, heads % 4 == 0, 16-byte aligned): a head of 128
// bf16 is 256 bytes = 16 lanes x one 128-bit vector, so a wave holds four
// heads of one token at a time; a lane processes up to four heads (16 per
// wave) when the head count allows.  Lane l of a head holds elements 8(l%16) .. +7; the
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
#include "dispatch.hpp"
#include "q3k_common.hpp"

namespace q3k
{
    // Declared in rms_norm.hip: the generic RMSNorm used by the fused op's
    // fallback path.
    int launch_rms_generic(uint16_t *x, const uint16_t *w, int64_t rows, int64_t n, float eps, hipStream_t stream);
    // Declared in kv_cache.hip: the KV-cache append's checks and its copy kernel.
    int validate_kv_append(const void *k, const void *v, const void *kc, const void *vc, int64_t B, int64_t S,
                           int64_t row_bytes, int64_t seq_cap, int64_t start);
    void launch_kv_append(const void *k, const void *v, void *kc, void *vc, int64_t B, int64_t S, int64_t row_bytes,
                          int64_t seq_cap, int64_t start, hipStream_t stream);

    namespace
    {
        constexpr int kHeadDim = 128;
        constexpr int kHalf = kHeadDim / 2;
        constexpr int kHeadsPerWave = kRopeHeadsPerWave;
        constexpr int kWavesPerBlock = kRopeWavesPerBlock;
        constexpr uint32_t kNanPair = 0x7fc07fc0u;
        // NT mode bits (loads | stores) and heads per lane, chosen by measurement.
        constexpr int kNtmRope = 3;
        constexpr int kNtmNormRope = 3;
        constexpr bool kRemapHeads = false;  // XCD-contiguous tiles measured slower
        // Wave priority while the head loads are issued.  Raising it helped
        // while stores were written back from L2 at the end of each kernel;
        // with write-through stores the default is faster (c4: 77.0%
        // against 75.6% of peak with priority 3; c5: 82.9% against 81.7%).
        constexpr int kPrioHeads = 0;

        struct RopeShape
        {
            int64_t tokens;   // B * S
            int64_t seq;      // S
            int64_t table_positions;
            int64_t start;
            const int32_t *positions;
            const float *cache;
        };

        // Position of a token: positions[t] (POS: a positions array was
        // given) or start + t % S; -1 when outside the table.
        template <bool POS>
        __device__ __forceinline__ int64_t token_position(const RopeShape &rs, int64_t token)
        {
            int64_t pos;
            if constexpr (POS)
                pos = rs.positions[token];
            else
                pos = rs.start + token % rs.seq;
            return (pos >= 0 && pos < rs.table_positions) ? pos : -1;
        }

        // token_position for a per-lane token, in 32-bit arithmetic (tokens and
        // the sequence length are below 2^31)
        template <bool POS>
        __device__ __forceinline__ int64_t lane_token_position(const RopeShape &rs, uint32_t token)
        {
            int64_t pos;
            if constexpr (POS)
                pos = rs.positions[token];
            else
            {
                const uint32_t seq = static_cast<uint32_t>(rs.seq);
                pos = rs.start + (token - token / seq * seq);
            }
            return (pos >= 0 && pos < rs.table_positions) ? pos : -1;
        }

        // Where the K (and V) heads of the fused KV-cache append go: token
        // t = b * S + s of the input lands in row b * seq_cap + cache_start + s
        // of the layer's [batch_cap, seq_cap, Hkv, D] cache.  V is copied
        // unchanged next to the roped K.
        struct KvDest
        {
            const uint16_t *v;
            uint16_t *k_cache;
            uint16_t *v_cache;
            int64_t seq_cap;
            int64_t cache_start;
        };

        constexpr int kVecPerHead = kHeadDim / 8;
        constexpr int kHeadStride = kHeadsPerWave * kVecPerHead;  // Vec8s between a lane's heads

        // cos and sin of pairs 8(l%8) .. +7 of position `pos` for the lane
        // (l = lane16); first-half lanes use -sin so that both halves compute
        // own * cos + partner * sin'.
        __device__ __forceinline__ void table_row(const float *table, int64_t pos, int lane16, float (&cs)[8],
                                                  float (&sn)[8])
        {
            const F4 *crow = reinterpret_cast<const F4 *>(table + (pos * kHalf + (lane16 % 8) * 8) * 2);
            const uint32_t sign = lane16 < 8 ? 0x80000000u : 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const F4 t = crow[i];
                cs[2 * i] = t.v[0];
                sn[2 * i] = __uint_as_float(__float_as_uint(t.v[1]) ^ sign);
                cs[2 * i + 1] = t.v[2];
                sn[2 * i + 1] = __uint_as_float(__float_as_uint(t.v[3]) ^ sign);
            }
        }

        // The lane's 8 norm weights (bf16 -> fp32).
        __device__ __forceinline__ void norm_weights(const uint16_t *w, int lane16, float (&wf)[8])
        {
            const Vec8 wv = reinterpret_cast<const Vec8 *>(w)[lane16];
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                wf[2 * j] = bf_lo(wv.d[j]);
                wf[2 * j + 1] = bf_hi(wv.d[j]);
            }
        }

        // One head's 8 elements of this lane: with NORM, rms_norm over the
        // head (128 values in 16 lanes, two roundings), then the rotation of
        // the rounded values; the partner element (lane ^ 8) comes through
        // DPP, folded into the multiply.  Every lane of the 16-lane group must
        // run it together.
        template <bool NORM>
        __device__ __forceinline__ Vec8 rotate_head(const Vec8 &x, const float (&wf)[8], const float (&cs)[8],
                                                    const float (&sn)[8], float eps)
        {
            float v[8];
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                v[2 * j] = bf_lo(x.d[j]);
                v[2 * j + 1] = bf_hi(x.d[j]);
            }
            if constexpr (NORM)
            {
                // the sum of squares in the order of the plain RMSNorm kernel's
                // 128-wide rows (sum_sq8, then the 16 lanes), so that the fused
                // op equals rms_norm + RoPE bit for bit
                const float total = group_sum<16>(sum_sq8(x));
                const float inv = inverse_rms(total, 1.0f / static_cast<float>(kHeadDim), eps);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    const uint32_t n = pack_rne(v[2 * j] * inv, v[2 * j + 1] * inv);
                    const uint32_t y = pack_rne(bf_lo(n) * wf[2 * j], bf_hi(n) * wf[2 * j + 1]);
                    v[2 * j] = bf_lo(y);
                    v[2 * j + 1] = bf_hi(y);
                }
            }
            Vec8 r;
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const float a0 = v[2 * j] * cs[2 * j];
                const float b0 = dpp_f<kDppRowRor8>(v[2 * j]) * sn[2 * j];
                const float a1 = v[2 * j + 1] * cs[2 * j + 1];
                const float b1 = dpp_f<kDppRowRor8>(v[2 * j + 1]) * sn[2 * j + 1];
                r.d[j] = pack_rne(a0 + b0, a1 + b1);
            }
            return r;
        }

        // One wave = 4 * HG consecutive heads of one token (heads % (4 * HG)
        // == 0): lane l of the wave works on heads l/16 + 4i, i < HG, of
        // `src`/`dst` (already offset to the wave's first head and the lane's
        // vector), elements 8(l%16) .. +7 of each.  The table row, the sign
        // pattern and the norm weights depend only on the lane and the
        // position, so they are loaded and unpacked once per wave.  With
        // COPY_V the wave also moves the matching V heads from vsrc to vdst.
        //
        // The position comes from `position()` (the token's table row, or -1
        // when it is outside the table), called once the head loads are
        // issued: the heads do not depend on it, so a position that has to be
        // read from memory (decode) costs one round trip beside the head
        // loads instead of one before them.  A position outside the table
        // reads row 0 and the results are replaced by NaN, so no branch
        // separates the loads.
        template <bool NORM, int NTM, int HG, bool COPY_V, int PR, typename Position>
        __device__ __forceinline__ void rope_heads(const Vec8 *src, Vec8 *dst, const Vec8 *vsrc, Vec8 *vdst,
                                                   const uint16_t *w, const float *table, Position position,
                                                   float eps)
        {
            const int lane16 = threadIdx.x % 16;
            Vec8 x[HG];
            Vec8 xv[COPY_V ? HG : 1];
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(PR);
#pragma unroll
            for (int i = 0; i < HG; ++i)
                x[i] = load8<nt_load(NTM)>(src + i * kHeadStride);
            if constexpr (COPY_V)
            {
#pragma unroll
                for (int i = 0; i < HG; ++i)
                    xv[i] = load8<nt_load(NTM)>(vsrc + i * kHeadStride);
            }
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(0);

            const int64_t pos = position();
            const bool in_table = pos >= 0;
            float wf[8];
            if constexpr (NORM)
                norm_weights(w, lane16, wf);
            float cs[8], sn[8];
            table_row(table, in_table ? pos : 0, lane16, cs, sn);
            const Vec8 nan = {{kNanPair, kNanPair, kNanPair, kNanPair}};
#pragma unroll
            for (int i = 0; i < HG; ++i)
            {
                const Vec8 r = rotate_head<NORM>(x[i], wf, cs, sn, eps);
                Vec8 out;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    out.d[j] = in_table ? r.d[j] : nan.d[j];
                store8<nt_store(NTM)>(dst + i * kHeadStride, out);
            }
            if constexpr (COPY_V)
            {
#pragma unroll
                for (int i = 0; i < HG; ++i)
                    store8<nt_store(NTM)>(vdst + i * kHeadStride, xv[i]);
            }
        }

        // The lane's vector of head `head` (counted over the whole tensor) of
        // a [tokens, heads, 128] tensor.
        __device__ __forceinline__ int64_t lane_vec(int64_t head)
        {
            return (head + (threadIdx.x % kWave) / 16) * kVecPerHead + threadIdx.x % 16;
        }

        // Waves [0, q_waves) cover q with HGQ heads per lane, the rest k with
        // HGK.  POS: positions come from rs.positions, else start + t % S.
        // Q is rewritten in place; K in place too, or with KV into the
        // cache rows given by `kv` (k itself is then only read).  Heads and
        // tokens are wave-uniform and below 2^31 (checked by the launcher).
        // ANYH bit 0 (Q) / bit 1 (K): that tensor's head count is not a
        // multiple of 4 (with HGQ = HGK = 1).  Lane group j of the tensor's
        // wave w then takes row 4 w + j of its flattened [tokens * heads]
        // rows, so the four rows of a wave may belong to different tokens
        // (token and position are per lane group), and the groups past the
        // last row of a partial last wave do nothing.
        template <bool NORM, int NTM, int HGQ, int HGK, bool REMAP, bool KV, int PR, int ANYH, bool POS>
        __global__ __launch_bounds__(kRopeBlock) void rope_heads_kernel(
            uint16_t *__restrict__ q, uint16_t *__restrict__ k,
            const uint16_t *__restrict__ qw, const uint16_t *__restrict__ kw,
            int32_t heads_q, int32_t heads_k, int64_t q_waves, int64_t total_waves,
            RopeShape rs, float eps, KvDest kv)
        {
            const int64_t wave = static_cast<int64_t>(tile_index<REMAP>(blockIdx.x, gridDim.x)) * kWavesPerBlock +
                                 __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
            if (wave >= total_waves)
                return;
            if constexpr (ANYH != 0)
            {
                static_assert(HGQ == 1 && HGK == 1, "one head per lane group");
                const bool is_q = wave < q_waves;
                if ((is_q && (ANYH & 1)) || (!is_q && (ANYH & 2)))
                {
                    const int32_t heads = is_q ? heads_q : heads_k;
                    const int64_t row = (is_q ? wave : wave - q_waves) * kHeadsPerWave + (threadIdx.x % kWave) / 16;
                    if (row >= rs.tokens * heads)
                        return;
                    // rows, tokens and the sequence length are below 2^31
                    // (checked by the launcher): 32-bit index arithmetic
                    const uint32_t token = static_cast<uint32_t>(row) / static_cast<uint32_t>(heads);
                    const auto pos = [&]() __attribute__((always_inline)) { return lane_token_position<POS>(rs, token); };
                    const int64_t vec = row * kVecPerHead + threadIdx.x % 16;
                    if (is_q)
                    {
                        Vec8 *p = reinterpret_cast<Vec8 *>(q) + vec;
                        rope_heads<NORM, NTM, 1, false, PR>(p, p, nullptr, nullptr, qw, rs.cache, pos, eps);
                        return;
                    }
                    Vec8 *src = reinterpret_cast<Vec8 *>(k) + vec;
                    if constexpr (KV)
                    {
                        const uint32_t seq = static_cast<uint32_t>(rs.seq);
                        const uint32_t b = token / seq;
                        const int64_t cache_row =
                            static_cast<int64_t>(b) * kv.seq_cap + kv.cache_start + (token - b * seq);
                        const int64_t dvec = (cache_row * heads_k + (row - static_cast<int64_t>(token) * heads_k)) *
                                                 kVecPerHead + threadIdx.x % 16;
                        rope_heads<NORM, NTM, 1, true, PR>(src, reinterpret_cast<Vec8 *>(kv.k_cache) + dvec,
                                                           reinterpret_cast<const Vec8 *>(kv.v) + vec,
                                                           reinterpret_cast<Vec8 *>(kv.v_cache) + dvec, kw, rs.cache,
                                                           pos, eps);
                    }
                    else
                    {
                        rope_heads<NORM, NTM, 1, false, PR>(src, src, nullptr, nullptr, kw, rs.cache, pos, eps);
                    }
                    return;
                }
            }
            if (wave < q_waves)
            {
                const uint32_t head0 = static_cast<uint32_t>(wave * kHeadsPerWave * HGQ);
                const uint32_t token = head0 / static_cast<uint32_t>(heads_q);
                Vec8 *p = reinterpret_cast<Vec8 *>(q) + lane_vec(head0);
                const auto pos = [&]() __attribute__((always_inline)) { return token_position<POS>(rs, token); };
                rope_heads<NORM, NTM, HGQ, false, PR>(p, p, nullptr, nullptr, qw, rs.cache, pos, eps);
                return;
            }
            const uint32_t head0 = static_cast<uint32_t>((wave - q_waves) * kHeadsPerWave * HGK);
            const uint32_t token = head0 / static_cast<uint32_t>(heads_k);
            const auto pos = [&]() __attribute__((always_inline)) { return token_position<POS>(rs, token); };
            Vec8 *src = reinterpret_cast<Vec8 *>(k) + lane_vec(head0);
            if constexpr (KV)
            {
                const uint32_t seq = static_cast<uint32_t>(rs.seq);
                const uint32_t b = token / seq;
                const int64_t row = static_cast<int64_t>(b) * kv.seq_cap + kv.cache_start + (token - b * seq);
                const int64_t dst_head = row * heads_k + (head0 - token * static_cast<uint32_t>(heads_k));
                rope_heads<NORM, NTM, HGK, true, PR>(src, reinterpret_cast<Vec8 *>(kv.k_cache) + lane_vec(dst_head),
                                                 reinterpret_cast<const Vec8 *>(kv.v) + lane_vec(head0),
                                                 reinterpret_cast<Vec8 *>(kv.v_cache) + lane_vec(dst_head), kw,
                                                 rs.cache, pos, eps);
            }
            else
            {
                rope_heads<NORM, NTM, HGK, false, PR>(src, src, nullptr, nullptr, kw, rs.cache, pos, eps);
            }
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
                const int64_t pos =
                    rs.positions != nullptr ? token_position<true>(rs, token) : token_position<false>(rs, token);
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

        template <bool NORM, bool KV, int HGQ, int HGK, int ANYH = 0>
        void launch_heads_hg(bool small, uint16_t *q, uint16_t *k, const uint16_t *qw, const uint16_t *kw, int32_t hq,
                             int32_t hk, int64_t tokens, const RopeShape &rs, float eps, const KvDest &kv,
                             hipStream_t stream)
        {
            constexpr int NTM = NORM ? kNtmNormRope : kNtmRope;
            const int64_t q_waves = rope_waves(tokens, hq, HGQ);
            const int64_t total = q_waves + (k == nullptr ? 0 : rope_waves(tokens, hk, HGK));
            const unsigned blocks = static_cast<unsigned>((total + kWavesPerBlock - 1) / kWavesPerBlock);
            const dim3 grid(blocks), block(kRopeBlock);
            const bool pos = rs.positions != nullptr;
            if (small && pos)
                rope_heads_kernel<NORM, ntm_small(NTM), HGQ, HGK, kRemapHeads, KV, kPrioHeads, ANYH, true>
                    <<<grid, block, 0, stream>>>(q, k, qw, kw, hq, hk, q_waves, total, rs, eps, kv);
            else if (small)
                rope_heads_kernel<NORM, ntm_small(NTM), HGQ, HGK, kRemapHeads, KV, kPrioHeads, ANYH, false>
                    <<<grid, block, 0, stream>>>(q, k, qw, kw, hq, hk, q_waves, total, rs, eps, kv);
            else if (pos)
                rope_heads_kernel<NORM, NTM, HGQ, HGK, kRemapHeads, KV, kPrioHeads, ANYH, true>
                    <<<grid, block, 0, stream>>>(q, k, qw, kw, hq, hk, q_waves, total, rs, eps, kv);
            else
                rope_heads_kernel<NORM, NTM, HGQ, HGK, kRemapHeads, KV, kPrioHeads, ANYH, false>
                    <<<grid, block, 0, stream>>>(q, k, qw, kw, hq, hk, q_waves, total, rs, eps, kv);
        }

        // The instance the plan (plan_rope) names: heads per lane of Q and K, or
        // rows per lane group for head counts that are not a multiple of 4.
        template <bool NORM, bool KV = false>
        void launch_heads(const RopePlan &plan, uint16_t *q, uint16_t *k, const uint16_t *qw, const uint16_t *kw,
                          int32_t hq, int32_t hk, int64_t tokens, const RopeShape &rs, float eps, hipStream_t stream,
                          const KvDest &kv = {})
        {
            if (plan.any_heads != 0)
            {
                if (plan.any_heads == 1)
                    launch_heads_hg<NORM, KV, 1, 1, 1>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream);
                else if (plan.any_heads == 2)
                    launch_heads_hg<NORM, KV, 1, 1, 2>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream);
                else
                    launch_heads_hg<NORM, KV, 1, 1, 3>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream);
                return;
            }
            switch (plan.hg_q * 10 + plan.hg_k)
            {
            case 44: launch_heads_hg<NORM, KV, 4, 4>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 42: launch_heads_hg<NORM, KV, 4, 2>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 41: launch_heads_hg<NORM, KV, 4, 1>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 24: launch_heads_hg<NORM, KV, 2, 4>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 22: launch_heads_hg<NORM, KV, 2, 2>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 21: launch_heads_hg<NORM, KV, 2, 1>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 14: launch_heads_hg<NORM, KV, 1, 4>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            case 12: launch_heads_hg<NORM, KV, 1, 2>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            default: launch_heads_hg<NORM, KV, 1, 1>(plan.small, q, k, qw, kw, hq, hk, tokens, rs, eps, kv, stream); break;
            }
        }
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
    const RopePlan plan = plan_rope(tokens, heads, 0, D, aligned16(x) && aligned16(cache));
    if (plan.fast)
        launch_heads<false>(plan, x, nullptr, nullptr, nullptr, heads, 0, tokens, rs, 0.0f, s);
    else
        launch_generic_rope(x, heads, D, rs, s);
    return check_launch("apply_rope");
}

extern "C" int q3k_rope_qk_bf16(uint16_t *q, uint16_t *k, int64_t B, int64_t S, int32_t Hq, int32_t Hkv, int32_t D,
                                const float *cache, int64_t P, int64_t start, const int32_t *positions,
                                q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_rope(q, B, S, Hq, D, cache, P, start, positions))
        return st;
    if (const int st = validate_rope(k, B, S, Hkv, D, cache, P, start, positions))
        return st;
    const int64_t tokens = B * S;
    if (tokens == 0)
        return Q3K_OK;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const RopeShape rs{tokens, S, P, start, positions, cache};
    const RopePlan plan = plan_rope(tokens, Hq, Hkv, D, aligned16(q) && aligned16(k) && aligned16(cache));
    if (plan.fast)
    {
        // one grid: the waves before q_waves rotate Q, the rest K
        launch_heads<false>(plan, q, k, nullptr, nullptr, Hq, Hkv, tokens, rs, 0.0f, s);
        return check_launch("apply_rope");
    }
    launch_generic_rope(q, Hq, D, rs, s);
    launch_generic_rope(k, Hkv, D, rs, s);
    return check_launch("apply_rope (generic)");
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
    const RopePlan plan =
        plan_rope(tokens, Hq, Hkv, D, aligned16(q) && aligned16(k) && aligned16(cache) && aligned16(qw) && aligned16(kw));
    if (plan.fast)
    {
        launch_heads<true>(plan, q, k, qw, kw, Hq, Hkv, tokens, rs, eps, s);
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

extern "C" int q3k_qk_norm_rope_kv_append_bf16(uint16_t *q, const uint16_t *k, const uint16_t *v,
                                               const uint16_t *qw, const uint16_t *kw, int64_t B, int64_t S,
                                               int32_t Hq, int32_t Hkv, int32_t D, float eps, const float *cache,
                                               int64_t P, int64_t start, const int32_t *positions,
                                               uint16_t *k_cache, uint16_t *v_cache, int64_t seq_cap,
                                               int64_t cache_start, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_rope(q, B, S, Hq, D, cache, P, start, positions))
        return st;
    if (const int st = validate_rope(k, B, S, Hkv, D, cache, P, start, positions))
        return st;
    if (!(eps > 0.0f) || eps == __builtin_huge_valf())
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm epsilon must be finite and positive");
    const int64_t row_bytes = static_cast<int64_t>(Hkv) * D * 2;
    if (const int st = validate_kv_append(k, v, k_cache, v_cache, B, S, row_bytes, seq_cap, cache_start))
        return st;
    const int64_t tokens = B * S;
    if (tokens == 0)
        return Q3K_OK;
    if (qw == nullptr || kw == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "Q/K norm weight pointer is null");
    if (!aligned_to(qw, 2) || !aligned_to(kw, 2) || !aligned_to(v, 2) || !aligned_to(k_cache, 2) ||
        !aligned_to(v_cache, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "bf16 pointers must be 2-byte aligned");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const RopeShape rs{tokens, S, P, start, positions, cache};
    const RopePlan plan = plan_rope(tokens, Hq, Hkv, D,
                                    aligned16(q) && aligned16(k) && aligned16(cache) && aligned16(qw) && aligned16(kw) &&
                                        aligned16(v) && aligned16(k_cache) && aligned16(v_cache));
    if (plan.fast)
    {
        const KvDest kv{v, k_cache, v_cache, seq_cap, cache_start};
        launch_heads<true, true>(plan, q, const_cast<uint16_t *>(k), qw, kw, Hq, Hkv, tokens, rs, eps, s, kv);
        return check_launch("qk_norm_rope_kv_append");
    }
    // Generic path: copy K and V into the cache, then norm and rotate the
    // cache rows of each sequence in place; Q as in qk_norm_rope.
    launch_kv_append(k, v, k_cache, v_cache, B, S, row_bytes, seq_cap, cache_start, s);
    int st = launch_rms_generic(q, qw, tokens * Hq, D, eps, s);
    for (int64_t b = 0; st == Q3K_OK && b < B; ++b)
        st = launch_rms_generic(k_cache + (b * seq_cap + cache_start) * Hkv * D, kw, S * Hkv, D, eps, s);
    if (st != Q3K_OK)
        return st;
    launch_generic_rope(q, Hq, D, rs, s);
    for (int64_t b = 0; b < B; ++b)
    {
        const RopeShape rb{S, S, P, start, positions == nullptr ? nullptr : positions + b * S, cache};
        launch_generic_rope(k_cache + (b * seq_cap + cache_start) * Hkv * D, Hkv, D, rb, s);
    }
    return check_launch("qk_norm_rope_kv_append (generic)");
}
