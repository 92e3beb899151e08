// Elementwise bf16 ops for gfx950: SwiGLU activation silu(gate) * up and the
// in-place residual add.
//
// Fast path (16-byte aligned pointers): each thread streams UNROLL 128-bit
// vectors (8 bf16) per operand (one for both ops, chosen by measurement),
// all loads issued before any arithmetic; a wave's load instruction covers
// 1 KiB of contiguous memory.  The n % 8 tail
// is finished by a scalar pass in the first block.  Unaligned pointers take a
// scalar grid-stride kernel.
//
// Arithmetic follows src/ops/elementwise.cu:28-35 (add: RNE(d + s)) and
// :45-66 (silu: RNE(RNE(g / (1 + exp(-g))) * u)).
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        // Launch shapes chosen by measurement on MI355X at the model's sizes:
        // vectors per thread (per operand) and non-temporal mode bits.
        constexpr int kUnrollSilu = 1;  // config 4, sustained: 79-80% of peak against 77% for 2 and 74% for 4
        constexpr int kNtmSilu = 3;
        constexpr int kPrioSilu = 1;  // wave priority while loads are issued
        constexpr int kUnrollAdd = 1;
        constexpr int kNtmAdd = 3;
        // Blocks of the large launches: one wave (1 KiB of each stream per
        // block), tiles in order.  Measured on MI355X for SwiGLU at 24-800 MB
        // per stream (configs 4 and 5, their tensor-parallel-8 shard, and three
        // sizes between): 64 threads gave 69.2-82.7% of peak HBM, the best or
        // within 0.5 points of the best at every size; 256 threads gave
        // 67.6-80.2% (config 4: 81.8% against 78.8%, config 5: 82.2% against
        // 80.2%), 128 and 512-1024 threads in between.  Workgroups go to the
        // eight XCDs in turn, so the block size sets how finely the streams
        // are interleaved over the XCDs.  XCD-contiguous or XOR-permuted tile
        // orders gained at some sizes and lost up to 5 points at others.
        constexpr int kStreamBlock = 64;

        // exp(x) for the SiLU denominator: Cody-Waite style split of
        // x * log2(e) into an integer and a fraction, the fraction through the
        // hardware 2^x and the integer part through ldexp.  Relative error is
        // about 1 ulp over the clamped range; inputs are clamped to
        // [-150, 128] so that the result saturates to 0 / +inf like expf.
        __device__ __forceinline__ float exp_f32(float x)
        {
            x = __builtin_amdgcn_fmed3f(x, -150.0f, 128.0f);
            const float kLog2eHi = 1.44269502162933349609375f;   // float(log2 e)
            const float kLog2eLo = 1.925963033500011079e-8f;     // log2 e - kLog2eHi
            const float ph = x * kLog2eHi;
            const float pl = __builtin_fmaf(x, kLog2eHi, -ph) + x * kLog2eLo;
            const float e = __builtin_rintf(ph);
            const float a = (ph - e) + pl;
            return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(a), static_cast<int>(e));
        }

        // The reciprocal serves a denominator below 2^126 (and NaN).
        __device__ __forceinline__ bool rcp_ok(float den) { return den < 0x1p126f || den != den; }

        // silu(g) = g / (1 + exp(-g)) for W packed words (2 W values), as
        // g * rcp(1 + exp(-g)): v_rcp_f32 is within 1 ulp, the whole
        // expression within about 3.5 ulp of the exact value.  v_rcp_f32
        // flushes denormal results, so a denominator >= 2^126 (g in
        // [-88.72, -87.3]) or +inf (exp(-g) overflow, g < -88.72) takes the
        // IEEE divide instead; there g / inf is the signed zero that the
        // reference's g / (1 + expf(-g)) gives.  The choice is per element,
        // so the result does not depend on how elements are grouped into
        // lanes.
        template <int W>
        __device__ __forceinline__ void silu_words(const uint32_t (&g)[W], float (&s)[2 * W])
        {
            float gv[2 * W], den[2 * W];
#pragma unroll
            for (int k = 0; k < W; ++k)
            {
                gv[2 * k] = bf_lo(g[k]);
                gv[2 * k + 1] = bf_hi(g[k]);
            }
            bool fast = true;
#pragma unroll
            for (int j = 0; j < 2 * W; ++j)
            {
                den[j] = 1.0f + exp_f32(-gv[j]);
                fast = fast && rcp_ok(den[j]);
            }
            // Tested for the whole wave first: a lane-divergent if/else is
            // issued on both sides under exec masks, and the IEEE divide would
            // then cost every element ~12 more VALU ops.  The slow side is
            // never taken on ordinary activations.
            if (__all(fast))
            {
#pragma unroll
                for (int j = 0; j < 2 * W; ++j)
                    s[j] = gv[j] * __builtin_amdgcn_rcpf(den[j]);
            }
            else
            {
#pragma unroll
                for (int j = 0; j < 2 * W; ++j)
                    s[j] = rcp_ok(den[j]) ? gv[j] * __builtin_amdgcn_rcpf(den[j]) : gv[j] / den[j];
            }
        }

        // RNE(RNE(silu(g)) * u) for W packed words.
        template <int W>
        __device__ __forceinline__ void silu_mul_words(const uint32_t (&g)[W], const uint32_t (&u)[W], uint32_t (&r)[W])
        {
            float s[2 * W];
            silu_words<W>(g, s);
#pragma unroll
            for (int k = 0; k < W; ++k)
            {
                const uint32_t n = pack_rne(s[2 * k], s[2 * k + 1]);
                r[k] = pack_rne(bf_lo(n) * bf_lo(u[k]), bf_hi(n) * bf_hi(u[k]));
            }
        }

        __device__ __forceinline__ Vec8 silu_mul8(const Vec8 &g, const Vec8 &u)
        {
            const uint32_t gw[4] = {g.d[0], g.d[1], g.d[2], g.d[3]}, uw[4] = {u.d[0], u.d[1], u.d[2], u.d[3]};
            uint32_t rw[4];
            silu_mul_words<4>(gw, uw, rw);
            return Vec8{{rw[0], rw[1], rw[2], rw[3]}};
        }

        __device__ __forceinline__ uint16_t silu_mul1(uint16_t g, uint16_t u)
        {
            const float gv = bf_to_f(g);
            const float s = bf_to_f(f_to_bf(gv / (1.0f + exp_f32(-gv))));
            return f_to_bf(s * bf_to_f(u));
        }

        __device__ __forceinline__ uint32_t add2(uint32_t a, uint32_t b)
        {
            return pack_rne(bf_lo(a) + bf_lo(b), bf_hi(a) + bf_hi(b));
        }

        template <int OP>
        __device__ __forceinline__ Vec8 apply8(const Vec8 &a, const Vec8 &b)
        {
            if constexpr (OP == 0)
                return silu_mul8(a, b);
            else
            {
                Vec8 r;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    r.d[k] = add2(a.d[k], b.d[k]);
                return r;
            }
        }

        template <int OP>
        __device__ __forceinline__ uint16_t apply1(uint16_t a, uint16_t b)
        {
            if constexpr (OP == 0)
                return silu_mul1(a, b);
            else
                return f_to_bf(bf_to_f(a) + bf_to_f(b));
        }

        // OP 0: out = silu(a) * b.  OP 1: out = a + b (out == a for add_inplace).
        // Blocks of BLOCK threads take tiles of BLOCK * U vectors; each thread
        // handles U vectors spaced BLOCK apart.
        template <int OP, int U, int NTM, int PR, int BLOCK>
        __global__ __launch_bounds__(BLOCK) void binary_vec_kernel(
            const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t nvec, int64_t n)
        {
            const Vec8 *av = reinterpret_cast<const Vec8 *>(a);
            const Vec8 *bv = reinterpret_cast<const Vec8 *>(b);
            Vec8 *ov = reinterpret_cast<Vec8 *>(out);
            const int64_t tile = blockIdx.x;
            const int64_t base = tile * (BLOCK * U) + threadIdx.x;

            Vec8 x[U], y[U];
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(PR);
#pragma unroll
            for (int i = 0; i < U; ++i)
            {
                const int64_t j = base + static_cast<int64_t>(i) * BLOCK;
                if (j < nvec)
                {
                    x[i] = load8<nt_load(NTM)>(av + j);
                    y[i] = load8<nt_load(NTM)>(bv + j);
                }
            }
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int i = 0; i < U; ++i)
            {
                const int64_t j = base + static_cast<int64_t>(i) * BLOCK;
                if (j < nvec)
                    store8<nt_store(NTM)>(ov + j, apply8<OP>(x[i], y[i]));
            }

            if (tile == 0)
            {
                for (int64_t e = nvec * 8 + threadIdx.x; e < n; e += BLOCK)
                    out[e] = apply1<OP>(a[e], b[e]);
            }
        }

        // Small launches (a decode step): 4 elements (64 bits) per lane, so
        // twice the waves of the 128-bit kernel with half the arithmetic each
        // (SwiGLU at [64, 12288] replayed from a HIP graph: 2.06 against
        // 2.20 us), and write-through stores.  The n % 4 tail is finished by
        // a scalar pass in the first block.
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

        template <int POLICY>
        __device__ __forceinline__ void store_words2(uint32_t *p, u32x2 v)
        {
            if constexpr (POLICY == kStoreStream)
                __asm__ volatile("global_store_dwordx2 %0, %1, off nt sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
            else if constexpr (POLICY == kStoreThrough)
                __asm__ volatile("global_store_dwordx2 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
            else
                *reinterpret_cast<u32x2 *>(p) = v;
        }

        template <int OP, int NTM>
        __global__ __launch_bounds__(kBlock) void binary_half_kernel(const uint16_t *a, const uint16_t *b,
                                                                      uint16_t *out, int64_t nhalf, int64_t n)
        {
            const int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
            if (j < nhalf)
            {
                const u32x2 *ap = reinterpret_cast<const u32x2 *>(a) + j;
                const u32x2 *bp = reinterpret_cast<const u32x2 *>(b) + j;
                const u32x2 x = nt_load(NTM) ? __builtin_nontemporal_load(ap) : *ap;
                const u32x2 y = nt_load(NTM) ? __builtin_nontemporal_load(bp) : *bp;
                const uint32_t xw[2] = {x.x, x.y}, yw[2] = {y.x, y.y};
                uint32_t rw[2];
                if constexpr (OP == 0)
                    silu_mul_words<2>(xw, yw, rw);
                else
                {
                    rw[0] = add2(xw[0], yw[0]);
                    rw[1] = add2(xw[1], yw[1]);
                }
                store_words2<nt_store(NTM)>(reinterpret_cast<uint32_t *>(out) + 2 * j, u32x2{rw[0], rw[1]});
            }
            if (blockIdx.x == 0)
            {
                for (int64_t e = nhalf * 4 + threadIdx.x; e < n; e += kBlock)
                    out[e] = apply1<OP>(a[e], b[e]);
            }
        }

        template <int OP>
        __global__ __launch_bounds__(kBlock) void binary_scalar_kernel(
            const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t n)
        {
            const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
            for (int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < n; e += stride)
                out[e] = apply1<OP>(a[e], b[e]);
        }

        template <int OP>
        int launch_binary(const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t n,
                          hipStream_t stream, const char *name)
        {
            constexpr int U = OP == 0 ? kUnrollSilu : kUnrollAdd;
            constexpr int NTM = OP == 0 ? kNtmSilu : kNtmAdd;
            constexpr int PR = OP == 0 ? kPrioSilu : 0;
            const int64_t nvec = n / 8;
            const bool small = n * 2 <= kSmallLaunchBytes;
            if (OP == 0 && small && aligned_to(a, 8) && aligned_to(b, 8) && aligned_to(out, 8))
            {
                // at most 2M elements: the grid fits one dispatch
                const int64_t nhalf = n / 4;
                const dim3 grid(static_cast<unsigned>(nhalf > 0 ? blocks_for(nhalf, kBlock) : 1));
                binary_half_kernel<OP, ntm_small(NTM)><<<grid, dim3(kBlock), 0, stream>>>(a, b, out, nhalf, n);
            }
            else if (small && aligned16(a) && aligned16(b) && aligned16(out))
            {
                const dim3 grid(static_cast<unsigned>(binary_vec_blocks(n, U)));
                binary_vec_kernel<OP, U, ntm_small(NTM), PR, kBlock><<<grid, dim3(kBlock), 0, stream>>>(a, b, out, nvec, n);
            }
            else if (aligned16(a) && aligned16(b) && aligned16(out) && binary_vec_fits(n, U, kStreamBlock))
            {
                const dim3 grid(static_cast<unsigned>(binary_vec_blocks(n, U, kStreamBlock)));
                binary_vec_kernel<OP, U, NTM, PR, kStreamBlock>
                    <<<grid, dim3(kStreamBlock), 0, stream>>>(a, b, out, nvec, n);
            }
            else
            {
                const int64_t want = (n + kBlock - 1) / kBlock;
                const int64_t grid = want < 65536 ? want : 65536;
                binary_scalar_kernel<OP><<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, stream>>>(a, b, out, n);
            }
            return check_launch(name);
        }

    } // namespace
} // namespace q3k

extern "C" int q3k_silu_mul_bf16(const uint16_t *g, const uint16_t *u, uint16_t *out,
                                 int64_t n, q3k_stream_t stream)
{
    using namespace q3k;
    if (n < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "silu_multiply element count cannot be negative");
    if (n == 0)
        return Q3K_OK;
    if (g == nullptr || u == nullptr || out == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "silu_multiply received a null pointer");
    if (!aligned_to(g, 2) || !aligned_to(u, 2) || !aligned_to(out, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "silu_multiply pointers must be 2-byte aligned");
    return launch_binary<0>(g, u, out, n, reinterpret_cast<hipStream_t>(stream), "silu_multiply");
}

extern "C" int q3k_add_inplace_bf16(uint16_t *d, const uint16_t *s, int64_t n, q3k_stream_t stream)
{
    using namespace q3k;
    if (n < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "add_inplace element count cannot be negative");
    if (n == 0)
        return Q3K_OK;
    if (d == nullptr || s == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "add_inplace received a null pointer");
    if (!aligned_to(d, 2) || !aligned_to(s, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "add_inplace pointers must be 2-byte aligned");
    return launch_binary<1>(d, s, d, n, reinterpret_cast<hipStream_t>(stream), "add_inplace");
}
