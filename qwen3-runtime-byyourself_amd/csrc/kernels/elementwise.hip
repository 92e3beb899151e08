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
        // XCD-contiguous tile remapping measured slower for both streams.
        constexpr bool kRemapSilu = false;
        constexpr bool kRemapAdd = false;
        constexpr int kUnrollAdd = 1;
        constexpr int kNtmAdd = 3;

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

        // silu(g) = g / (1 + exp(-g)) for eight packed values, as
        // g * rcp(1 + exp(-g)): v_rcp_f32 is within 1 ulp, the whole
        // expression within about 3.5 ulp of the exact value.  v_rcp_f32
        // flushes denormal results, so a group holding a denominator >= 2^126
        // (g in [-88.72, -87.3]) or +inf (exp(-g) overflow, g < -88.72) takes
        // the IEEE divide instead; there g / inf is the signed zero that the
        // reference's g / (1 + expf(-g)) gives.  The branch is wave-uniform
        // in practice and never taken on ordinary activations.
        __device__ __forceinline__ void silu8(const uint32_t g[4], float s[8])
        {
            float gv[8], den[8];
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                gv[2 * k] = bf_lo(g[k]);
                gv[2 * k + 1] = bf_hi(g[k]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
                den[j] = 1.0f + exp_f32(-gv[j]);
            const float m = fmaxf(fmaxf(fmaxf(den[0], den[1]), fmaxf(den[2], den[3])),
                                  fmaxf(fmaxf(den[4], den[5]), fmaxf(den[6], den[7])));
            const bool fast = m < 0x1p126f || m != m;
            // The test is per lane, but its outcome is tested for the whole
            // wave first: a lane-divergent if/else is issued on both sides
            // under exec masks, and the IEEE divide would then cost every
            // element ~12 more VALU ops.
            if (__all(fast))
            {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    s[j] = gv[j] * __builtin_amdgcn_rcpf(den[j]);
            }
            else
            {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    s[j] = fast ? gv[j] * __builtin_amdgcn_rcpf(den[j]) : gv[j] / den[j];
            }
        }

        __device__ __forceinline__ Vec8 silu_mul8(const Vec8 &g, const Vec8 &u)
        {
            float s[8];
            silu8(g.d, s);
            Vec8 r;
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const uint32_t n = pack_rne(s[2 * k], s[2 * k + 1]);
                r.d[k] = pack_rne(bf_lo(n) * bf_lo(u.d[k]), bf_hi(n) * bf_hi(u.d[k]));
            }
            return r;
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
        // Each thread handles U vectors spaced one block apart.
        template <int OP, int U, int NTM, int PR, bool REMAP>
        __global__ __launch_bounds__(kBlock) void binary_vec_kernel(
            const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t nvec, int64_t n)
        {
            const Vec8 *av = reinterpret_cast<const Vec8 *>(a);
            const Vec8 *bv = reinterpret_cast<const Vec8 *>(b);
            Vec8 *ov = reinterpret_cast<Vec8 *>(out);
            const int64_t tile = tile_index<REMAP>(blockIdx.x, gridDim.x);
            const int64_t base = tile * (kBlock * U) + threadIdx.x;

            Vec8 x[U], y[U];
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(PR);
#pragma unroll
            for (int i = 0; i < U; ++i)
            {
                const int64_t j = base + static_cast<int64_t>(i) * kBlock;
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
                const int64_t j = base + static_cast<int64_t>(i) * kBlock;
                if (j < nvec)
                    store8<nt_store(NTM)>(ov + j, apply8<OP>(x[i], y[i]));
            }

            if (tile == 0)
            {
                for (int64_t e = nvec * 8 + threadIdx.x; e < n; e += kBlock)
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
            constexpr bool REMAP = OP == 0 ? kRemapSilu : kRemapAdd;
            const int64_t nvec = n / 8;
            if (aligned16(a) && aligned16(b) && aligned16(out) && binary_vec_fits(n, U))
            {
                const dim3 grid(static_cast<unsigned>(binary_vec_blocks(n, U)));
                binary_vec_kernel<OP, U, NTM, PR, REMAP><<<grid, dim3(kBlock), 0, stream>>>(a, b, out, nvec, n);
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
