// Shared device helpers for the gfx950 kernels: bf16 packing, 128-bit
// vectors, DPP lane reductions, and the host-side error slot of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "q3k_abi.h"
#include "q3k_bench.h"

namespace q3k
{
    constexpr int kWave = 64;

    // Eight bf16 values (16 bytes); element 2i sits in the low half of d[i].
    struct alignas(16) Vec8
    {
        uint32_t d[4];
    };

    // Four fp32 values (16 bytes).
    struct alignas(16) F4
    {
        float v[4];
    };

    __device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
    __device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
    __device__ __forceinline__ float bf_to_f(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

    // Round two floats to bf16 (round-to-nearest-even) and pack them; gfx950
    // lowers this to one v_cvt_pk_bf16_f32.
    __device__ __forceinline__ uint32_t pack_rne(float lo, float hi)
    {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        bf16x2 r;
        r.x = static_cast<__bf16>(lo);
        r.y = static_cast<__bf16>(hi);
        return __builtin_bit_cast(uint32_t, r);
    }

    __device__ __forceinline__ uint16_t f_to_bf(float v)
    {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }

    // Value of lane CTRL-permuted within the wave (DPP, no LDS traffic).
    template <int CTRL>
    __device__ __forceinline__ float dpp_f(float v)
    {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
    }

    template <int CTRL>
    __device__ __forceinline__ uint32_t dpp_u(uint32_t v)
    {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xf, 0xf, false));
    }

    // DPP controls used below.
    constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
    constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
    constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7-i within each 8 lanes
    constexpr int kDppMirror = 0x140;      // lane i <- lane 15-i within each 16 lanes
    constexpr int kDppRowRor8 = 0x128;     // lane i <- lane (i+8) mod 16 within each 16 lanes

    // Sum over aligned groups of G consecutive lanes.  Every lane of a group
    // receives the bit-identical total (each step adds a commutative pair).
    template <int G>
    __device__ __forceinline__ float group_sum(float v)
    {
        static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
        if constexpr (G >= 2)
            v += dpp_f<kDppQuadXor1>(v);
        if constexpr (G >= 4)
            v += dpp_f<kDppQuadXor2>(v);
        if constexpr (G >= 8)
            v += dpp_f<kDppHalfMirror>(v);
        if constexpr (G >= 16)
            v += dpp_f<kDppMirror>(v);
        if constexpr (G >= 32)
            v += __shfl_xor(v, 16, 64);
        if constexpr (G >= 64)
            v += __shfl_xor(v, 32, 64);
        return v;
    }

    // Sum of the squares of eight bf16 values, pairwise (exact products).
    __device__ __forceinline__ float sum_sq8(const Vec8 &x)
    {
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const float a = bf_lo(x.d[i]);
            const float b = bf_hi(x.d[i]);
            s[i] = a * a + b * b;
        }
        return (s[0] + s[1]) + (s[2] + s[3]);
    }

    // 1 / sqrt(sum / n + eps) with IEEE-rounded divide and square root.
    __device__ __forceinline__ float inverse_rms(float sum, float n, float eps)
    {
        return 1.0f / sqrtf(sum / n + eps);
    }

    // y = RNE(RNE(x * inv) * w) for eight elements.
    __device__ __forceinline__ Vec8 norm_scale8(const Vec8 &x, const Vec8 &w, float inv)
    {
        Vec8 y;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const uint32_t n = pack_rne(bf_lo(x.d[i]) * inv, bf_hi(x.d[i]) * inv);
            y.d[i] = pack_rne(bf_lo(n) * bf_lo(w.d[i]), bf_hi(n) * bf_hi(w.d[i]));
        }
        return y;
    }

    // ---- host side: per-thread error slot of the C ABI -------------------
    int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
    int check_launch(const char *kernel_name);

    inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

    // Natural alignment of an element pointer (2 for bf16, 4 for int32/float).
    inline bool aligned_to(const void *p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; }

    // Blocks of 256 threads (four waves) unless stated otherwise.
    constexpr int kBlock = 256;
} // namespace q3k
