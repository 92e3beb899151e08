// Shared device helpers for the gfx950 kernels: bf16 packing, 128-bit
// vectors, DPP lane reductions, and the host-side error slot of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "launch_limits.hpp"
#include "q3k_abi.h"
#include "q3k_bench.h"

namespace q3k
{

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

    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

    // 128-bit global load / store.  NT = true marks the access non-temporal
    // (streamed data that is not re-read soon), which keeps it from
    // displacing reused lines and measurably raises HBM throughput on gfx950.
    template <bool NT>
    __device__ __forceinline__ Vec8 load8(const Vec8 *p)
    {
        u32x4 v;
        if constexpr (NT)
            v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
        else
            v = *reinterpret_cast<const u32x4 *>(p);
        Vec8 r;
        r.d[0] = v.x;
        r.d[1] = v.y;
        r.d[2] = v.z;
        r.d[3] = v.w;
        return r;
    }

    // Store policies of the 128-bit store.
    //   kStoreStream (`nt sc1`): a streaming store with device scope.  The
    //     eight XCDs of MI355X each have their own L2, and a store at device
    //     scope is written through it instead of leaving a dirty line that the
    //     end of the kernel has to write back before the next kernel may
    //     start.  Measured on a 64 MB -> 64 MB copy: 72.8% of peak HBM with
    //     `nt` alone, 76.1% with `nt sc1`.
    //   kStoreThrough (`sc1`): written through at device scope without the
    //     non-temporal hint.  For launches of a few MB that write over what
    //     they have just read (the in-place ops at decode sizes) it is
    //     faster: a 1 MB in-place copy replayed from a HIP graph took 1.97 us
    //     against 2.18 us with `nt sc1`, add + RMSNorm [64, 4096] 2.41 against
    //     2.69 us; out of place the two are equal, and at 64 MB `nt sc1` is 2%
    //     faster.
    // No compiler builtin sets sc1 on a global store, hence the asm.  A
    // 128-bit store reads its data VGPRs a few cycles after it issues, and a
    // VALU write to them in that window corrupts the store; for its own
    // stores the compiler keeps such a write two wait states back (`s_nop 1`),
    // but it cannot see into the asm, so the asm carries those wait states
    // itself.  A store returns nothing, so there is no counter wait for the
    // compiler to track.
    constexpr int kStorePlain = 0;
    constexpr int kStoreStream = 1;
    constexpr int kStoreThrough = 2;

    template <int POLICY>
    __device__ __forceinline__ void store8(Vec8 *p, const Vec8 &r)
    {
        u32x4 v;
        v.x = r.d[0];
        v.y = r.d[1];
        v.z = r.d[2];
        v.w = r.d[3];
        if constexpr (POLICY == kStoreStream)
            __asm__ volatile("global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
        else if constexpr (POLICY == kStoreThrough)
            __asm__ volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
        else
            *reinterpret_cast<u32x4 *>(p) = v;
    }

    __device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
    __device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
    __device__ __forceinline__ float bf_to_f(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

    // Round two floats to bf16 (round-to-nearest-even) and pack them: one
    // v_cvt_pk_bf16_f32.  The empty asm makes the packed word opaque, so that
    // a later bf_lo/bf_hi of it stays a shift/mask of this one conversion
    // instead of being rewritten into a separate convert per element.
    __device__ __forceinline__ uint32_t pack_rne(float lo, float hi)
    {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        bf16x2 r;
        r.x = static_cast<__bf16>(lo);
        r.y = static_cast<__bf16>(hi);
        uint32_t v = __builtin_bit_cast(uint32_t, r);
        __asm__("" : "+v"(v));
        return v;
    }

    __device__ __forceinline__ uint16_t f_to_bf(float v)
    {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }

    // Value of lane CTRL-permuted within the wave (DPP, no LDS traffic).
    // Every control used here reads a lane inside the same 16-lane row, so
    // bound_ctrl (zero for out-of-row sources) never applies; setting it lets
    // the compiler fold the move into the consuming add/mul (v_add_f32_dpp).
    template <int CTRL>
    __device__ __forceinline__ float dpp_f(float v)
    {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
    }

    template <int CTRL>
    __device__ __forceinline__ uint32_t dpp_u(uint32_t v)
    {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xf, 0xf, true));
    }

    // DPP controls used below.
    constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
    constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
    constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7-i within each 8 lanes
    constexpr int kDppMirror = 0x140;      // lane i <- lane 15-i within each 16 lanes
    constexpr int kDppRowRor8 = 0x128;     // lane i <- lane (i+8) mod 16 within each 16 lanes

    // Sum over aligned groups of G consecutive lanes.  Every lane of a group
    // receives the bit-identical total (each step adds a commutative pair).
    // Across 16-lane rows the partner value comes from v_permlane16_swap /
    // v_permlane32_swap (VALU, no LDS round trip): after a swap of v with
    // itself one result holds the even row (lower half) and the other the odd
    // row (upper half), so their sum is the pair's total in every lane.
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
        {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        if constexpr (G >= 64)
        {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        return v;
    }

    // Sum of the squares of eight bf16 values in element order, one product
    // and seven fused multiply-adds (each square is exact in fp32).  The
    // fused Q/K norm + RoPE kernel runs four heads per lane through this;
    // the pairwise form cost it 6% (28.8 against 27.0 us at config 4).
    __device__ __forceinline__ float sum_sq8(const Vec8 &x)
    {
        float s = bf_lo(x.d[0]) * bf_lo(x.d[0]);
        s = __builtin_fmaf(bf_hi(x.d[0]), bf_hi(x.d[0]), s);
#pragma unroll
        for (int i = 1; i < 4; ++i)
        {
            s = __builtin_fmaf(bf_lo(x.d[i]), bf_lo(x.d[i]), s);
            s = __builtin_fmaf(bf_hi(x.d[i]), bf_hi(x.d[i]), s);
        }
        return s;
    }

    // 1 / sqrt(sum * inv_n + eps) with the hardware reciprocal square root
    // (v_rsq_f32, measured within 0.9 ulp; the reference uses CUDA rsqrtf).
    // inv_n = 1/N is exact for the power-of-two widths of the model (128,
    // 1024, 4096) and within half an ulp otherwise.
    __device__ __forceinline__ float inverse_rms(float sum, float inv_n, float eps)
    {
        return __builtin_amdgcn_rsqf(sum * inv_n + eps);
    }

    // Workgroups are dispatched round-robin over the 8 XCDs (block b runs on
    // XCD b % 8).  With REMAP the block works on tile (b % 8) * (n / 8) + b / 8
    // instead, so each XCD streams one contiguous eighth of the tiles; tiles
    // past the last multiple of 8 keep their own index.
    template <bool REMAP>
    __device__ __forceinline__ uint32_t tile_index(uint32_t block, uint32_t blocks)
    {
        if constexpr (!REMAP)
            return block;
        const uint32_t per = blocks / 8;
        if (block >= per * 8)
            return block;
        return (block % 8) * per + block / 8;
    }

    // NT mode bits of a kernel: bit 0 = non-temporal loads, bit 1 = streaming
    // stores (`nt sc1`), bit 2 = write-through stores (`sc1`, small launches;
    // takes precedence over bit 1).
    constexpr int kNtmThroughStores = 4;
    constexpr bool nt_load(int ntm) { return (ntm & 1) != 0; }
    constexpr int nt_store(int ntm)
    {
        return (ntm & kNtmThroughStores) != 0 ? kStoreThrough : (ntm & 2) != 0 ? kStoreStream : kStorePlain;
    }
    // The mode bits of a small launch (at most kSmallLaunchBytes written):
    // the loads of `ntm`, write-through stores.
    constexpr int ntm_small(int ntm) { return (ntm & 1) | kNtmThroughStores; }

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
} // namespace q3k
