// Argmax over the last dimension for gfx950 (src/ops/argmax.cu:28-100 of the
// reference: bf16 rows, NaN counts as -inf, ties go to the smaller index,
// int32 indices).
//
// Every candidate becomes one 64-bit key: the bf16 bits mapped to an
// order-preserving unsigned value (NaN -> -inf, -0 -> +0, since the
// reference's float compare treats them as equal) in the high word and
// ~index in the low word, so "larger value, then smaller index" is a plain
// unsigned max.  One block of 1024 threads per row (rows strided over the
// grid): 128-bit loads when the row allows, wave max by lane shuffles, block
// max through LDS.
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        constexpr int kArgmaxBlock = 1024;

        __device__ __forceinline__ uint64_t argmax_key(uint32_t b, uint32_t index)
        {
            if ((b & 0x7fffu) > 0x7f80u)
                b = 0xff80u; // NaN -> -inf
            if (b == 0x8000u)
                b = 0u; // -0 -> +0
            const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
            return (static_cast<uint64_t>(ord) << 32) | (0xffffffffu - index);
        }

        __device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

        template <bool VEC>
        __global__ __launch_bounds__(kArgmaxBlock) void argmax_kernel(const uint16_t *__restrict__ x,
                                                                      int32_t *__restrict__ out, int64_t rows,
                                                                      int64_t stride, int64_t n)
        {
            __shared__ uint64_t wave_best[kArgmaxBlock / kWave];
            const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                const uint16_t *r = x + row * stride;
                uint64_t best = 0; // below every candidate
                int64_t tail = 0;
                if constexpr (VEC)
                {
                    const int64_t nvec = n / 8;
                    const Vec8 *rv = reinterpret_cast<const Vec8 *>(r);
                    // four independent 16-byte loads in flight per thread
                    constexpr int U = 4;
                    int64_t i = threadIdx.x;
                    for (; i + (U - 1) * kArgmaxBlock < nvec; i += U * kArgmaxBlock)
                    {
                        Vec8 v[U];
#pragma unroll
                        for (int u = 0; u < U; ++u)
                            v[u] = rv[i + u * kArgmaxBlock];
#pragma unroll
                        for (int u = 0; u < U; ++u)
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                            {
                                const uint32_t idx = static_cast<uint32_t>(8 * (i + u * kArgmaxBlock) + 2 * j);
                                best = max_u64(best, argmax_key(v[u].d[j] & 0xffffu, idx));
                                best = max_u64(best, argmax_key(v[u].d[j] >> 16, idx + 1));
                            }
                    }
                    for (; i < nvec; i += kArgmaxBlock)
                    {
                        const Vec8 v = rv[i];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                        {
                            const uint32_t idx = static_cast<uint32_t>(8 * i + 2 * j);
                            best = max_u64(best, argmax_key(v.d[j] & 0xffffu, idx));
                            best = max_u64(best, argmax_key(v.d[j] >> 16, idx + 1));
                        }
                    }
                    tail = nvec * 8;
                }
                for (int64_t c = tail + threadIdx.x; c < n; c += kArgmaxBlock)
                    best = max_u64(best, argmax_key(r[c], static_cast<uint32_t>(c)));
#pragma unroll
                for (int off = 32; off > 0; off /= 2)
                    best = max_u64(best, __shfl_xor(best, off, kWave));
                if (lane == 0)
                    wave_best[wave] = best;
                __syncthreads();
                if (wave == 0)
                {
                    best = lane < kArgmaxBlock / kWave ? wave_best[lane] : 0;
#pragma unroll
                    for (int off = 8; off > 0; off /= 2)
                        best = max_u64(best, __shfl_xor(best, off, kWave));
                    if (lane == 0)
                        out[row] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(best));
                }
                __syncthreads(); // wave_best is reused by the next row
            }
        }
    } // namespace
} // namespace q3k

extern "C" int q3k_argmax_bf16(const uint16_t *x, int32_t *out, int64_t rows, int64_t row_stride,
                               int64_t search_size, q3k_stream_t stream)
{
    using namespace q3k;
    if (rows < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax row count cannot be negative");
    if (row_stride <= 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax reduction dimension must be positive");
    if (row_stride > INT32_MAX)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax reduction dimension exceeds Int32 index range");
    if (search_size <= 0 || search_size > row_stride)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "valid reduction size is outside the last dimension");
    if (rows == 0)
        return Q3K_OK;
    if (x == nullptr || out == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax received a null pointer");
    if (!aligned_to(x, 2) || !aligned_to(out, 4))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax pointers must be aligned to their element size");
    if (rows > INT64_MAX / row_stride)
        return set_error(Q3K_ERR_OVERFLOW, "argmax input size overflows");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const unsigned grid = static_cast<unsigned>(rows < 65535 ? rows : 65535);
    if (aligned16(x) && row_stride % 8 == 0)
        argmax_kernel<true><<<dim3(grid), dim3(kArgmaxBlock), 0, s>>>(x, out, rows, row_stride, search_size);
    else
        argmax_kernel<false><<<dim3(grid), dim3(kArgmaxBlock), 0, s>>>(x, out, rows, row_stride, search_size);
    return check_launch("argmax_last_dimension");
}
