// Measurement aids of the benchmark (include/q3k_bench.h), built into their
// own library, lib/libq3k_bench.so, so that the product library exports only
// the kernels of the op API.  Not part of the runtime: a plain 128-bit copy
// whose bytes are known exactly (to calibrate rocprofv3 FETCH_SIZE /
// WRITE_SIZE and to give the stream ceiling of a launch size), the same with
// one or two streams in and out (an op's own pattern), and a reader of a
// strided row layout (the HBM read ceiling of a KV-cache view).
#include "../csrc/kernels/q3k_common.hpp"

#include <cstdarg>
#include <cstdio>

namespace q3k
{
    namespace
    {
        constexpr int kNtmCopy = 3;
        thread_local char g_bench_error[256] = "";

        int bench_error(int status, const char *message)
        {
            std::snprintf(g_bench_error, sizeof g_bench_error, "%s", message);
            return status;
        }

        int bench_launch_status(const char *what)
        {
            const hipError_t e = hipGetLastError();
            if (e == hipSuccess)
                return Q3K_OK;
            std::snprintf(g_bench_error, sizeof g_bench_error, "%s: %s", what, hipGetErrorString(e));
            return Q3K_ERR_HIP;
        }

        // Plain 128-bit copy used to calibrate hardware byte counters; the same
        // access pattern as the streaming kernels.
        __global__ __launch_bounds__(kBlock) void copy_vec_kernel(const Vec8 *src, Vec8 *dst, int64_t nvec)
        {
            const int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
            if (j < nvec)
                store8<nt_store(kNtmCopy)>(dst + j, load8<nt_load(kNtmCopy)>(src + j));
        }

        // One or two 128-bit streams in, one or two out, with the loads and
        // stores of the streaming ops: out0 = in0 XOR in1, out1 = in0 + in1
        // (word-wise; in1 absent reads as zero).  In place when out0 is in0.
        // The HBM ceiling of an op's access pattern at its size.
        __global__ __launch_bounds__(1024) void stream_vec_kernel(const Vec8 *in0, const Vec8 *in1, Vec8 *out0,
                                                                  Vec8 *out1, int64_t nvec)
        {
            const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
            if (j >= nvec)
                return;
            const Vec8 zero = {{0u, 0u, 0u, 0u}};
            const Vec8 x = load8<nt_load(kNtmCopy)>(in0 + j);
            const Vec8 y = in1 != nullptr ? load8<nt_load(kNtmCopy)>(in1 + j) : zero;
            Vec8 r, t;
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                r.d[k] = x.d[k] ^ y.d[k];
                t.d[k] = x.d[k] + y.d[k];
            }
            store8<nt_store(kNtmCopy)>(out0 + j, r);
            if (out1 != nullptr)
                store8<nt_store(kNtmCopy)>(out1 + j, t);
        }

        // Reads the row views of a KV-cache-like layout with 128-bit loads (one
        // block per view, kReadUnroll row groups in flight per thread) to give
        // the HBM read ceiling of that access pattern.  Everything read is
        // XOR-folded into sink, one word per thread, so the loads stay.
        constexpr int kReadUnroll = 8;
        __global__ __launch_bounds__(kBlock) void read_rows_kernel(const unsigned char *base,
                                                                   const unsigned char *base2, int64_t inner,
                                                                   int64_t outer_stride, int64_t inner_stride,
                                                                   int64_t rows, int64_t row_stride, int chunks,
                                                                   uint32_t *sink)
        {
            const int64_t view = blockIdx.x;
            const int64_t off0 = (view / inner) * outer_stride + (view % inner) * inner_stride;
            const int rows_per_pass = kBlock / chunks;
            const int r_in = static_cast<int>(threadIdx.x) / chunks, c = static_cast<int>(threadIdx.x) % chunks;
            const Vec8 zero = {{0u, 0u, 0u, 0u}};
            uint32_t acc = 0u;
            for (int64_t r0 = 0; r0 < rows; r0 += static_cast<int64_t>(rows_per_pass) * kReadUnroll)
            {
                Vec8 x[kReadUnroll], y[kReadUnroll];
#pragma unroll
                for (int u = 0; u < kReadUnroll; ++u)
                {
                    const int64_t r = r0 + static_cast<int64_t>(u) * rows_per_pass + r_in;
                    x[u] = zero;
                    y[u] = zero;
                    if (r < rows)
                    {
                        const int64_t off = off0 + r * row_stride + 16 * c;
                        x[u] = load8<false>(reinterpret_cast<const Vec8 *>(base + off));
                        if (base2 != nullptr)
                            y[u] = load8<false>(reinterpret_cast<const Vec8 *>(base2 + off));
                    }
                }
#pragma unroll
                for (int u = 0; u < kReadUnroll; ++u)
                    acc ^= (x[u].d[0] + x[u].d[3]) ^ (y[u].d[1] + y[u].d[2]);
            }
            sink[view * kBlock + threadIdx.x] = acc;
        }
    } // namespace
} // namespace q3k

extern "C" const char *q3k_bench_last_error_string(void) { return q3k::g_bench_error; }

extern "C" int q3k_bench_copy_u128(const void *src, void *dst, int64_t bytes, q3k_stream_t stream)
{
    using namespace q3k;
    if (bytes < 0 || bytes % 16 != 0)
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "copy size must be a non-negative multiple of 16 bytes");
    if (bytes == 0)
        return Q3K_OK;
    if (src == nullptr || dst == nullptr || !aligned16(src) || !aligned16(dst))
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "copy pointers must be non-null and 16-byte aligned");
    const int64_t nvec = bytes / 16;
    const int64_t blocks = (nvec + kBlock - 1) / kBlock;
    if (!launch_fits(blocks, kBlock))
        return bench_error(Q3K_ERR_OVERFLOW, "copy size exceeds one launch");
    copy_vec_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const Vec8 *>(src), static_cast<Vec8 *>(dst), nvec);
    return bench_launch_status("bench_copy_u128");
}

extern "C" int q3k_bench_stream_u128(const void *in0, const void *in1, void *out0, void *out1, int64_t bytes,
                                     int32_t threads, q3k_stream_t stream)
{
    using namespace q3k;
    if (bytes < 0 || bytes % 16 != 0)
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "stream size must be a non-negative multiple of 16 bytes");
    if (threads < kWave || threads > 1024 || threads % kWave != 0)
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "stream threads per block must be a multiple of 64 in [64, 1024]");
    if (bytes == 0)
        return Q3K_OK;
    if (in0 == nullptr || out0 == nullptr || !aligned16(in0) || !aligned16(out0) ||
        (in1 != nullptr && !aligned16(in1)) || (out1 != nullptr && !aligned16(out1)))
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "stream pointers must be 16-byte aligned (in0, out0 non-null)");
    const int64_t nvec = bytes / 16;
    const int64_t blocks = blocks_for(nvec, threads);
    if (!launch_fits(blocks, threads))
        return bench_error(Q3K_ERR_OVERFLOW, "stream size exceeds one launch");
    stream_vec_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const Vec8 *>(in0), static_cast<const Vec8 *>(in1), static_cast<Vec8 *>(out0),
        static_cast<Vec8 *>(out1), nvec);
    return bench_launch_status("bench_stream_u128");
}

extern "C" int q3k_bench_read_rows_u128(const void *base, const void *base2, int64_t outer, int64_t outer_stride,
                                        int64_t inner, int64_t inner_stride, int64_t rows, int64_t row_stride,
                                        int64_t row_bytes, uint32_t *sink, q3k_stream_t stream)
{
    using namespace q3k;
    if (outer < 0 || inner < 0 || rows < 0)
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "read view counts cannot be negative");
    if (outer_stride < 0 || inner_stride < 0 || row_stride < 0 || outer_stride % 16 != 0 || inner_stride % 16 != 0 ||
        row_stride % 16 != 0)
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "read strides must be non-negative multiples of 16 bytes");
    if (row_bytes < 16 || row_bytes > 16 * kBlock || (row_bytes & (row_bytes - 1)) != 0)
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "read row size must be a power of two from 16 to 4096 bytes");
    if (outer == 0 || inner == 0 || rows == 0)
        return Q3K_OK;
    if (base == nullptr || sink == nullptr || !aligned16(base) || (base2 != nullptr && !aligned16(base2)) ||
        !aligned_to(sink, 4))
        return bench_error(Q3K_ERR_INVALID_ARGUMENT, "read pointers must be non-null and 16-byte aligned");
    if (outer > INT64_MAX / inner || !launch_fits(outer * inner, kBlock))
        return bench_error(Q3K_ERR_OVERFLOW, "read view count exceeds one launch");
    read_rows_kernel<<<dim3(static_cast<unsigned>(outer * inner)), dim3(kBlock), 0,
                       reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const unsigned char *>(base), static_cast<const unsigned char *>(base2), inner, outer_stride,
        inner_stride, rows, row_stride, static_cast<int>(row_bytes / 16), sink);
    return bench_launch_status("bench_read_rows_u128");
}
