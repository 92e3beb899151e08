/*
 * q3k_bench.h -- measurement aids of the benchmark, exported by their own
 * library (lib/libq3k_bench.so), not by the product library libq3k.so.  No
 * counterpart in the reference runtime: they exist so that hardware byte
 * counters (rocprofv3 FETCH_SIZE / WRITE_SIZE) can be calibrated against a
 * kernel whose traffic is known exactly, and to give the stream ceilings the
 * kernels are compared with.  Status codes are those of q3k_abi.h; the
 * message of the last failure on the calling thread comes from
 * q3k_bench_last_error_string().
 */
#ifndef Q3K_BENCH_H
#define Q3K_BENCH_H

#include "q3k_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failing call of this library on the calling thread. */
Q3K_API const char *q3k_bench_last_error_string(void);

/* dst[0 .. bytes) = src[0 .. bytes) with 128-bit loads and stores; bytes a
 * multiple of 16, both pointers 16-byte aligned, no overlap. */
Q3K_API int q3k_bench_copy_u128(const void *src, void *dst, int64_t bytes, q3k_stream_t stream);

/* One or two streams in, one or two out, over `bytes` bytes each, with
 * 128-bit loads and stores and no arithmetic to speak of: out0 = in0 XOR in1,
 * out1 = in0 + in1 word by word (in1 and out1 nullable; a missing in1 reads
 * as zero).  out0 may be in0 (in place).  The access pattern of a streaming op
 * at its size: silu_mul is (g, u) -> out, add + RMSNorm (h, d) -> (h, y), the
 * in-place RoPE q -> q.  One 16-byte vector per thread, `threads` threads per
 * block (64 .. 1024, a multiple of 64: the block size sets how finely the
 * streams are spread over the XCDs, which moves the rate by several points).
 * bytes a multiple of 16, pointers 16-byte aligned. */
Q3K_API int q3k_bench_stream_u128(const void *in0, const void *in1, void *out0, void *out1, int64_t bytes,
                                  int32_t threads, q3k_stream_t stream);

/* Read ceiling of a strided row layout such as a KV-cache view: outer x inner
 * views, view (o, i) at base + o * outer_stride + i * inner_stride, each
 * `rows` rows of row_bytes at row_stride (bytes; strides multiples of 16,
 * row_bytes a power of two from 16 to 4096).  base2 (nullable) is read with
 * the same layout (keys and values).  One 256-thread block per view; the XOR
 * of the data goes to sink[view * 256 + thread] (outer * inner * 256 words). */
Q3K_API int q3k_bench_read_rows_u128(const void *base, const void *base2, int64_t outer, int64_t outer_stride,
                                     int64_t inner, int64_t inner_stride, int64_t rows, int64_t row_stride,
                                     int64_t row_bytes, uint32_t *sink, q3k_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif
