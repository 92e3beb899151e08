/*
 * q3k_bench.h -- measurement aid exported by the same library as q3k_abi.h.
 * It has no counterpart in the reference runtime: it exists so that hardware
 * byte counters (rocprofv3 FETCH_SIZE / WRITE_SIZE) can be calibrated
 * against a kernel whose traffic is known exactly.
 */
#ifndef Q3K_BENCH_H
#define Q3K_BENCH_H

#include "q3k_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dst[0 .. bytes) = src[0 .. bytes) with 128-bit loads and stores; bytes a
 * multiple of 16, both pointers 16-byte aligned, no overlap. */
Q3K_API int q3k_bench_copy_u128(const void *src, void *dst, int64_t bytes, q3k_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif
