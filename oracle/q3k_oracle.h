/*
 * q3k_oracle.h -- CPU restatement of the reference runtime's arithmetic for
 * the Qwen3 decoder layer's non-GEMM ops.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or, for the CPU baseline, as the timed CPU path).  The product
 * library never links or calls it.
 *
 * Every bf16 value is a uint16_t bit pattern.  Each floating-point op
 * returns a primary result plus, when lo/hi are non-NULL, a per-element band
 * [lo, hi]: the bf16 values an fp32 implementation of the reference could
 * produce given the fp32 noise the reference itself cannot pin (CUDA
 * rsqrtf/expf approximation error, FMA-contraction choice, reduction order).
 * The acceptance rule of the tests is: a kernel value passes when it lies in
 * [lo - 1 ulp, hi + 1 ulp] (bf16 ordered space).  Elements with lo == hi
 * are therefore held to 1 ulp of the primary result.
 */
#ifndef Q3K_ORACLE_H
#define Q3K_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 -> bf16 round-to-nearest-even, as the reference tests' helper
 * float_to_bfloat16 (tests/unit/rms_norm_cuda_test.cpp:28-46) for finite
 * values; NaN maps to the quiet NaN 0x7fc0 (sign kept). */
uint16_t q3o_bf16_from_f32(float x);
float q3o_f32_from_bf16(uint16_t b);

/* Relative fp32 noise bounds used to build the bands. */
double q3o_band_rel_inv(void);   /* on 1/rms */
double q3o_band_rel_silu(void);  /* on silu(g) */

/* src/ops/embedding.cu:29-54 */
void q3o_embedding(const int32_t *ids, int64_t T, const uint16_t *table, int64_t V, int64_t H,
                   uint16_t *out, int nthreads);

/* src/ops/elementwise.cu:28-35, in place; bit-exact (no band). */
void q3o_add_inplace(uint16_t *d, const uint16_t *s, int64_t n, int nthreads);

/* src/ops/rms_norm.cu:82-121 (sum in the kernel's reduction order). */
void q3o_rms_norm(const uint16_t *x, const uint16_t *w, int64_t rows, int64_t N, float eps,
                  uint16_t *y, uint16_t *lo, uint16_t *hi, int nthreads);

/* The reference test's own CPU RMSNorm (tests/unit/rms_norm_cuda_test.cpp:
 * 174-244): fp32 sum of squares in column order; no band. */
void q3o_rms_norm_test_order(const uint16_t *x, const uint16_t *w, int64_t rows, int64_t N, float eps,
                             uint16_t *y, int nthreads);

/* add_inplace then rms_norm on the rounded h (decoder_layer.cpp:78->88). h is updated. */
void q3o_add_rms_norm(uint16_t *h, const uint16_t *d, const uint16_t *w, int64_t rows, int64_t N,
                      float eps, uint16_t *y, uint16_t *lo, uint16_t *hi, int nthreads);

/* src/ops/elementwise.cu:45-66 */
void q3o_silu_mul(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *out,
                  uint16_t *lo, uint16_t *hi, int nthreads);

/* src/ops/rope.cu:267-296: writes P * D floats. Returns 0, or -1 on bad arguments. */
int q3o_build_rope_cache(int64_t P, int32_t D, float theta, float *cache);

/* src/ops/rope.cu:38-85 on x [B, S, heads * D], in place.  positions may be
 * NULL (position = start + s).  A head whose position is outside [0, P) is
 * set to NaN (0x7fc0), the documented rule of the positions form.
 * Returns 0, or -1 on bad arguments. */
int q3o_rope(uint16_t *x, int64_t B, int64_t S, int32_t heads, int32_t D, const float *cache,
             int64_t P, int64_t start, const int32_t *positions, uint16_t *lo, uint16_t *hi,
             int nthreads);

/* rms_norm over each head (weight w[D]) then rope on the rounded result
 * (self_attention.cpp:147-152), in place on one tensor (q or k). */
int q3o_qk_norm_rope(uint16_t *x, const uint16_t *w, int64_t B, int64_t S, int32_t heads, int32_t D,
                     float eps, const float *cache, int64_t P, int64_t start,
                     const int32_t *positions, uint16_t *lo, uint16_t *hi, int nthreads);

/* KV-cache append, src/model/kv_cache.cpp:147-185: two 2-D copies of B rows
 * of S * row_bytes bytes, source pitch S * row_bytes, destination pitch
 * seq_cap * row_bytes, starting at row start of the layer block
 * [batch_cap, seq_cap, row_bytes] that kc / vc point at.  Bit-exact. */
void q3o_kv_append(const void *k, const void *v, void *kc, void *vc, int64_t B, int64_t S, int64_t row_bytes,
                   int64_t seq_cap, int64_t start);

/* Grouped-query attention, src/ops/gqa_attention.cu:20-155 and :304-345:
 * query [B, S, Hq * D]; key/value caches addressed as
 * k[b * ks[0] + j * ks[1] + h * ks[2] + d * ks[3]] (element strides of the
 * [B, cached, Hkv, D] views); query (b, s) sees keys 0 .. start + s, which
 * requires cached == start + S.  Primary: the kernel's order (256-slot tree
 * dot, online softmax with fmaf updates, final divide).  rows (optional)
 * lists row indices (b * S + s) * Hq + h to compute; out/lo/hi hold
 * [nrows or B * S * Hq, D].  Returns 0, or -1 on bad arguments. */
int q3o_gqa_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v, int64_t B, int64_t S, int32_t Hq,
                      int32_t Hkv, int32_t D, int64_t cached, int64_t start, const int64_t *k_strides,
                      const int64_t *v_strides, const int64_t *rows, int64_t nrows, uint16_t *out, uint16_t *lo,
                      uint16_t *hi, int nthreads);

/* Argmax over the last dimension, src/ops/argmax.cu:28-100: per row the
 * index of the largest of x[r * row_stride + 0 .. search_size - 1]; NaN
 * counts as -inf, ties go to the smaller index.  Bit-exact. */
void q3o_argmax(const uint16_t *x, int64_t rows, int64_t row_stride, int64_t search_size, int32_t *out);

/* Sampling, src/generation/sampler.cpp:134-265.  q3o_topk_set: the
 * reference's top-k set of row[0 .. n-1] (every token whose logit is >= the
 * k-th best, ties kept; k <= 0 or >= n keeps all), ids best first (higher
 * logit, then smaller id); returns the count, or -1 for a non-finite logit.
 * q3o_sample_row: the whole per-row algorithm (temperature, top-k, sort,
 * stable softmax in double, top-p, draw) given the uniform u in [0, 1) the
 * reference takes from its mt19937_64 (:34-43); returns the token id, or -1
 * for a non-finite logit. */
int64_t q3o_topk_set(const uint16_t *row, int64_t n, int32_t k, int32_t *ids);
int32_t q3o_sample_row(const uint16_t *row, int64_t n, float temperature, int32_t top_k, float top_p, double u);

/* Comparison of kernel output against (primary, lo, hi).
 * stats[0] = elements, [1] = failures (outside [lo-1, hi+1]),
 * [2] = first failing index or -1, [3] = ambiguous elements (lo != hi),
 * [4..7] = histogram of |got - primary| in ulps: 0, 1, 2, >2 (NaN mismatch counts as >2). */
void q3o_compare_band(const uint16_t *got, const uint16_t *primary, const uint16_t *lo,
                      const uint16_t *hi, int64_t n, int64_t *stats);

/* Distance in bf16 ulps between two bit patterns (ordered space; +0 == -0;
 * two NaNs are 0 apart, a NaN and a number are INT32_MAX apart). */
int32_t q3o_ulp_distance(uint16_t a, uint16_t b);

#ifdef __cplusplus
}
#endif

#endif
