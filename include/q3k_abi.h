/*
 * q3k_abi.h -- C ABI of the MI355X (gfx950) kernels for the Qwen3 decoder
 * layer's non-GEMM ops.
 *
 * Every entry point takes plain device pointers and sizes, launches
 * asynchronously on the given HIP stream (NULL = the legacy default stream,
 * as the reference's ops use) and returns a q3k_status.  Nothing here
 * allocates device memory, synchronises, switches the current device or
 * throws.  The caller owns every buffer.  On a non-zero status the message is
 * available from q3k_last_error_string() on the same host thread.
 *
 * Element types: bf16 buffers are uint16_t bit patterns (IEEE bfloat16),
 * token ids and positions are int32_t, the RoPE table is float
 * [positions, head_dim / 2, 2] with (cos, sin) pairs.
 *
 * Rounding contract (bf16 out, fp32 arithmetic, round-to-nearest-even at the
 * same points as the reference kernels):
 *   add          d = RNE(d + s)
 *   rms_norm     y = RNE(RNE(x * inv) * w),  inv = 1 / sqrt(sum(x^2)/N + eps)
 *   silu_mul     o = RNE(RNE(g / (1 + exp(-g))) * u)
 *   rope         x1' = RNE(x1*c - x2*s), x2' = RNE(x2*c + x1*s), pairs (p, p + D/2)
 *   add_rms_norm h = RNE(h + d); y = rms_norm(h) computed from the rounded h
 *   qk_norm_rope per head: n = rms_norm(x) (two roundings), then rope(n)
 */
#ifndef Q3K_ABI_H
#define Q3K_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define Q3K_API __attribute__((visibility("default")))
#else
#define Q3K_API
#endif

/* Same object as hipStream_t (a pointer to the runtime's opaque stream);
 * declared here so that C callers need no HIP header. */
struct ihipStream_t;
typedef struct ihipStream_t *q3k_stream_t;

typedef enum q3k_status {
    Q3K_OK = 0,
    Q3K_ERR_INVALID_ARGUMENT = 1, /* std::invalid_argument in the C++ ops layer */
    Q3K_ERR_OUT_OF_RANGE = 2,     /* std::out_of_range */
    Q3K_ERR_OVERFLOW = 3,         /* std::overflow_error */
    Q3K_ERR_HIP = 4               /* std::runtime_error (HIP launch/runtime failure) */
} q3k_status;

/* Message for the last non-zero status returned on this host thread. */
Q3K_API const char *q3k_last_error_string(void);

/* Library version, "major.minor.patch". */
Q3K_API const char *q3k_version(void);

/*
 * Embedding gather: out[t, :] = table[ids[t], :] for t in [0, T); a row of
 * +0.0 for ids outside [0, V).  Bit-exact copy.
 * Replaces qwen3::ops::embedding_lookup, src/ops/embedding.cu:85-149
 * (kernel :23-55, out-of-range rule :38-45).
 */
Q3K_API int q3k_embedding_bf16(const int32_t *ids, int64_t T,
                       const uint16_t *table, int64_t V, int64_t H,
                       uint16_t *out, q3k_stream_t stream);

/*
 * RMSNorm over contiguous chunks of N elements: rows = numel / N.  N may be
 * the head dimension of packed heads ([.., heads * N] with weight [N]).
 * y must not overlap x.
 * Replaces qwen3::ops::rms_norm, src/ops/rms_norm.cu:218-267 (kernel :69-127).
 */
Q3K_API int q3k_rms_norm_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y,
                      int64_t rows, int64_t N, float eps, q3k_stream_t stream);

/*
 * Fused residual add + RMSNorm: h = RNE(h + d) written back in place, then
 * y = rms_norm(h, w).  y must not overlap h or d.
 * Replaces the pair add_inplace -> rms_norm at src/model/decoder_layer.cpp:78->88
 * and :94 -> the next layer's :72 (or src/model/model.cpp:146 after the last
 * layer); ops at src/ops/elementwise.cu:133-157 and src/ops/rms_norm.cu:218-267.
 */
Q3K_API int q3k_add_rms_norm_bf16(uint16_t *h, const uint16_t *d, const uint16_t *w,
                          uint16_t *y, int64_t rows, int64_t N, float eps,
                          q3k_stream_t stream);

/*
 * RMSNorm of selected rows into a compact output: y row i = rms_norm(x row
 * first_row + i * row_stride), i in [0, count).  With first_row = S - 1 and
 * row_stride = S over x [B, S, N] this is the final norm of the last token of
 * every sequence, the only rows the LM head reads.
 * Replaces rms_norm at src/model/model.cpp:146 followed by the last-token
 * select of src/model/lm_head.cpp:123-181.
 */
Q3K_API int q3k_rms_norm_rows_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y,
                           int64_t count, int64_t first_row, int64_t row_stride,
                           int64_t N, float eps, q3k_stream_t stream);

/*
 * Fused residual add + RMSNorm of selected rows: for i in [0, count), with
 * r = first_row + i * row_stride: h row r = RNE(h row r + d row r) (in place)
 * and y row i = rms_norm(h row r).  Other rows of h are left untouched (after
 * the last layer only the last tokens' residuals are still needed).  The
 * selected rows must be distinct: row_stride 0 with count > 1 is
 * Q3K_ERR_INVALID_ARGUMENT.
 * Replaces add_inplace at src/model/decoder_layer.cpp:94 of the last layer,
 * rms_norm at src/model/model.cpp:146 and the last-token select of
 * src/model/lm_head.cpp:123-181.
 */
Q3K_API int q3k_add_rms_norm_rows_bf16(uint16_t *h, const uint16_t *d, const uint16_t *w,
                               uint16_t *y, int64_t count, int64_t first_row,
                               int64_t row_stride, int64_t N, float eps,
                               q3k_stream_t stream);

/*
 * Fused embedding gather + RMSNorm: hidden[t, :] = table[ids[t], :] (a zero
 * row for ids outside [0, V)), then y = rms_norm(hidden, w).  The table row is
 * read once; hidden (the residual stream) and y are written.
 * Replaces embedding_lookup at src/model/model.cpp:118 followed by the first
 * layer's input rms_norm at src/model/decoder_layer.cpp:72.
 */
Q3K_API int q3k_embedding_rms_norm_bf16(const int32_t *ids, int64_t T,
                                const uint16_t *table, int64_t V, int64_t H,
                                const uint16_t *w, float eps,
                                uint16_t *hidden, uint16_t *y, q3k_stream_t stream);

/*
 * In-place residual add: d[i] = RNE(d[i] + s[i]), n elements.
 * Replaces qwen3::ops::add_inplace, src/ops/elementwise.cu:133-157 (kernel :21-36).
 */
Q3K_API int q3k_add_inplace_bf16(uint16_t *d, const uint16_t *s, int64_t n,
                         q3k_stream_t stream);

/*
 * SwiGLU activation: out[i] = RNE(RNE(silu(g[i])) * u[i]), n elements.
 * out may alias g or u exactly (same pointer), not partially.
 * Replaces qwen3::ops::silu_multiply, src/ops/elementwise.cu:159-190 (kernel :38-67).
 */
Q3K_API int q3k_silu_mul_bf16(const uint16_t *g, const uint16_t *u, uint16_t *out,
                      int64_t n, q3k_stream_t stream);

/*
 * In-place half-split RoPE on x [B, S, heads * D].  Token (b, s) uses
 * position positions[b * S + s] when positions != NULL, else start + s
 * (the reference's scalar form).  The table has P positions; with the scalar
 * form start + S must not exceed P (Q3K_ERR_OUT_OF_RANGE).  With a positions
 * array, a head whose position lies outside [0, P) is overwritten with NaN
 * (the kernel never reads outside the table).
 * Replaces one launch_rope of qwen3::ops::apply_rope_inplace,
 * src/ops/rope.cu:213-247 / :305-342 (kernel :21-86, range check :190-210).
 */
Q3K_API int q3k_rope_bf16(uint16_t *x, int64_t B, int64_t S, int32_t heads, int32_t D,
                  const float *cache, int64_t P, int64_t start,
                  const int32_t *positions, q3k_stream_t stream);

/*
 * In-place half-split RoPE on q [B, S, Hq * D] and k [B, S, Hkv * D] in one
 * launch (one grid over the heads of both tensors), with the position rule,
 * range check and out-of-range behaviour of q3k_rope_bf16; the results equal
 * q3k_rope_bf16 on q, then on k, bit for bit.  q and k must not overlap.
 * Replaces both launch_rope calls of qwen3::ops::apply_rope_inplace,
 * src/ops/rope.cu:305-342 (one launch each for query and key, :326-332).
 */
Q3K_API int q3k_rope_qk_bf16(uint16_t *q, uint16_t *k, int64_t B, int64_t S,
                  int32_t Hq, int32_t Hkv, int32_t D,
                  const float *cache, int64_t P, int64_t start,
                  const int32_t *positions, q3k_stream_t stream);

/*
 * Fused per-head Q/K RMSNorm + RoPE, in place, one pass over Q [B, S, Hq*D]
 * and K [B, S, Hkv*D] with weights qw[D], kw[D].  Position rule and the
 * out-of-range behaviour are those of q3k_rope_bf16.
 * Replaces the sequence rms_norm(q) -> rms_norm(k) -> apply_rope_inplace at
 * src/model/self_attention.cpp:147-152 (ops src/ops/rms_norm.cu:218-267,
 * src/ops/rope.cu:305-342).
 */
Q3K_API int q3k_qk_norm_rope_bf16(uint16_t *q, uint16_t *k,
                          const uint16_t *qw, const uint16_t *kw,
                          int64_t B, int64_t S, int32_t Hq, int32_t Hkv,
                          int32_t D, float eps,
                          const float *cache, int64_t P, int64_t start,
                          const int32_t *positions, q3k_stream_t stream);

/*
 * Causal grouped-query attention.  q [B, S, Hq * D] bf16 (contiguous);
 * k_cache / v_cache are [B, cached, Hkv, D] bf16 views given by element
 * strides k_strides[4] / v_strides[4] (batch, position, head, dim), e.g. a
 * KV cache layer with strides {Smax * Hkv * D, Hkv * D, D, 1}.  Query
 * (b, s) attends to keys 0 .. start + s; query head h reads KV head
 * h / (Hq / Hkv); scale 1 / sqrt(D).  cached must equal start + S.
 * out [B, S, Hq * D] bf16.  head_dim 128 with unit dim stride and 16-byte
 * aligned rows takes the matrix-core kernel, anything up to 256 the generic
 * one.  workspace (16-byte aligned device memory, may be NULL) of at least
 * q3k_gqa_attention_workspace_bytes(...) bytes lets a launch too small to
 * fill the GPU (decode with few sequences) split the key range across
 * blocks and merge the slices; without it the launch is not split.  Calls
 * that share a workspace must not overlap.
 * Replaces qwen3::ops::grouped_query_attention,
 * src/ops/gqa_attention.cu:304-345 (kernel :20-155, checks :157-302).
 */
Q3K_API int q3k_gqa_attention_bf16(const uint16_t *q, const uint16_t *k_cache,
                          const uint16_t *v_cache, uint16_t *out, int64_t B,
                          int64_t S, int32_t Hq, int32_t Hkv, int32_t D,
                          int64_t cached, int64_t start,
                          const int64_t *k_strides, const int64_t *v_strides,
                          void *workspace, int64_t workspace_bytes,
                          q3k_stream_t stream);

/*
 * Workspace bytes q3k_gqa_attention_bf16 would use to split this shape's
 * key range (0: it does not split).  No counterpart in the reference (its
 * kernel is one block per query row).
 */
Q3K_API int64_t q3k_gqa_attention_workspace_bytes(int64_t B, int64_t S,
                          int32_t Hq, int32_t Hkv, int32_t D, int64_t cached);

/*
 * Argmax over the last dimension: out[r] = index of the largest of
 * x[r * row_stride + 0 .. search_size - 1] (bf16), NaN counted as -inf, ties
 * to the smaller index; int32 out [rows].  search_size in [1, row_stride]
 * (a valid vocabulary prefix of padded logits).  Bit-exact.  workspace
 * (8-byte aligned device memory, may be NULL) of at least
 * q3k_argmax_workspace_bytes(rows, search_size) bytes lets a launch with
 * few rows cut each row into slices searched by separate blocks; the result
 * is the same either way.  Calls that share a workspace must not overlap.
 * Replaces qwen3::ops::argmax_last_dimension, src/ops/argmax.cu:163-214
 * (kernel :34-100), the greedy path of Sampler::sample
 * (src/generation/sampler.cpp:288-291).
 */
Q3K_API int q3k_argmax_bf16(const uint16_t *x, int32_t *out, int64_t rows,
                  int64_t row_stride, int64_t search_size,
                  void *workspace, int64_t workspace_bytes,
                  q3k_stream_t stream);

/*
 * Workspace bytes q3k_argmax_bf16 would use to slice these rows (0: it does
 * not slice).  No counterpart in the reference (its kernel is one block per
 * row).
 */
Q3K_API int64_t q3k_argmax_workspace_bytes(int64_t rows, int64_t search_size);

/*
 * q3k_argmax_bf16 for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops): the same result, with the slice
 * results in a fixed 16 KiB array in device memory that the library holds on
 * each GPU it runs on until the process ends, instead of a caller
 * workspace.  Every input fits it (slicing needs fewer than 8 KiB); a plan
 * needing more returns Q3K_ERR_INVALID_ARGUMENT.  The call itself allocates
 * nothing.  Calls on one GPU share that array, so calls that overlap on one
 * GPU race.  The first call on each GPU looks up the array's device address
 * (a host-side query under a lock); make that call before capturing the
 * entry point into a HIP graph.  No counterpart in the reference.
 */
Q3K_API int q3k_argmax_bf16_noalloc(const uint16_t *x, int32_t *out, int64_t rows,
                  int64_t row_stride, int64_t search_size,
                  q3k_stream_t stream);

/*
 * Top-k candidates of sampling.  For each row r of logits (bf16, row_stride
 * columns, the first search_size searched): every token whose logit is >=
 * the k-th largest logit (ties at the k-th all kept; -0 equals +0), written
 * as cand_index[r * cap + i] / cand_logit[r * cap + i] (bf16 bits) for
 * i < min(count[r], cap), in no particular order; count[r] may exceed cap
 * (then the caller falls back to the whole row).  nonfinite[r] != 0 when
 * the searched row holds a NaN or infinity.  This is the top-k step of the
 * reference's host sampler (temperature is monotone, so it does not change
 * the set), src/generation/sampler.cpp:160-190, moved to the GPU so that
 * only the candidates cross to the host (the reference copies all logits,
 * :296-312).
 */
Q3K_API int q3k_topk_candidates_bf16(const uint16_t *logits, int64_t rows,
                          int64_t row_stride, int64_t search_size, int32_t k,
                          int32_t cap, int32_t *count, int32_t *cand_index,
                          uint16_t *cand_logit, int32_t *nonfinite,
                          void *workspace, int64_t workspace_bytes,
                          q3k_stream_t stream);

/*
 * Workspace bytes q3k_topk_candidates_bf16 would use to cut these rows into
 * slices searched by separate blocks (0: it does not); the workspace (16-byte
 * aligned device memory, may be NULL) changes the speed, not the result, and
 * calls that share one must not overlap.  No counterpart in the reference
 * (its selection runs on the host).
 */
Q3K_API int64_t q3k_topk_workspace_bytes(int64_t rows, int64_t search_size, int32_t k);

/*
 * KV-cache append: K and V [B, S, row_bytes] (contiguous) are copied to rows
 * start .. start + S - 1 of batch rows 0 .. B - 1 of one layer's cache
 * [batch_cap, seq_cap, row_bytes] (key_cache / value_cache point at the
 * layer; the caller guarantees B <= batch_cap).  Bytes are copied unchanged
 * (bf16 or fp32 caches).  start + S > seq_cap is Q3K_ERR_OUT_OF_RANGE.
 * Replaces the two cudaMemcpy2DAsync of qwen3::KvCache::append,
 * src/model/kv_cache.cpp:76-204 (capacity check :121-125).
 */
Q3K_API int q3k_kv_append(const void *key, const void *value, void *key_cache,
                  void *value_cache, int64_t B, int64_t S, int64_t row_bytes,
                  int64_t seq_cap, int64_t start, q3k_stream_t stream);

/*
 * Fused Q/K RMSNorm + RoPE + KV-cache append: Q is normalised and rotated in
 * place as by q3k_qk_norm_rope_bf16; K is normalised and rotated straight
 * into the bf16 key cache and V copied into the value cache, at the rows
 * q3k_kv_append would use (cache_start = the layer's cached length).  K and V
 * are only read.  The results equal q3k_qk_norm_rope_bf16 followed by
 * q3k_kv_append bit for bit.  Cache rows must not overlap q, k or v.
 * Replaces the sequence rms_norm(q) -> rms_norm(k) -> apply_rope_inplace ->
 * kv_cache.append at src/model/self_attention.cpp:147-156
 * (src/model/kv_cache.cpp:76-204).
 */
Q3K_API int q3k_qk_norm_rope_kv_append_bf16(uint16_t *q, const uint16_t *k,
                          const uint16_t *v, const uint16_t *qw,
                          const uint16_t *kw, int64_t B, int64_t S,
                          int32_t Hq, int32_t Hkv, int32_t D, float eps,
                          const float *cache, int64_t P, int64_t start,
                          const int32_t *positions, uint16_t *k_cache,
                          uint16_t *v_cache, int64_t seq_cap,
                          int64_t cache_start, q3k_stream_t stream);

/*
 * Host-side RoPE table: cache[p, i, 0] = (float)cos(p * theta^(-2i/D)),
 * cache[p, i, 1] = (float)sin(...), evaluated in double, for p in [0, P),
 * i in [0, D/2).  Writes P * D floats to host memory.  Same recipe and
 * result as qwen3::ops::build_rope_cache, src/ops/rope.cu:250-303 (before
 * its copy to the device).
 */
Q3K_API int q3k_build_rope_cache_f32(float *host_cache, int64_t P, int32_t D, float theta);

#ifdef __cplusplus
}
#endif

#endif /* Q3K_ABI_H */
