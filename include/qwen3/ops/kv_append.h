#pragma once

// The attention prologue's non-GEMM tail in one pass: per-head Q/K RMSNorm,
// RoPE, and the KV-cache append.

#include "qwen3/core/tensor.h"
#include "qwen3/model/kv_cache.h"

#include <cstdint>

namespace qwen3::ops
{
    // query = rope(rms_norm(query, q_weight)) in place; rope(rms_norm(key,
    // k_weight)) and value are appended to layer_index of kv_cache at
    // start_position, which is both the first RoPE position and the layer's
    // cached length.  key and value are only read.  Equal, bit for bit, to
    // the reference's sequence at src/model/self_attention.cpp:147-156:
    //   query = rms_norm(query, q_weight, eps); key = rms_norm(key, k_weight, eps);
    //   apply_rope_inplace(query, key, rope_cache, Hq, Hkv, start_position);
    //   kv_cache.append(layer_index, start_position, key, value);
    // with the same checks and exception types (RoPE first, then the cache).
    // The cache must be BFloat16.
    void qk_norm_rope_kv_append(Tensor &query, const Tensor &key, const Tensor &value, const Tensor &q_weight,
                                const Tensor &k_weight, float epsilon, const Tensor &rope_cache,
                                std::int32_t num_query_heads, std::int32_t num_key_value_heads,
                                std::int64_t start_position, KvCache &kv_cache, std::int32_t layer_index);
} // namespace qwen3::ops
