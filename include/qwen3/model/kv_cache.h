#pragma once

// Per-layer key/value cache of the Qwen3 runtime on one GPU: storage
// [num_layers, max_batch_size, max_sequence_length, num_key_value_heads,
// head_dim] for keys and for values, one logical length per layer.  The
// contract (constructor checks, append rules and their exception types,
// views with strides) is that of the reference's qwen3::KvCache
// (include/qwen3/model/kv_cache.h, src/model/kv_cache.cpp); the copy is a
// gfx950 kernel (q3k_kv_append) instead of two 2-D memcpys.

#include "qwen3/core/tensor.h"
#include "qwen3/core/tensor_view.h"

#include <cstdint>
#include <vector>

namespace qwen3
{
    class KvCache final
    {
    public:
        KvCache(std::int32_t num_layers, std::int64_t max_batch_size, std::int64_t max_sequence_length,
                std::int32_t num_key_value_heads, std::int32_t head_dim, DType dtype, Device device);
        ~KvCache() = default;
        KvCache(const KvCache &) = delete;
        KvCache &operator=(const KvCache &) = delete;
        KvCache(KvCache &&) noexcept = default;
        KvCache &operator=(KvCache &&) noexcept = default;

        // key / value [batch, sequence, num_key_value_heads * head_dim] go to
        // positions start_position .. + sequence - 1 of layer_index;
        // start_position must equal that layer's cached length.
        void append(std::int32_t layer_index, std::int64_t start_position, const Tensor &key, const Tensor &value);

        // Logical reset: lengths to 0, batch size unset; memory is not cleared.
        void reset() noexcept;

        [[nodiscard]] std::int64_t cached_length(std::int32_t layer_index) const;
        [[nodiscard]] std::int64_t active_batch_size() const noexcept;

        // [active_batch_size, cached_length, num_key_value_heads, head_dim]
        // with strides {max_sequence_length * H * D, H * D, D, 1}: not
        // contiguous when batch > 1 and the layer is not full.
        [[nodiscard]] TensorView key_view(std::int32_t layer_index);
        [[nodiscard]] TensorView value_view(std::int32_t layer_index);

        [[nodiscard]] const Tensor &key_storage() const noexcept { return key_storage_; }
        [[nodiscard]] const Tensor &value_storage() const noexcept { return value_storage_; }
        [[nodiscard]] std::int32_t num_layers() const noexcept { return num_layers_; }
        [[nodiscard]] std::int64_t max_batch_size() const noexcept { return max_batch_size_; }
        [[nodiscard]] std::int64_t max_sequence_length() const noexcept { return max_sequence_length_; }
        [[nodiscard]] std::int32_t num_key_value_heads() const noexcept { return num_key_value_heads_; }
        [[nodiscard]] std::int32_t head_dim() const noexcept { return head_dim_; }
        [[nodiscard]] DType dtype() const noexcept { return dtype_; }
        [[nodiscard]] const Device &device() const noexcept { return device_; }

        // For kernels that write the appended rows themselves (the fused Q/K
        // norm + RoPE + append): prepare_append runs exactly append()'s checks
        // and returns where layer_index's block starts; commit_append then
        // records the append.  Nothing changes between the two.
        struct AppendTarget
        {
            void *key_layer;
            void *value_layer;
            std::int64_t batch;
            std::int64_t sequence;
        };
        [[nodiscard]] AppendTarget prepare_append(std::int32_t layer_index, std::int64_t start_position,
                                                  const Tensor &key, const Tensor &value);
        void commit_append(std::int32_t layer_index, std::int64_t start_position, const AppendTarget &target);

    private:
        void validate_layer_index(std::int32_t layer_index) const;
        [[nodiscard]] TensorView layer_view(Tensor &storage, std::int32_t layer_index);
        [[nodiscard]] void *layer_data(const Tensor &storage, std::int32_t layer_index) const;

        std::int32_t num_layers_ = 0;
        std::int64_t max_batch_size_ = 0;
        std::int64_t max_sequence_length_ = 0;
        std::int32_t num_key_value_heads_ = 0;
        std::int32_t head_dim_ = 0;
        DType dtype_ = DType::BFloat16;
        Device device_ = Device::cpu();
        Tensor key_storage_;
        Tensor value_storage_;
        std::vector<std::int64_t> cached_lengths_;
        std::int64_t active_batch_size_ = 0;
    };
} // namespace qwen3
