// qwen3::KvCache over the gfx950 append kernel.  Checks, their order and
// exception types follow src/model/kv_cache.cpp:17-144 and :274-302 of the
// reference; the rows are written by q3k_kv_append (one launch for K and V).
#include "qwen3/model/kv_cache.h"

#include "../ops/ops_common.hpp"

#include <algorithm>
#include <stdexcept>
#include <string>

namespace qwen3
{
    namespace
    {
        template <typename T>
        T require_positive(T value, const char *name)
        {
            if (value <= 0)
                throw std::invalid_argument(std::string(name) + " must be positive");
            return value;
        }

        DType require_cache_dtype(DType dtype)
        {
            if (dtype != DType::BFloat16 && dtype != DType::Float32)
                throw std::invalid_argument("KV cache supports only bfloat16 or float32");
            return dtype;
        }

        Device require_gpu(Device device)
        {
            if (!device.is_cuda())
                throw std::invalid_argument("KV cache must be stored on CUDA");
            return device;
        }

        Shape storage_shape(std::int32_t layers, std::int64_t batch, std::int64_t seq, std::int32_t heads,
                            std::int32_t head_dim)
        {
            return Shape{layers, batch, seq, heads, head_dim};
        }
    } // namespace

    KvCache::KvCache(std::int32_t num_layers, std::int64_t max_batch_size, std::int64_t max_sequence_length,
                     std::int32_t num_key_value_heads, std::int32_t head_dim, DType dtype, Device device)
        : num_layers_(require_positive(num_layers, "num_layers")),
          max_batch_size_(require_positive(max_batch_size, "max_batch_size")),
          max_sequence_length_(require_positive(max_sequence_length, "max_sequence_length")),
          num_key_value_heads_(require_positive(num_key_value_heads, "num_key_value_heads")),
          head_dim_(require_positive(head_dim, "head_dim")),
          dtype_(require_cache_dtype(dtype)),
          device_(require_gpu(device)),
          key_storage_(Tensor::empty(storage_shape(num_layers_, max_batch_size_, max_sequence_length_,
                                                   num_key_value_heads_, head_dim_),
                                     dtype_, device_)),
          value_storage_(Tensor::empty(storage_shape(num_layers_, max_batch_size_, max_sequence_length_,
                                                     num_key_value_heads_, head_dim_),
                                       dtype_, device_)),
          cached_lengths_(static_cast<std::size_t>(num_layers_), 0)
    {
    }

    KvCache::AppendTarget KvCache::prepare_append(std::int32_t layer_index, std::int64_t start_position,
                                                  const Tensor &key, const Tensor &value)
    {
        validate_layer_index(layer_index);
        if (key.dtype() != dtype_ || value.dtype() != dtype_)
            throw std::invalid_argument("KV cache input dtype does not match cache dtype");
        if (key.device() != device_ || value.device() != device_)
            throw std::invalid_argument("KV cache inputs must be on the cache device");
        if (key.shape().rank() != 3 || value.shape().rank() != 3)
            throw std::invalid_argument("KV cache inputs must have rank 3");
        if (key.shape() != value.shape())
            throw std::invalid_argument("KV cache key and value shape must match");
        const std::int64_t batch = key.shape()[0];
        const std::int64_t sequence = key.shape()[1];
        if (batch <= 0 || sequence <= 0)
            throw std::invalid_argument("KV cache input batch and sequence dimensions must be positive");
        if (batch > max_batch_size_)
            throw std::out_of_range("KV cache batch size exceeds capacity");
        if (key.shape()[2] != static_cast<std::int64_t>(num_key_value_heads_) * head_dim_)
            throw std::invalid_argument("KV cache projection size does not match num_key_value_heads * head_dim");
        if (start_position != cached_lengths_[static_cast<std::size_t>(layer_index)])
            throw std::logic_error("KV cache append must start at the current cached length");
        if (start_position < 0 || start_position > max_sequence_length_ ||
            sequence > max_sequence_length_ - start_position)
            throw std::out_of_range("KV cache append exceeds sequence capacity");
        if (active_batch_size_ != 0 && batch != active_batch_size_)
            throw std::invalid_argument("KV cache batch size cannot change before reset");
        return AppendTarget{layer_data(key_storage_, layer_index), layer_data(value_storage_, layer_index), batch,
                            sequence};
    }

    void KvCache::commit_append(std::int32_t layer_index, std::int64_t start_position, const AppendTarget &target)
    {
        validate_layer_index(layer_index);
        if (active_batch_size_ == 0)
            active_batch_size_ = target.batch;
        cached_lengths_[static_cast<std::size_t>(layer_index)] = start_position + target.sequence;
    }

    void KvCache::append(std::int32_t layer_index, std::int64_t start_position, const Tensor &key, const Tensor &value)
    {
        const AppendTarget target = prepare_append(layer_index, start_position, key, value);
        const std::int64_t row_bytes =
            static_cast<std::int64_t>(num_key_value_heads_) * head_dim_ * static_cast<std::int64_t>(dtype_size(dtype_));
        ops::detail::launch_on(device_, [&](q3k_stream_t stream) {
            return q3k_kv_append(key.data(), value.data(), target.key_layer, target.value_layer, target.batch,
                                 target.sequence, row_bytes, max_sequence_length_, start_position, stream);
        });
        commit_append(layer_index, start_position, target);
    }

    void KvCache::reset() noexcept
    {
        std::fill(cached_lengths_.begin(), cached_lengths_.end(), 0);
        active_batch_size_ = 0;
    }

    std::int64_t KvCache::cached_length(std::int32_t layer_index) const
    {
        validate_layer_index(layer_index);
        return cached_lengths_[static_cast<std::size_t>(layer_index)];
    }

    std::int64_t KvCache::active_batch_size() const noexcept { return active_batch_size_; }

    TensorView KvCache::key_view(std::int32_t layer_index) { return layer_view(key_storage_, layer_index); }

    TensorView KvCache::value_view(std::int32_t layer_index) { return layer_view(value_storage_, layer_index); }

    void KvCache::validate_layer_index(std::int32_t layer_index) const
    {
        if (layer_index < 0 || layer_index >= num_layers_)
            throw std::out_of_range("KV cache layer index is out of range");
    }

    void *KvCache::layer_data(const Tensor &storage, std::int32_t layer_index) const
    {
        const std::int64_t layer_elements =
            max_batch_size_ * max_sequence_length_ * static_cast<std::int64_t>(num_key_value_heads_) * head_dim_;
        const auto offset = static_cast<std::size_t>(layer_index) * static_cast<std::size_t>(layer_elements) *
                            dtype_size(dtype_);
        return static_cast<std::byte *>(const_cast<void *>(storage.data())) + offset;
    }

    TensorView KvCache::layer_view(Tensor &storage, std::int32_t layer_index)
    {
        validate_layer_index(layer_index);
        const std::int64_t row = static_cast<std::int64_t>(num_key_value_heads_) * head_dim_;
        return TensorView{layer_data(storage, layer_index), dtype_, device_,
                          Shape{active_batch_size_, cached_lengths_[static_cast<std::size_t>(layer_index)],
                                num_key_value_heads_, head_dim_},
                          std::vector<std::int64_t>{max_sequence_length_ * row, row, head_dim_, 1}};
    }
} // namespace qwen3
