// qwen3::KvCache on the GPU: the reference test's scenario
// (tests/unit/kv_cache_cuda_test.cpp: prefill of 2 tokens and a decode step
// into both layers, view shape and strides, a rejected non-append write,
// reset), the other append rules, and the fused Q/K norm + RoPE + append
// against the reference's op sequence bit for bit.
#include "gpu_util.hpp"
#include "qwen3/model/kv_cache.h"
#include "qwen3/ops/gqa_attention.h"
#include "qwen3/ops/kv_append.h"
#include "qwen3/ops/rms_norm.h"
#include "qwen3/ops/rope.h"

#include <cmath>
#include <cstring>

using qwen3::DType;
using qwen3::KvCache;
using qwen3::Shape;
using qwen3::Tensor;
using test::require;
using test::require_throws;

namespace
{
    // kv_cache_cuda_test.cpp:27-43: bf16(start + 0.25 i), nearest even.
    std::vector<uint16_t> make_values(std::size_t count, float start)
    {
        std::vector<uint16_t> out(count);
        for (std::size_t i = 0; i < count; ++i)
            out[i] = q3o_bf16_from_f32(start + static_cast<float>(i) * 0.25F);
        return out;
    }

    void check_slice(const std::vector<uint16_t> &storage, std::int64_t batch_cap, std::int64_t seq_cap,
                     std::int64_t projection, std::int32_t layer, std::int64_t start, std::int64_t seq,
                     const std::vector<uint16_t> &expected)
    {
        for (std::int64_t b = 0; b < batch_cap; ++b)
            for (std::int64_t t = 0; t < seq; ++t)
                for (std::int64_t c = 0; c < projection; ++c)
                {
                    const std::int64_t dst = ((layer * batch_cap + b) * seq_cap + start + t) * projection + c;
                    require(storage[dst] == expected[(b * seq + t) * projection + c], "KV cache data mismatch");
                }
    }

    void reference_scenario()
    {
        constexpr std::int32_t layers = 2, heads = 2, head_dim = 4;
        constexpr std::int64_t batch_cap = 2, seq_cap = 5, projection = heads * head_dim;
        KvCache cache{layers, batch_cap, seq_cap, heads, head_dim, DType::BFloat16, qwen3::Device::cuda(0)};
        const Shape prefill{batch_cap, 2, projection};
        const auto pk = make_values(static_cast<std::size_t>(prefill.numel()), 1.0F);
        const auto pv = make_values(static_cast<std::size_t>(prefill.numel()), 21.0F);
        Tensor pkt = test::to_gpu(pk, prefill, DType::BFloat16), pvt = test::to_gpu(pv, prefill, DType::BFloat16);
        cache.append(0, 0, pkt, pvt);
        cache.append(1, 0, pkt, pvt);
        require(cache.cached_length(0) == 2 && cache.cached_length(1) == 2, "prefill length");
        const Shape decode{batch_cap, 1, projection};
        const auto dk = make_values(static_cast<std::size_t>(decode.numel()), 41.0F);
        const auto dv = make_values(static_cast<std::size_t>(decode.numel()), 61.0F);
        Tensor dkt = test::to_gpu(dk, decode, DType::BFloat16), dvt = test::to_gpu(dv, decode, DType::BFloat16);
        cache.append(0, 2, dkt, dvt);
        cache.append(1, 2, dkt, dvt);
        require(cache.cached_length(0) == 3 && cache.cached_length(1) == 3, "decode length");
        const auto view = cache.key_view(1);
        require(view.shape() == (Shape{batch_cap, 3, heads, head_dim}), "view shape");
        require(view.strides() == (std::vector<std::int64_t>{seq_cap * projection, projection, head_dim, 1}),
                "view strides");
        const auto keys = test::to_host<uint16_t>(cache.key_storage());
        const auto vals = test::to_host<uint16_t>(cache.value_storage());
        check_slice(keys, batch_cap, seq_cap, projection, 1, 0, 2, pk);
        check_slice(vals, batch_cap, seq_cap, projection, 1, 0, 2, pv);
        check_slice(keys, batch_cap, seq_cap, projection, 1, 2, 1, dk);
        check_slice(vals, batch_cap, seq_cap, projection, 1, 2, 1, dv);
        check_slice(keys, batch_cap, seq_cap, projection, 0, 2, 1, dk);
        require_throws<std::logic_error>([&] { cache.append(0, 1, dkt, dvt); }, "non-append write accepted");
        // the other rules of append
        require_throws<std::out_of_range>([&] { cache.append(2, 3, dkt, dvt); }, "layer index out of range");
        Tensor one = test::to_gpu(make_values(projection, 1.0F), Shape{1, 1, projection}, DType::BFloat16);
        require_throws<std::invalid_argument>([&] { cache.append(0, 3, one, one); }, "batch change accepted");
        Tensor big = test::to_gpu(make_values(batch_cap * 3 * projection, 1.0F), Shape{batch_cap, 3, projection},
                                  DType::BFloat16);
        require_throws<std::out_of_range>([&] { cache.append(0, 3, big, big); }, "capacity overrun accepted");
        require_throws<std::invalid_argument>([&] { cache.append(0, 3, dkt, pvt); }, "key/value shape mismatch");
        cache.reset();
        require(cache.cached_length(0) == 0 && cache.cached_length(1) == 0 && cache.active_batch_size() == 0,
                "reset");
        cache.append(0, 0, one, one);
        require(cache.active_batch_size() == 1, "batch size after reset");
    }

    void fp32_cache()
    {
        KvCache cache{1, 1, 4, 1, 6, DType::Float32, qwen3::Device::cuda(0)};
        std::vector<float> k(18), v(18);
        for (std::size_t i = 0; i < k.size(); ++i)
        {
            k[i] = 0.1F * static_cast<float>(i);
            v[i] = -1.0F - static_cast<float>(i);
        }
        cache.append(0, 0, test::to_gpu(k, Shape{1, 3, 6}, DType::Float32),
                     test::to_gpu(v, Shape{1, 3, 6}, DType::Float32));
        const auto keys = test::to_host<float>(cache.key_storage());
        const auto vals = test::to_host<float>(cache.value_storage());
        require(std::memcmp(keys.data(), k.data(), k.size() * 4) == 0, "fp32 keys");
        require(std::memcmp(vals.data(), v.data(), v.size() * 4) == 0, "fp32 values");
    }

    void fused_append()
    {
        constexpr std::int64_t B = 2, S = 9, D = 128, cap = 24;
        constexpr std::int32_t Hq = 16, Hkv = 8;
        const float eps = 1e-6F;
        Tensor rope = qwen3::ops::build_rope_cache(64, static_cast<std::int32_t>(D), 1.0e6F, qwen3::Device::cuda(0));
        const auto q0 = test::values(B * S * Hq * D, 50), k0 = test::values(B * S * Hkv * D, 51);
        const auto v0 = test::values(B * S * Hkv * D, 52);
        Tensor qw = test::to_gpu(test::values(D, 53, 0.1F, 1.0F), Shape{D}, DType::BFloat16);
        Tensor kw = test::to_gpu(test::values(D, 54, 0.1F, 1.0F), Shape{D}, DType::BFloat16);
        KvCache fused{2, B, cap, Hkv, static_cast<std::int32_t>(D), DType::BFloat16, qwen3::Device::cuda(0)};
        KvCache plain{2, B, cap, Hkv, static_cast<std::int32_t>(D), DType::BFloat16, qwen3::Device::cuda(0)};
        // two steps (prefill at 0, then a second chunk at S) into layer 1
        for (std::int64_t step = 0; step < 2; ++step)
        {
            const std::int64_t start = step * S;
            Tensor q1 = test::to_gpu(q0, Shape{B, S, Hq * D}, DType::BFloat16);
            Tensor k1 = test::to_gpu(k0, Shape{B, S, Hkv * D}, DType::BFloat16);
            Tensor v1 = test::to_gpu(v0, Shape{B, S, Hkv * D}, DType::BFloat16);
            qwen3::ops::qk_norm_rope_kv_append(q1, k1, v1, qw, kw, eps, rope, Hq, Hkv, start, fused, 1);
            require(test::to_host<uint16_t>(k1) == k0, "fused op modified the key input");
            Tensor q2 = qwen3::ops::rms_norm(test::to_gpu(q0, Shape{B, S, Hq * D}, DType::BFloat16), qw, eps);
            Tensor k2 = qwen3::ops::rms_norm(test::to_gpu(k0, Shape{B, S, Hkv * D}, DType::BFloat16), kw, eps);
            qwen3::ops::apply_rope_inplace(q2, k2, rope, Hq, Hkv, start);
            plain.append(1, start, k2, v1);
            require(test::to_host<uint16_t>(q1) == test::to_host<uint16_t>(q2), "fused query equals the sequence");
        }
        require(fused.cached_length(1) == 2 * S && fused.cached_length(0) == 0, "fused append lengths");
        const auto fk = test::to_host<uint16_t>(fused.key_storage()), pk = test::to_host<uint16_t>(plain.key_storage());
        const auto fv = test::to_host<uint16_t>(fused.value_storage()),
                   pv = test::to_host<uint16_t>(plain.value_storage());
        const std::size_t layer = static_cast<std::size_t>(B * cap * Hkv * D);
        const std::size_t used = static_cast<std::size_t>(2 * S * Hkv * D);
        for (std::int64_t b = 0; b < B; ++b)
        {
            const std::size_t at = layer + static_cast<std::size_t>(b * cap * Hkv * D);
            require(std::equal(fk.begin() + at, fk.begin() + at + used, pk.begin() + at), "fused keys");
            require(std::equal(fv.begin() + at, fv.begin() + at + used, pv.begin() + at), "fused values");
        }
        Tensor q3 = test::to_gpu(q0, Shape{B, S, Hq * D}, DType::BFloat16);
        Tensor k3 = test::to_gpu(k0, Shape{B, S, Hkv * D}, DType::BFloat16);
        require_throws<std::logic_error>(
            [&] { qwen3::ops::qk_norm_rope_kv_append(q3, k3, k3, qw, kw, eps, rope, Hq, Hkv, 0, fused, 1); },
            "fused append at a stale position accepted");
        require_throws<std::out_of_range>(
            [&] { qwen3::ops::qk_norm_rope_kv_append(q3, k3, k3, qw, kw, eps, rope, Hq, Hkv, 60, fused, 1); },
            "RoPE range past the table accepted");
    }

    // gqa_attention_cuda_test.cpp:259-357: one history token and two current
    // tokens through KvCache, then attention over the cache views.
    std::vector<uint16_t> att_values(std::size_t count, float scale, int offset)
    {
        std::vector<uint16_t> out(count);
        for (std::size_t i = 0; i < count; ++i)
            out[i] = q3o_bf16_from_f32(static_cast<float>(static_cast<int>((i + offset) % 11) - 5) * scale);
        return out;
    }

    void attention_scenario()
    {
        constexpr std::int64_t B = 2, S = 2, start = 1, cap = 4;
        constexpr std::int32_t Hq = 4, Hkv = 2, D = 4;
        KvCache cache{1, B, cap, Hkv, D, DType::BFloat16, qwen3::Device::cuda(0)};
        const auto hk = att_values(B * Hkv * D, 0.125F, 1), hv = att_values(B * Hkv * D, 0.25F, 2);
        const auto ck = att_values(B * S * Hkv * D, 0.125F, 3), cv = att_values(B * S * Hkv * D, 0.25F, 4);
        const auto q = att_values(B * S * Hq * D, 0.125F, 5);
        cache.append(0, 0, test::to_gpu(hk, Shape{B, 1, Hkv * D}, DType::BFloat16),
                     test::to_gpu(hv, Shape{B, 1, Hkv * D}, DType::BFloat16));
        cache.append(0, start, test::to_gpu(ck, Shape{B, S, Hkv * D}, DType::BFloat16),
                     test::to_gpu(cv, Shape{B, S, Hkv * D}, DType::BFloat16));
        Tensor qt = test::to_gpu(q, Shape{B, S, Hq * D}, DType::BFloat16);
        const auto kview = cache.key_view(0), vview = cache.value_view(0);
        Tensor out = qwen3::ops::grouped_query_attention(qt, kview, vview, Hq, start);
        require(out.shape() == qt.shape(), "attention output shape");
        const auto got = test::to_host<uint16_t>(out);
        // the oracle over the cache storage, with the view's strides
        const auto ks = test::to_host<uint16_t>(cache.key_storage()), vs = test::to_host<uint16_t>(cache.value_storage());
        const std::int64_t st[4] = {cap * Hkv * D, Hkv * D, D, 1};
        std::vector<uint16_t> prim(got.size()), lo(got.size()), hi(got.size());
        require(q3o_gqa_attention(q.data(), ks.data(), vs.data(), B, S, Hq, Hkv, D, start + S, start, st, st, nullptr, 0,
                                  prim.data(), lo.data(), hi.data(), 2) == 0,
                "oracle attention");
        for (std::size_t i = 0; i < got.size(); ++i)
            require(std::fabs(q3o_f32_from_bf16(got[i]) - q3o_f32_from_bf16(prim[i])) <= 0.04F,
                    "attention within the reference test's tolerance");
        test::require_band(got, prim, lo, hi, "attention");
        // the reference's checks
        require_throws<std::invalid_argument>([&] { (void)qwen3::ops::grouped_query_attention(qt, kview, vview, Hq, 0); },
                                              "cache length not start + S accepted");
        require_throws<std::invalid_argument>([&] { (void)qwen3::ops::grouped_query_attention(qt, kview, vview, 3, start); },
                                              "query heads not divisible by KV heads accepted");
    }

    void body()
    {
        test::require_gpu();
        const int before = test::current_device();
        reference_scenario();
        fp32_cache();
        fused_append();
        attention_scenario();
        require(test::current_device() == before, "a KV cache call changed the current device");
    }
} // namespace

int main() { return test::run("GPU KV cache test", body); }
