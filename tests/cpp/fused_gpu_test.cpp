// Fused ops and the non-GEMM layer chain on the GPU: each fused result is
// bit-identical to the reference-order composition of the unfused ops, and
// within the oracle's 1-ulp band.
#include "gpu_util.hpp"
#include "qwen3/model/non_gemm_layer.h"
#include "qwen3/ops/elementwise.h"
#include "qwen3/ops/embedding.h"
#include "qwen3/ops/fused.h"
#include "qwen3/ops/rms_norm.h"
#include "qwen3/ops/rope.h"

#include <algorithm>

using qwen3::DType;
using qwen3::Shape;
using qwen3::Tensor;
using test::require;
using test::require_throws;

namespace
{
    constexpr std::int64_t B = 2, S = 40, H = 1024, I = 3072, D = 128;
    constexpr std::int32_t Hq = 16, Hkv = 8;
    constexpr float kEps = 1e-6f;

    Tensor gpu_values(const Shape &shape, uint64_t seed, float scale = 1.0f, float offset = 0.0f)
    {
        return test::to_gpu(test::values(static_cast<std::size_t>(shape.numel()), seed, scale, offset), shape,
                            DType::BFloat16);
    }

    void add_rms_norm_case()
    {
        Tensor h1 = gpu_values(Shape{B, S, H}, 1), h2 = gpu_values(Shape{B, S, H}, 1);
        Tensor d = gpu_values(Shape{B, S, H}, 2), w = gpu_values(Shape{H}, 3, 0.1f, 1.0f);
        const auto h0 = test::to_host<uint16_t>(h1);
        void *hp = h1.data();
        Tensor y1 = qwen3::ops::add_rms_norm(h1, d, w, kEps);
        require(h1.data() == hp, "add_rms_norm updates the residual in place");
        qwen3::ops::add_inplace(h2, d);
        Tensor y2 = qwen3::ops::rms_norm(h2, w, kEps);
        require(test::to_host<uint16_t>(h1) == test::to_host<uint16_t>(h2), "residual equals add_inplace");
        const auto y = test::to_host<uint16_t>(y1);
        require(y == test::to_host<uint16_t>(y2), "add_rms_norm equals add_inplace + rms_norm");
        std::vector<uint16_t> hh = h0, prim(y.size()), lo(y.size()), hi(y.size());
        const auto dv = test::to_host<uint16_t>(d), wv = test::to_host<uint16_t>(w);
        q3o_add_rms_norm(hh.data(), dv.data(), wv.data(), B * S, H, kEps, prim.data(), lo.data(), hi.data(), 4);
        test::require_band(y, prim, lo, hi, "add_rms_norm");
        Tensor into = Tensor::empty(Shape{B, S, H}, DType::BFloat16, qwen3::Device::cuda(0));
        require_throws<std::invalid_argument>([&] { qwen3::ops::add_rms_norm(h1, d, w, kEps, h1); }, "output aliasing residual");
        require_throws<std::invalid_argument>([&] { qwen3::ops::add_rms_norm(h1, w, w, kEps, into); }, "delta shape mismatch");
    }

    void qk_norm_rope_case()
    {
        Tensor cache = qwen3::ops::build_rope_cache(64, static_cast<std::int32_t>(D), 1.0e6f, qwen3::Device::cuda(0));
        Tensor q1 = gpu_values(Shape{B, S, Hq * D}, 4), k1 = gpu_values(Shape{B, S, Hkv * D}, 5);
        Tensor qw = gpu_values(Shape{D}, 6, 0.1f, 1.0f), kw = gpu_values(Shape{D}, 7, 0.1f, 1.0f);
        const auto q0 = test::to_host<uint16_t>(q1), k0 = test::to_host<uint16_t>(k1);
        void *qp = q1.data();
        qwen3::ops::qk_norm_rope_inplace(q1, k1, qw, kw, kEps, cache, Hq, Hkv, 7);
        require(q1.data() == qp, "qk_norm_rope is in place");
        Tensor q2 = qwen3::ops::rms_norm(test::to_gpu(q0, Shape{B, S, Hq * D}, DType::BFloat16), qw, kEps);
        Tensor k2 = qwen3::ops::rms_norm(test::to_gpu(k0, Shape{B, S, Hkv * D}, DType::BFloat16), kw, kEps);
        qwen3::ops::apply_rope_inplace(q2, k2, cache, Hq, Hkv, 7);
        const auto gq = test::to_host<uint16_t>(q1);
        require(gq == test::to_host<uint16_t>(q2), "fused Q equals rms_norm + apply_rope_inplace");
        require(test::to_host<uint16_t>(k1) == test::to_host<uint16_t>(k2), "fused K equals rms_norm + apply_rope_inplace");
        std::vector<float> table(64 * D);
        q3o_build_rope_cache(64, static_cast<std::int32_t>(D), 1.0e6f, table.data());
        std::vector<uint16_t> prim = q0, lo(q0.size()), hi(q0.size());
        const auto qwv = test::to_host<uint16_t>(qw);
        require(q3o_qk_norm_rope(prim.data(), qwv.data(), B, S, Hq, static_cast<std::int32_t>(D), kEps, table.data(), 64, 7,
                                 nullptr, lo.data(), hi.data(), 4) == 0,
                "oracle qk_norm_rope");
        test::require_band(gq, prim, lo, hi, "qk_norm_rope");
        // positions overload with start + s positions equals the scalar form
        std::vector<int32_t> pos(B * S);
        for (std::int64_t b = 0; b < B; ++b)
            for (std::int64_t s = 0; s < S; ++s)
                pos[b * S + s] = static_cast<int32_t>(7 + s);
        Tensor gp = test::to_gpu(pos, Shape{B, S}, DType::Int32);
        Tensor q3 = test::to_gpu(q0, Shape{B, S, Hq * D}, DType::BFloat16), k3 = test::to_gpu(k0, Shape{B, S, Hkv * D}, DType::BFloat16);
        qwen3::ops::qk_norm_rope_inplace(q3, k3, qw, kw, kEps, cache, Hq, Hkv, gp);
        require(test::to_host<uint16_t>(q3) == gq, "positions overload equals the scalar form");
        require_throws<std::out_of_range>([&] { qwen3::ops::qk_norm_rope_inplace(q3, k3, qw, kw, kEps, cache, Hq, Hkv, 30); },
                                          "position range past the cache accepted");
        require_throws<std::invalid_argument>([&] { qwen3::ops::qk_norm_rope_inplace(q3, k3, kw, cache, kEps, cache, Hq, Hkv, 0); },
                                              "float32 norm weight accepted");
    }

    // Rows [b, S-1, :] of a [B, S, H] host copy, as select_last_token_hidden returns them.
    std::vector<uint16_t> last_rows(const std::vector<uint16_t> &all, std::int64_t b, std::int64_t s, std::int64_t h)
    {
        std::vector<uint16_t> out;
        for (std::int64_t i = 0; i < b; ++i)
            out.insert(out.end(), all.begin() + ((i * s + s - 1) * h), all.begin() + ((i * s + s) * h));
        return out;
    }

    void embedding_rms_norm_case()
    {
        constexpr std::int64_t V = 300;
        Tensor table = gpu_values(Shape{V, H}, 30), w = gpu_values(Shape{H}, 31, 0.1f, 1.0f);
        std::vector<int32_t> ids(B * S);
        for (std::size_t i = 0; i < ids.size(); ++i)
            ids[i] = static_cast<int32_t>((i * 7919) % V);
        ids[3] = -1;
        ids[5] = static_cast<int32_t>(V);
        Tensor gid = test::to_gpu(ids, Shape{B, S}, DType::Int32);
        const auto fused = qwen3::ops::embedding_rms_norm(gid, table, w, kEps);
        require(fused.hidden.shape() == (Shape{B, S, H}) && fused.normalized.shape() == (Shape{B, S, H}),
                "embedding_rms_norm shapes");
        Tensor hidden = qwen3::ops::embedding_lookup(gid, table);
        Tensor normalized = qwen3::ops::rms_norm(hidden, w, kEps);
        require(test::to_host<uint16_t>(fused.hidden) == test::to_host<uint16_t>(hidden), "gather equals embedding_lookup");
        require(test::to_host<uint16_t>(fused.normalized) == test::to_host<uint16_t>(normalized),
                "embedding_rms_norm equals embedding_lookup + rms_norm");
        require_throws<std::invalid_argument>([&] { (void)qwen3::ops::embedding_rms_norm(gid, table, table, kEps); },
                                              "two-dimensional norm weight accepted");
        require_throws<std::invalid_argument>(
            [&] { (void)qwen3::ops::embedding_rms_norm(gid, table, gpu_values(Shape{H + 8}, 32), kEps); },
            "norm weight of the wrong size accepted");
    }

    void last_token_case()
    {
        Tensor h1 = gpu_values(Shape{B, S, H}, 40), h2 = gpu_values(Shape{B, S, H}, 40);
        Tensor d = gpu_values(Shape{B, S, H}, 41), w = gpu_values(Shape{H}, 42, 0.1f, 1.0f);
        const auto h0 = test::to_host<uint16_t>(h1);
        Tensor y = qwen3::ops::rms_norm_last_token(h1, w, kEps);
        require(y.shape() == (Shape{B, H}), "last-token norm shape");
        const auto full = test::to_host<uint16_t>(qwen3::ops::rms_norm(h1, w, kEps));
        require(test::to_host<uint16_t>(y) == last_rows(full, B, S, H),
                "rms_norm_last_token equals the last rows of rms_norm");

        Tensor ya = qwen3::ops::add_rms_norm_last_token(h1, d, w, kEps);
        qwen3::ops::add_inplace(h2, d);
        const auto summed = test::to_host<uint16_t>(h2);
        const auto full_a = test::to_host<uint16_t>(qwen3::ops::rms_norm(h2, w, kEps));
        require(test::to_host<uint16_t>(ya) == last_rows(full_a, B, S, H),
                "add_rms_norm_last_token equals the last rows of add_inplace + rms_norm");
        const auto got = test::to_host<uint16_t>(h1);
        for (std::int64_t b = 0; b < B; ++b)
            for (std::int64_t s = 0; s < S; ++s)
            {
                const auto &want = s == S - 1 ? summed : h0;
                const std::int64_t at = (b * S + s) * H;
                require(std::equal(got.begin() + at, got.begin() + at + H, want.begin() + at),
                        "residual: last rows updated, earlier rows untouched");
            }
        require_throws<std::invalid_argument>([&] { (void)qwen3::ops::rms_norm_last_token(w, w, kEps); },
                                              "rank-1 hidden states accepted");
    }

    void layer_chain_case()
    {
        Tensor cache = qwen3::ops::build_rope_cache(S, static_cast<std::int32_t>(D), 1.0e6f, qwen3::Device::cuda(0));
        Tensor qn = gpu_values(Shape{D}, 10, 0.1f, 1.0f), kn = gpu_values(Shape{D}, 11, 0.1f, 1.0f);
        Tensor post = gpu_values(Shape{H}, 12, 0.1f, 1.0f), next = gpu_values(Shape{H}, 13, 0.1f, 1.0f);
        const qwen3::NonGemmLayerWeights weights{qn, kn, post, next};
        Tensor attn = gpu_values(Shape{B, S, H}, 14), gate = gpu_values(Shape{B, S, I}, 15), up = gpu_values(Shape{B, S, I}, 16);
        Tensor mlp = gpu_values(Shape{B, S, H}, 17);
        Tensor h1 = gpu_values(Shape{B, S, H}, 18), h2 = gpu_values(Shape{B, S, H}, 18);
        Tensor q1 = gpu_values(Shape{B, S, Hq * D}, 19), q2 = gpu_values(Shape{B, S, Hq * D}, 19);
        Tensor k1 = gpu_values(Shape{B, S, Hkv * D}, 20), k2 = gpu_values(Shape{B, S, Hkv * D}, 20);
        const auto fused = qwen3::qwen3_non_gemm_layer({h1, q1, k1, attn, gate, up, mlp}, weights, cache, Hq, Hkv, 0, kEps);
        const auto plain = qwen3::qwen3_non_gemm_layer_unfused({h2, q2, k2, attn, gate, up, mlp}, weights, cache, Hq, Hkv, 0, kEps);
        require(test::to_host<uint16_t>(h1) == test::to_host<uint16_t>(h2), "chain residual stream");
        require(test::to_host<uint16_t>(q1) == test::to_host<uint16_t>(q2), "chain query");
        require(test::to_host<uint16_t>(k1) == test::to_host<uint16_t>(k2), "chain key");
        require(test::to_host<uint16_t>(fused.mlp_input) == test::to_host<uint16_t>(plain.mlp_input), "chain mlp input");
        require(test::to_host<uint16_t>(fused.activation) == test::to_host<uint16_t>(plain.activation), "chain activation");
        require(test::to_host<uint16_t>(fused.next_input) == test::to_host<uint16_t>(plain.next_input), "chain next input");
    }

    void body()
    {
        test::require_gpu();
        const int before = test::current_device();
        add_rms_norm_case();
        qk_norm_rope_case();
        embedding_rms_norm_case();
        last_token_case();
        layer_chain_case();
        require(test::current_device() == before, "a fused op changed the current device");
    }
} // namespace

int main() { return test::run("GPU fused ops test", body); }
