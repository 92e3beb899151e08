// qwen3::ops on the GPU with the reference tests' known-answer inputs
// (tests/unit/{rms_norm,rope,elementwise,embedding}_cuda_test.cpp): shapes,
// dtypes, in-place pointer identity, the current device left unchanged, the
// reference tests' tolerances, and the 1-ulp band of the oracle.
#include "gpu_util.hpp"
#include "qwen3/ops/elementwise.h"
#include "qwen3/ops/embedding.h"
#include "qwen3/ops/rms_norm.h"
#include "qwen3/ops/rope.h"

#include <cmath>

using qwen3::DType;
using qwen3::Shape;
using qwen3::Tensor;
using test::bf16;
using test::f32;
using test::require;
using test::require_throws;

namespace
{
    void rms_norm_case(const Shape &shape)
    {
        const std::int64_t hidden = shape[shape.rank() - 1];
        const std::int64_t n = shape.numel();
        std::vector<uint16_t> x(static_cast<std::size_t>(n)), w(static_cast<std::size_t>(hidden));
        for (std::int64_t i = 0; i < n; ++i)
            x[i] = bf16(static_cast<float>(static_cast<int>(i % 31) - 15) * 0.125f);
        for (std::int64_t j = 0; j < hidden; ++j)
            w[j] = bf16(0.5f + static_cast<float>(j % 17) * 0.03125f);
        Tensor gx = test::to_gpu(x, shape, DType::BFloat16);
        Tensor gw = test::to_gpu(w, Shape{hidden}, DType::BFloat16);
        Tensor gy = qwen3::ops::rms_norm(gx, gw, 1e-6f);
        require(gy.shape() == shape && gy.dtype() == DType::BFloat16 && gy.device() == gx.device(), "rms_norm output");
        const auto y = test::to_host<uint16_t>(gy);
        for (std::int64_t r = 0; r < n / hidden; ++r)
        {
            double ss = 0;
            for (std::int64_t c = 0; c < hidden; ++c)
                ss += static_cast<double>(f32(x[r * hidden + c])) * f32(x[r * hidden + c]);
            const double inv = 1.0 / std::sqrt(ss / hidden + 1e-6);
            for (std::int64_t c = 0; c < hidden; ++c)
            {
                const double e = f32(x[r * hidden + c]) * inv * f32(w[c]);
                require(std::fabs(f32(y[r * hidden + c]) - e) <= 0.02 + 0.01 * std::fabs(e), "rms_norm tolerance");
            }
        }
        std::vector<uint16_t> prim(y.size()), lo(y.size()), hi(y.size());
        q3o_rms_norm(x.data(), w.data(), n / hidden, hidden, 1e-6f, prim.data(), lo.data(), hi.data(), 1);
        test::require_band(y, prim, lo, hi, "rms_norm " + shape.to_string());
        Tensor into = Tensor::empty(shape, DType::BFloat16, gx.device());
        qwen3::ops::rms_norm(gx, gw, 1e-6f, into);
        require(test::to_host<uint16_t>(into) == y, "rms_norm into-variant equals the returning form");
        require_throws<std::invalid_argument>([&] { qwen3::ops::rms_norm(gx, gw, 1e-6f, gx); }, "aliasing output accepted");
        require_throws<std::invalid_argument>([&] { (void)qwen3::ops::rms_norm(gx, gw, 0.0f); }, "zero epsilon accepted");
    }

    void rope_case()
    {
        const std::int64_t B = 1, S = 3, D = 8, P = 16, start = 5;
        const std::int32_t Hq = 2, Hkv = 1;
        auto make = [](std::size_t n, int off) {
            std::vector<uint16_t> v(n);
            for (std::size_t i = 0; i < n; ++i)
                v[i] = bf16(static_cast<float>(static_cast<int>((i + off) % 17) - 8) * 0.25f);
            return v;
        };
        const auto qv = make(B * S * Hq * D, 0), kv = make(B * S * Hkv * D, 5);
        Tensor q = test::to_gpu(qv, Shape{B, S, Hq * D}, DType::BFloat16);
        Tensor k = test::to_gpu(kv, Shape{B, S, Hkv * D}, DType::BFloat16);
        Tensor cache = qwen3::ops::build_rope_cache(P, static_cast<std::int32_t>(D), 1.0e6f, qwen3::Device::cuda(0));
        require(cache.shape() == (Shape{P, D / 2, 2}) && cache.device().is_cuda(), "rope cache on the GPU");
        void *qp = q.data(), *kp = k.data();
        qwen3::ops::apply_rope_inplace(q, k, cache, Hq, Hkv, start);
        require(q.data() == qp && k.data() == kp, "rope is in place");
        std::vector<float> table(P * D);
        q3o_build_rope_cache(P, static_cast<std::int32_t>(D), 1.0e6f, table.data());
        auto check = [&](const Tensor &t, const std::vector<uint16_t> &v, int heads) {
            const auto got = test::to_host<uint16_t>(t);
            std::vector<uint16_t> prim = v, lo(v.size()), hi(v.size());
            require(q3o_rope(prim.data(), B, S, heads, static_cast<std::int32_t>(D), table.data(), P, start, nullptr,
                             lo.data(), hi.data(), 1) == 0,
                    "oracle rope");
            for (std::int64_t s = 0; s < S; ++s)
                for (int h = 0; h < heads; ++h)
                    for (std::int64_t p = 0; p < D / 2; ++p)
                    {
                        const double ang = static_cast<double>(start + s) * std::pow(1.0e6, -(2.0 * p) / D);
                        const std::size_t o = static_cast<std::size_t>((s * heads + h) * D + p);
                        const double x1 = f32(v[o]), x2 = f32(v[o + D / 2]);
                        require(std::fabs(f32(got[o]) - (x1 * std::cos(ang) - x2 * std::sin(ang))) <= 0.03,
                                "rope x1 tolerance");
                        require(std::fabs(f32(got[o + D / 2]) - (x2 * std::cos(ang) + x1 * std::sin(ang))) <= 0.03,
                                "rope x2 tolerance");
                    }
            test::require_band(got, prim, lo, hi, "rope");
        };
        check(q, qv, Hq);
        check(k, kv, Hkv);
        require_throws<std::out_of_range>([&] { qwen3::ops::apply_rope_inplace(q, k, cache, Hq, Hkv, P - 1); },
                                          "rope position range past the cache accepted");
        require_throws<std::invalid_argument>([&] { qwen3::ops::apply_rope_inplace(q, k, cache, Hq, Hkv, -1); },
                                              "negative start accepted");
        require_throws<std::invalid_argument>([&] { qwen3::ops::apply_rope_inplace(q, k, cache, 3, Hkv, 0); },
                                              "head count mismatch accepted");
        // positions overload: positions start + s give the same result as the scalar form
        Tensor q1 = test::to_gpu(qv, Shape{B, S, Hq * D}, DType::BFloat16);
        Tensor k1 = test::to_gpu(kv, Shape{B, S, Hkv * D}, DType::BFloat16);
        Tensor pos = test::to_gpu(std::vector<int32_t>{5, 6, 7}, Shape{B, S}, DType::Int32);
        qwen3::ops::apply_rope_inplace(q1, k1, cache, Hq, Hkv, pos);
        Tensor q2 = test::to_gpu(qv, Shape{B, S, Hq * D}, DType::BFloat16);
        Tensor k2 = test::to_gpu(kv, Shape{B, S, Hkv * D}, DType::BFloat16);
        qwen3::ops::apply_rope_inplace(q2, k2, cache, Hq, Hkv, start);
        require(test::to_host<uint16_t>(q1) == test::to_host<uint16_t>(q2) &&
                    test::to_host<uint16_t>(k1) == test::to_host<uint16_t>(k2),
                "positions overload equals the scalar form");
    }

    void elementwise_case()
    {
        const Shape shape{2, 3, 257};
        const std::size_t n = static_cast<std::size_t>(shape.numel());
        std::vector<uint16_t> r(n), d(n), g(n), u(n);
        for (std::size_t i = 0; i < n; ++i)
        {
            r[i] = bf16(static_cast<float>(static_cast<int>(i % 41) - 20) * 0.0625f);
            d[i] = bf16(static_cast<float>(static_cast<int>(i % 17) - 8) * 0.03125f);
            g[i] = bf16(static_cast<float>(static_cast<int>(i % 37) - 18) * 0.25f);
            u[i] = bf16(static_cast<float>(static_cast<int>(i % 23) - 11) * 0.125f);
        }
        Tensor gr = test::to_gpu(r, shape, DType::BFloat16), gd = test::to_gpu(d, shape, DType::BFloat16);
        void *rp = gr.data();
        qwen3::ops::add_inplace(gr, gd);
        require(gr.data() == rp, "add_inplace is in place");
        const auto added = test::to_host<uint16_t>(gr);
        std::vector<uint16_t> ref = r;
        q3o_add_inplace(ref.data(), d.data(), static_cast<int64_t>(n), 1);
        require(added == ref, "add_inplace is bit-exact");
        for (std::size_t i = 0; i < n; ++i)
            require(std::fabs(f32(added[i]) - (f32(r[i]) + f32(d[i]))) < 0.001, "add_inplace tolerance");
        Tensor gg = test::to_gpu(g, shape, DType::BFloat16), gu = test::to_gpu(u, shape, DType::BFloat16);
        Tensor out = qwen3::ops::silu_multiply(gg, gu);
        require(out.shape() == shape && out.dtype() == DType::BFloat16, "silu_multiply output");
        const auto o = test::to_host<uint16_t>(out);
        for (std::size_t i = 0; i < n; ++i)
        {
            const double x = f32(g[i]), e = x / (1.0 + std::exp(-x)) * f32(u[i]);
            require(std::fabs(f32(o[i]) - e) <= 0.02 + 0.01 * std::fabs(e), "silu_multiply tolerance");
        }
        std::vector<uint16_t> prim(n), lo(n), hi(n);
        q3o_silu_mul(g.data(), u.data(), static_cast<int64_t>(n), prim.data(), lo.data(), hi.data(), 1);
        test::require_band(o, prim, lo, hi, "silu_multiply");
        qwen3::ops::silu_multiply(gg, gu, gg);
        require(test::to_host<uint16_t>(gg) == o, "silu_multiply into its own gate input");
        Tensor bad = Tensor::empty(Shape{2, 3, 256}, DType::BFloat16, qwen3::Device::cuda(0));
        require_throws<std::invalid_argument>([&] { qwen3::ops::add_inplace(bad, gd); }, "shape mismatch accepted");
    }

    void embedding_case()
    {
        const std::int64_t V = 5, H = 4;
        std::vector<uint16_t> table(V * H);
        for (std::int64_t t = 0; t < V; ++t)
            for (std::int64_t h = 0; h < H; ++h)
                table[t * H + h] = bf16(static_cast<float>(t * 10 + h));
        const std::vector<int32_t> ids{2, 0, 4, 1, 2, 3};
        Tensor gt = test::to_gpu(table, Shape{V, H}, DType::BFloat16);
        Tensor gi = test::to_gpu(ids, Shape{2, 3}, DType::Int32);
        Tensor out = qwen3::ops::embedding_lookup(gi, gt);
        require(out.shape() == (Shape{2, 3, H}) && out.dtype() == DType::BFloat16 && out.device() == qwen3::Device::cuda(0),
                "embedding output");
        const auto o = test::to_host<uint16_t>(out);
        for (std::size_t t = 0; t < ids.size(); ++t)
            for (std::int64_t h = 0; h < H; ++h)
                require(f32(o[t * H + h]) == static_cast<float>(ids[t] * 10 + h), "embedding value");
        const std::vector<int32_t> bad_ids{-1, 5, 3};
        Tensor gb = test::to_gpu(bad_ids, Shape{3}, DType::Int32);
        const auto ob = test::to_host<uint16_t>(qwen3::ops::embedding_lookup(gb, gt));
        for (std::int64_t h = 0; h < H; ++h)
            require(ob[h] == 0 && ob[H + h] == 0 && f32(ob[2 * H + h]) == 30.0f + h, "out-of-range ids give zero rows");
    }

    void body()
    {
        test::require_gpu();
        const int before = test::current_device();
        rms_norm_case(Shape{2, 3, 1024});
        rms_norm_case(Shape{2, 3, 4, 128});
        rms_norm_case(Shape{3, 5120});
        rope_case();
        elementwise_case();
        embedding_case();
        require(test::current_device() == before, "an op changed the current device");
    }
} // namespace

int main() { return test::run("GPU ops test", body); }
