// The per-layer non-GEMM chain on the GPU against the oracle's composition of
// the reference's ops, output by output.  Both C++ chains run:
//   qwen3_non_gemm_layer          the fused ops (four launches);
//   qwen3_non_gemm_layer_unfused  the drop-in ops in the reference's order
//                                 (decoder_layer.cpp:63-98,
//                                 self_attention.cpp:147-152, mlp.cpp:111).
// The oracle side composes, in the layer's order,
//   q3o_qk_norm_rope (Q with q_norm, K with k_norm)
//   -> q3o_add_rms_norm (attention residual, post-attention norm)
//   -> q3o_silu_mul
//   -> q3o_add_rms_norm (MLP residual, the next layer's input norm),
// each on the oracle's own previous results.  Two workloads:
//   config 2 in full (Qwen3-0.6B, T = 512 at positions 0..511), its residual
//   stream produced by the embedding gather of model.cpp:118 (checked
//   bit-exact against q3o_embedding, one id outside the table);
//   a slice of config 4 (Qwen3-8B shapes, 2 sequences x 128 tokens at
//   positions 64..191 of the 2048-position table).
// Residual streams must be bit-exact; every other output inside the oracle's
// band widened by one bf16 ulp; and the two chains' outputs equal bit for
// bit.  Each comparison prints a PARITY line (JSON:
// case, elements, failures, ulp histogram) that the pytest runner adds to the
// parity report.
#include "gpu_util.hpp"
#include "qwen3/model/non_gemm_layer.h"
#include "qwen3/ops/embedding.h"
#include "qwen3/ops/rope.h"

#include <cstdio>
#include <thread>

using qwen3::DType;
using qwen3::Shape;
using qwen3::Tensor;
using test::require;

namespace
{
    constexpr float kEps = 1e-6f;
    constexpr std::int32_t kD = 128;

    int oracle_threads()
    {
        const unsigned n = std::thread::hardware_concurrency();
        return n == 0 ? 1 : static_cast<int>(n < 16 ? n : 16);
    }

    void report(const std::string &name, const std::vector<uint16_t> &got, const std::vector<uint16_t> &primary,
                const std::vector<uint16_t> *lo, const std::vector<uint16_t> *hi)
    {
        require(got.size() == primary.size(), name + ": size mismatch");
        int64_t st[8];
        q3o_compare_band(got.data(), primary.data(), lo ? lo->data() : nullptr, hi ? hi->data() : nullptr,
                         static_cast<int64_t>(got.size()), st);
        std::printf("PARITY {\"case\": \"%s\", \"n\": %lld, \"fail\": %lld, \"ambiguous\": %lld, "
                    "\"ulp_hist\": [%lld, %lld, %lld, %lld], \"exact\": %s}\n",
                    name.c_str(), static_cast<long long>(st[0]), static_cast<long long>(st[1]),
                    static_cast<long long>(st[3]), static_cast<long long>(st[4]), static_cast<long long>(st[5]),
                    static_cast<long long>(st[6]), static_cast<long long>(st[7]), lo ? "false" : "true");
        std::fflush(stdout);
        if (lo == nullptr)
        {
            require(got == primary, name + ": not bit-exact");
            return;
        }
        test::require_band(got, primary, *lo, *hi, name);
    }

    struct Workload
    {
        const char *name;
        std::int64_t B, S, H, I, start, P;
        std::int32_t Hq, Hkv;
        bool embedding;
        uint64_t seed;
    };

    Tensor gpu(const std::vector<uint16_t> &v, const Shape &shape) { return test::to_gpu(v, shape, DType::BFloat16); }

    void run(const Workload &w)
    {
        const std::int64_t T = w.B * w.S;
        const int nt = oracle_threads();
        const auto values = [&](std::int64_t n, uint64_t k, float scale = 1.0f, float offset = 0.0f) {
            return test::values(static_cast<std::size_t>(n), w.seed * 100 + k, scale, offset);
        };
        const Shape hs{w.B, w.S, w.H}, qs{w.B, w.S, w.Hq * kD}, ks{w.B, w.S, w.Hkv * kD}, is{w.B, w.S, w.I};

        // residual stream: the embedding gather (config 2) or seeded values
        std::vector<uint16_t> h0;
        if (w.embedding)
        {
            constexpr std::int64_t V = 151936;
            const auto table = values(V * w.H, 1, 0.02f);
            std::vector<int32_t> ids(static_cast<std::size_t>(T));
            uint64_t s = w.seed * 0x9E3779B97F4A7C15ull + 7;
            for (auto &id : ids)
            {
                s ^= s << 13;
                s ^= s >> 7;
                s ^= s << 17;
                id = static_cast<int32_t>(s % V);
            }
            ids[3] = static_cast<int32_t>(V); // outside the table: a zero row (embedding.cu:38-45)
            Tensor gt = gpu(table, Shape{V, w.H});
            Tensor gid = test::to_gpu(ids, Shape{w.B, w.S}, DType::Int32);
            h0 = test::to_host<uint16_t>(qwen3::ops::embedding_lookup(gid, gt));
            std::vector<uint16_t> want(static_cast<std::size_t>(T * w.H));
            q3o_embedding(ids.data(), T, table.data(), V, w.H, want.data(), nt);
            report(std::string(w.name) + " embedding", h0, want, nullptr, nullptr);
        }
        else
        {
            h0 = values(T * w.H, 1);
        }
        const auto q0 = values(T * w.Hq * kD, 2), k0 = values(T * w.Hkv * kD, 3);
        const auto attn = values(T * w.H, 4), gate = values(T * w.I, 5), up = values(T * w.I, 6);
        const auto mlp = values(T * w.H, 7);
        const auto qn = values(kD, 8, 0.1f, 1.0f), kn = values(kD, 9, 0.1f, 1.0f);
        const auto post = values(w.H, 10, 0.1f, 1.0f), next = values(w.H, 11, 0.1f, 1.0f);

        // oracle composition, in the layer's order
        std::vector<float> table(static_cast<std::size_t>(w.P * kD));
        require(q3o_build_rope_cache(w.P, kD, 1.0e6f, table.data()) == 0, "oracle RoPE table");
        std::vector<uint16_t> oq = q0, ok = k0, qlo(q0.size()), qhi(q0.size()), klo(k0.size()), khi(k0.size());
        require(q3o_qk_norm_rope(oq.data(), qn.data(), w.B, w.S, w.Hq, kD, kEps, table.data(), w.P, w.start, nullptr,
                                 qlo.data(), qhi.data(), nt) == 0, "oracle Q norm + RoPE");
        require(q3o_qk_norm_rope(ok.data(), kn.data(), w.B, w.S, w.Hkv, kD, kEps, table.data(), w.P, w.start, nullptr,
                                 klo.data(), khi.data(), nt) == 0, "oracle K norm + RoPE");
        const std::size_t nh = h0.size(), ni = gate.size();
        std::vector<uint16_t> oh = h0, y1(nh), y1lo(nh), y1hi(nh), y2(nh), y2lo(nh), y2hi(nh);
        q3o_add_rms_norm(oh.data(), attn.data(), post.data(), T, w.H, kEps, y1.data(), y1lo.data(), y1hi.data(), nt);
        std::vector<uint16_t> act(ni), alo(ni), ahi(ni);
        q3o_silu_mul(gate.data(), up.data(), static_cast<int64_t>(ni), act.data(), alo.data(), ahi.data(), nt);
        q3o_add_rms_norm(oh.data(), mlp.data(), next.data(), T, w.H, kEps, y2.data(), y2lo.data(), y2hi.data(), nt);

        Tensor cache = qwen3::ops::build_rope_cache(w.P, kD, 1.0e6f, qwen3::Device::cuda(0));
        Tensor gqn = gpu(qn, Shape{kD}), gkn = gpu(kn, Shape{kD}), gpost = gpu(post, Shape{w.H}), gnext = gpu(next, Shape{w.H});
        const qwen3::NonGemmLayerWeights weights{gqn, gkn, gpost, gnext};
        Tensor gattn = gpu(attn, hs), ggate = gpu(gate, is), gup = gpu(up, is), gmlp = gpu(mlp, hs);
        std::vector<std::vector<uint16_t>> first;
        for (const bool fused : {true, false})
        {
            const std::string tag = std::string(w.name) + (fused ? " fused" : " unfused");
            Tensor h = gpu(h0, hs), q = gpu(q0, qs), k = gpu(k0, ks);
            const qwen3::NonGemmLayerTensors tensors{h, q, k, gattn, ggate, gup, gmlp};
            const auto out = fused ? qwen3::qwen3_non_gemm_layer(tensors, weights, cache, w.Hq, w.Hkv, w.start, kEps)
                                   : qwen3::qwen3_non_gemm_layer_unfused(tensors, weights, cache, w.Hq, w.Hkv,
                                                                         w.start, kEps);
            const std::vector<std::vector<uint16_t>> got{
                test::to_host<uint16_t>(h), test::to_host<uint16_t>(q), test::to_host<uint16_t>(k),
                test::to_host<uint16_t>(out.mlp_input), test::to_host<uint16_t>(out.activation),
                test::to_host<uint16_t>(out.next_input)};
            report(tag + " residual", got[0], oh, nullptr, nullptr);
            report(tag + " query", got[1], oq, &qlo, &qhi);
            report(tag + " key", got[2], ok, &klo, &khi);
            report(tag + " mlp_input", got[3], y1, &y1lo, &y1hi);
            report(tag + " activation", got[4], act, &alo, &ahi);
            report(tag + " next_input", got[5], y2, &y2lo, &y2hi);
            if (fused)
                first = got;
            else
                require(got == first, std::string(w.name) + ": the unfused chain differs from the fused one");
        }
    }

    void body()
    {
        test::require_gpu();
        // config 2 in full: Qwen3-0.6B, 1 x 512 tokens at positions 0..511
        run({"config 2", 1, 512, 1024, 3072, 0, 512, 16, 8, true, 1});
        // config 4 slice: Qwen3-8B shapes, 2 x 128 tokens at positions 64..191
        run({"config 4 slice", 2, 128, 4096, 12288, 64, 2048, 32, 8, false, 3});
    }
} // namespace

int main() { return test::run("GPU layer chain against the oracle", body); }
