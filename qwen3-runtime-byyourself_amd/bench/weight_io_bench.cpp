// Weight IO throughput: the time to bring every tensor of a safetensors file
// to the GPU, for a synthetic checkpoint shaped like Qwen3-8B decoder layers
// (bf16, 386 MiB of weights per layer).  The file is written first, so its
// pages are in the host page cache: what is measured is the mapping, the
// host-side staging copies and the host-to-device DMA, not the disk.
//
// Each timed load starts from a fresh mapping of the file (a process loads
// its weights once, so first-touch page faults are part of the cost) and
// ends when the last copy has completed on the GPU.
//
// Legs (all in GB/s of tensor bytes):
//   loader          qwen3::SafetensorsLoader::load_many, the product path;
//   loader_second_batch  the same, as the second batch of one loader (file
//                   pages mapped and staging touched by the first);
//   reference       the reference's staging scheme, restated here as the
//                   baseline (src/io/safetensors_loader.cpp:141-248: one
//                   host thread, two 32 MiB pinned buffers, one event each);
//   dma_ceiling     hipMemcpyAsync from one resident pinned buffer, no host
//                   copy: the host-to-device link's rate for this process
//                   (32 MiB pieces; dma_ceiling_8MiB in the loader's chunks);
//   host_copy_tN    the staging copies alone (fresh mapping -> pinned
//                   buffers, N threads, no DMA);
//   setup           milliseconds of the one-off steps inside a load.
// --sweep adds the staged scheme over a grid of copy threads, slots and
// slot sizes.  The loaded bytes are compared with the file once.
//
// Usage: q3k_weight_io_bench [--layers L] [--repeats R] [--dir D] [--sweep]
#include "qwen3/core/tensor.h"
#include "qwen3/hip/hip_check.h"
#include "qwen3/io/copy_crew.h"
#include "qwen3/io/safetensors_file.h"
#include "qwen3/io/safetensors_loader.h"
#include "qwen3/io/safetensors_metadata.h"

#include "../csrc/io/staged_upload.hpp"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <stdexcept>
#include <string>
#include <unistd.h>
#include <vector>

namespace fs = std::filesystem;

namespace
{
    struct Entry
    {
        std::string name;
        std::vector<std::int64_t> shape;
    };

    // Qwen3-8B: hidden 4096, 32 query / 8 KV heads of 128, MLP 12288.
    std::vector<Entry> layer_entries(int layer)
    {
        const std::string p = "model.layers." + std::to_string(layer) + ".";
        return {{p + "input_layernorm.weight", {4096}},
                {p + "self_attn.q_proj.weight", {4096, 4096}},
                {p + "self_attn.k_proj.weight", {1024, 4096}},
                {p + "self_attn.v_proj.weight", {1024, 4096}},
                {p + "self_attn.o_proj.weight", {4096, 4096}},
                {p + "self_attn.q_norm.weight", {128}},
                {p + "self_attn.k_norm.weight", {128}},
                {p + "post_attention_layernorm.weight", {4096}},
                {p + "mlp.gate_proj.weight", {12288, 4096}},
                {p + "mlp.up_proj.weight", {12288, 4096}},
                {p + "mlp.down_proj.weight", {4096, 12288}}};
    }

    std::size_t elements(const std::vector<std::int64_t> &shape)
    {
        std::size_t n = 1;
        for (auto d : shape)
            n *= static_cast<std::size_t>(d);
        return n;
    }

    // Writes the checkpoint; returns the tensor names in file order.
    std::vector<std::string> write_checkpoint(const fs::path &path, int layers, std::size_t &data_bytes)
    {
        std::vector<Entry> entries;
        for (int l = 0; l < layers; ++l)
            for (auto &e : layer_entries(l))
                entries.push_back(std::move(e));
        std::string header = "{";
        std::size_t offset = 0;
        std::vector<std::string> names;
        for (std::size_t i = 0; i < entries.size(); ++i)
        {
            const std::size_t bytes = 2 * elements(entries[i].shape);
            std::string shape;
            for (std::size_t d = 0; d < entries[i].shape.size(); ++d)
                shape += (d ? "," : "") + std::to_string(entries[i].shape[d]);
            header += (i ? "," : "") + ("\"" + entries[i].name + "\":{\"dtype\":\"BF16\",\"shape\":[" + shape +
                                        "],\"data_offsets\":[" + std::to_string(offset) + "," +
                                        std::to_string(offset + bytes) + "]}");
            offset += bytes;
            names.push_back(entries[i].name);
        }
        header += "}";
        data_bytes = offset;
        std::ofstream f(path, std::ios::binary);
        std::uint64_t len = header.size();
        char prefix[8];
        for (int i = 0; i < 8; ++i)
            prefix[i] = static_cast<char>((len >> (8 * i)) & 0xff);
        f.write(prefix, 8);
        f.write(header.data(), static_cast<std::streamsize>(header.size()));
        std::vector<std::uint64_t> block(4u << 20);   // 32 MiB of xorshift words at a time
        std::uint64_t s = 0x9e3779b97f4a7c15ull;
        for (std::size_t done = 0; done < offset;)
        {
            for (auto &w : block)
            {
                s ^= s << 13;
                s ^= s >> 7;
                s ^= s << 17;
                w = s;
            }
            const std::size_t n = std::min(offset - done, block.size() * 8);
            f.write(reinterpret_cast<const char *>(block.data()), static_cast<std::streamsize>(n));
            done += n;
        }
        if (!f)
            throw std::runtime_error("writing " + path.string() + " failed");
        return names;
    }

    double seconds_since(std::chrono::steady_clock::time_point t0)
    {
        return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    }

    // The staged scheme with a configurable shape: each chunk of at most
    // slot_bytes is copied by `threads` host threads (the loader's copy crew)
    // into the next pinned slot (after that slot's previous DMA has
    // completed), then sent with an async copy on one stream.  threads = 1,
    // slots = 2, 32 MiB is the reference's scheme (src/io/
    // safetensors_loader.cpp:92 allocates with cudaHostAllocDefault, as this
    // does).  Returns seconds from the mapping to the last DMA.
    double staged_load(const fs::path &path, const std::vector<std::string> &names, int threads, int slots,
                       std::size_t slot_bytes, std::vector<qwen3::Tensor> &out)
    {
        const auto t0 = std::chrono::steady_clock::now();
        qwen3::SafetensorsFile file(path);
        qwen3::SafetensorsMetadata meta(file);
        hipStream_t stream = nullptr;
        QWEN3_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        std::vector<void *> staging(slots, nullptr);
        std::vector<hipEvent_t> events(slots, nullptr);
        for (int i = 0; i < slots; ++i)
        {
            QWEN3_HIP_CHECK(hipHostMalloc(&staging[i], slot_bytes, hipHostMallocDefault));
            QWEN3_HIP_CHECK(hipEventCreateWithFlags(&events[i], hipEventDisableTiming));
        }
        out.clear();
        for (const auto &n : names)
        {
            const auto &info = meta.tensor(n);
            out.push_back(qwen3::Tensor::empty(info.shape, info.dtype, qwen3::Device::cuda(0)));
        }
        std::vector<bool> busy(slots, false);
        std::size_t next = 0;
        qwen3::detail::CopyCrew crew(static_cast<unsigned>(threads - 1));
        for (std::size_t t = 0; t < names.size(); ++t)
        {
            const auto &info = meta.tensor(names[t]);
            const std::byte *src = file.data_bytes().data() + info.begin_offset;
            auto *dst = static_cast<std::byte *>(out[t].data());
            for (std::size_t done = 0; done < info.size_bytes();)
            {
                const std::size_t slot = next++ % static_cast<std::size_t>(slots);
                if (busy[slot])
                    QWEN3_HIP_CHECK(hipEventSynchronize(events[slot]));
                const std::size_t chunk = std::min(info.size_bytes() - done, slot_bytes);
                crew.copy(staging[slot], src + done, chunk);
                QWEN3_HIP_CHECK(hipMemcpyAsync(dst + done, staging[slot], chunk, hipMemcpyHostToDevice, stream));
                QWEN3_HIP_CHECK(hipEventRecord(events[slot], stream));
                busy[slot] = true;
                done += chunk;
            }
        }
        QWEN3_HIP_CHECK(hipStreamSynchronize(stream));
        const double s = seconds_since(t0);
        for (int i = 0; i < slots; ++i)
        {
            QWEN3_HIP_CHECK(hipEventDestroy(events[i]));
            QWEN3_HIP_CHECK(hipHostFree(staging[i]));
        }
        QWEN3_HIP_CHECK(hipStreamDestroy(stream));
        return s;
    }

    double loader_load(const fs::path &path, const std::vector<std::string> &names, std::vector<qwen3::Tensor> &out)
    {
        const auto t0 = std::chrono::steady_clock::now();
        qwen3::SafetensorsLoader loader(path);
        out = loader.load_many(names, qwen3::Device::cuda(0));
        return seconds_since(t0);
    }

    // Host-to-device DMA from one resident pinned buffer, total bytes in pieces of `piece`.
    double dma_ceiling(std::size_t total, std::size_t piece)
    {
        void *host = nullptr, *dev = nullptr;
        QWEN3_HIP_CHECK(hipHostMalloc(&host, piece, hipHostMallocDefault));
        QWEN3_HIP_CHECK(hipMalloc(&dev, piece));
        std::memset(host, 1, piece);
        hipStream_t stream = nullptr;
        QWEN3_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        QWEN3_HIP_CHECK(hipMemcpyAsync(dev, host, piece, hipMemcpyHostToDevice, stream));
        QWEN3_HIP_CHECK(hipStreamSynchronize(stream));
        const auto t0 = std::chrono::steady_clock::now();
        for (std::size_t done = 0; done < total; done += piece)
            QWEN3_HIP_CHECK(hipMemcpyAsync(dev, host, std::min(piece, total - done), hipMemcpyHostToDevice, stream));
        QWEN3_HIP_CHECK(hipStreamSynchronize(stream));
        const double s = seconds_since(t0);
        QWEN3_HIP_CHECK(hipStreamDestroy(stream));
        QWEN3_HIP_CHECK(hipFree(dev));
        QWEN3_HIP_CHECK(hipHostFree(host));
        return s;
    }

    // The staging copies alone: a fresh mapping copied into a pinned ring by `threads` threads.
    double host_copy(const fs::path &path, const std::vector<std::string> &names, int threads)
    {
        constexpr std::size_t ring = 64u << 20, slot = 32u << 20;
        void *host = nullptr;
        QWEN3_HIP_CHECK(hipHostMalloc(&host, ring, hipHostMallocDefault));
        const auto t0 = std::chrono::steady_clock::now();
        {
            qwen3::SafetensorsFile file(path);
            qwen3::SafetensorsMetadata meta(file);
            qwen3::detail::CopyCrew crew(static_cast<unsigned>(threads - 1));
            std::size_t pos = 0;
            for (const auto &n : names)
            {
                const auto &info = meta.tensor(n);
                const std::byte *src = file.data_bytes().data() + info.begin_offset;
                for (std::size_t done = 0; done < info.size_bytes();)
                {
                    const std::size_t chunk = std::min(info.size_bytes() - done, slot);
                    crew.copy(static_cast<char *>(host) + pos, src + done, chunk);
                    pos = (pos + slot) % ring;
                    done += chunk;
                }
            }
        }
        const double s = seconds_since(t0);
        QWEN3_HIP_CHECK(hipHostFree(host));
        return s;
    }

    // One-off costs inside a load: mapping + header parse, the output
    // tensors' device allocations, the pinned staging, the stream.
    std::string setup_breakdown(const fs::path &path, const std::vector<std::string> &names)
    {
        auto t0 = std::chrono::steady_clock::now();
        qwen3::SafetensorsFile file(path);
        qwen3::SafetensorsMetadata meta(file);
        const double map_s = seconds_since(t0);
        t0 = std::chrono::steady_clock::now();
        std::vector<qwen3::Tensor> out;
        for (const auto &n : names)
        {
            const auto &info = meta.tensor(n);
            out.push_back(qwen3::Tensor::empty(info.shape, info.dtype, qwen3::Device::cuda(0)));
        }
        const double alloc_s = seconds_since(t0);
        t0 = std::chrono::steady_clock::now();
        std::vector<void *> staging(qwen3::io_detail::StagedUpload::kSlots, nullptr);
        for (auto &p : staging)
            QWEN3_HIP_CHECK(hipHostMalloc(&p, qwen3::io_detail::StagedUpload::kSlotBytes, hipHostMallocDefault));
        const double pin_s = seconds_since(t0);
        t0 = std::chrono::steady_clock::now();
        hipStream_t stream = nullptr;
        QWEN3_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        const double stream_s = seconds_since(t0);
        QWEN3_HIP_CHECK(hipStreamDestroy(stream));
        for (auto p : staging)
            QWEN3_HIP_CHECK(hipHostFree(p));
        char buf[256];
        std::snprintf(buf, sizeof(buf),
                      "{\"map_ms\": %.3f, \"tensor_alloc_ms\": %.3f, \"staging_alloc_ms\": %.3f, \"stream_ms\": %.3f}",
                      map_s * 1e3, alloc_s * 1e3, pin_s * 1e3, stream_s * 1e3);
        return buf;
    }

    double best_of(int repeats, const std::function<double()> &f)
    {
        double best = 1e30;
        for (int r = 0; r < repeats; ++r)
            best = std::min(best, f());
        return best;
    }

    void check_bytes(const fs::path &path, const std::vector<std::string> &names, const std::vector<qwen3::Tensor> &got)
    {
        qwen3::SafetensorsFile file(path);
        qwen3::SafetensorsMetadata meta(file);
        std::vector<char> host;
        for (std::size_t t = 0; t < names.size(); ++t)
        {
            const auto &info = meta.tensor(names[t]);
            host.resize(info.size_bytes());
            QWEN3_HIP_CHECK(hipMemcpy(host.data(), got[t].data(), host.size(), hipMemcpyDeviceToHost));
            if (std::memcmp(host.data(), file.data_bytes().data() + info.begin_offset, host.size()) != 0)
                throw std::runtime_error("loaded bytes differ from the file for " + names[t]);
        }
    }
} // namespace

int main(int argc, char **argv)
{
    int layers = 4, repeats = 3;
    bool sweep = false;
    fs::path dir = fs::temp_directory_path();
    for (int i = 1; i < argc; ++i)
    {
        const std::string a = argv[i];
        if (a == "--layers" && i + 1 < argc)
            layers = std::stoi(argv[++i]);
        else if (a == "--repeats" && i + 1 < argc)
            repeats = std::stoi(argv[++i]);
        else if (a == "--dir" && i + 1 < argc)
            dir = argv[++i];
        else if (a == "--sweep")
            sweep = true;
        else
        {
            std::fprintf(stderr, "usage: %s [--layers L] [--repeats R] [--dir D] [--sweep]\n", argv[0]);
            return 2;
        }
    }
    if (layers < 1 || repeats < 1)
    {
        std::fprintf(stderr, "--layers and --repeats must be positive\n");
        return 2;
    }
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1)
    {
        std::fprintf(stderr, "no visible GPU\n");
        return 1;
    }
    const fs::path path = dir / ("q3k_weight_io_" + std::to_string(::getpid()) + ".safetensors");
    try
    {
        std::size_t bytes = 0;
        const auto names = write_checkpoint(path, layers, bytes);
        std::fprintf(stderr, "[weight_io] wrote %s: %d layers, %.1f MiB of tensors\n", path.c_str(), layers,
                     bytes / 1048576.0);
        const double gb = bytes / 1e9;
        std::vector<qwen3::Tensor> out;
        auto rate = [&](double s) { return gb / s; };

        const double ref = best_of(repeats, [&] { return staged_load(path, names, 1, 2, 32u << 20, out); });
        out.clear();
        std::fprintf(stderr, "[weight_io] reference scheme %.2f GB/s\n", rate(ref));
        const double ld = best_of(repeats, [&] { return loader_load(path, names, out); });
        out.clear();
        const double warm = best_of(repeats, [&] {
            qwen3::SafetensorsLoader loader(path);
            out = loader.load_many(names, qwen3::Device::cuda(0));
            out.clear();
            const auto t0 = std::chrono::steady_clock::now();
            out = loader.load_many(names, qwen3::Device::cuda(0));
            return seconds_since(t0);
        });
        std::fprintf(stderr, "[weight_io] loader, second batch on one loader %.2f GB/s\n", rate(warm));
        check_bytes(path, names, out);
        out.clear();
        std::fprintf(stderr, "[weight_io] loader %.2f GB/s (bytes checked)\n", rate(ld));
        const double dma = best_of(repeats, [&] { return dma_ceiling(bytes, 32u << 20); });
        const double dma8 = best_of(repeats, [&] { return dma_ceiling(bytes, 8u << 20); });
        std::fprintf(stderr, "[weight_io] dma ceiling %.2f GB/s (8 MiB pieces %.2f)\n", rate(dma), rate(dma8));
        std::string host_legs;
        for (int t : {1, 2, 4, 8})
        {
            const double h = best_of(repeats, [&] { return host_copy(path, names, t); });
            host_legs += ", \"host_copy_t" + std::to_string(t) + "\": " + std::to_string(rate(h));
        }
        const std::string setup = setup_breakdown(path, names);
        std::fprintf(stderr, "[weight_io] setup %s\n", setup.c_str());
        std::string sweep_legs;
        if (sweep)
            for (int t : {1, 4, 8})
                for (int s : {2, 3, 4})
                    for (std::size_t mb : {4u, 8u, 16u, 32u})
                    {
                        const double x = best_of(repeats, [&] { return staged_load(path, names, t, s, mb << 20, out); });
                        out.clear();
                        std::fprintf(stderr, "[weight_io] sweep threads %d slots %d slot %zu MiB: %.2f GB/s\n", t, s,
                                     mb, rate(x));
                        sweep_legs += std::string(sweep_legs.empty() ? "" : ", ") + "\"t" + std::to_string(t) + "_s" +
                                      std::to_string(s) + "_" + std::to_string(mb) + "MiB\": " + std::to_string(rate(x));
                    }
        std::printf("{\"metric\": \"weight_io\", \"unit\": \"GB/s\", \"bytes\": %zu, \"layers\": %d, \"repeats\": %d, "
                    "\"loader\": %.3f, \"loader_second_batch\": %.3f, \"reference\": %.3f, \"dma_ceiling\": %.3f, "
                    "\"dma_ceiling_8MiB\": %.3f%s, \"setup\": %s%s%s%s}\n",
                    bytes, layers, repeats, rate(ld), rate(warm), rate(ref), rate(dma), rate(dma8), host_legs.c_str(), setup.c_str(),
                    sweep ? ", \"sweep\": {" : "", sweep_legs.c_str(), sweep ? "}" : "");
    }
    catch (const std::exception &e)
    {
        std::fprintf(stderr, "weight_io bench failed: %s\n", e.what());
        fs::remove(path);
        return 1;
    }
    fs::remove(path);
    return 0;
}
