// The safetensors loader to the GPU: load() and the pinned, staged
// load_many() (a tensor larger than all staging buffers together, batches
// large enough for the copy crew, an unknown name in such a batch),
// byte-identical to the host load; the checkpoint's grouped load_many.
#include "gpu_util.hpp"
#include "qwen3/io/safetensors_checkpoint.h"
#include "qwen3/io/safetensors_loader.h"

#include <cstring>
#include <filesystem>
#include <fstream>
#include <stdexcept>
#include <string>
#include <unistd.h>

namespace fs = std::filesystem;
using qwen3::Shape;
using test::require;

namespace
{
    fs::path golden_dir()
    {
        return fs::canonical("/proc/self/exe").parent_path().parent_path().parent_path() / "golden";
    }

    bool same_bytes(const qwen3::Tensor &gpu, const qwen3::Tensor &host)
    {
        const auto g = test::to_host<std::uint8_t>(gpu);
        return g.size() == host.nbytes() && std::memcmp(g.data(), host.data(), host.nbytes()) == 0;
    }

    void body()
    {
        test::require_gpu();
        const int before = test::current_device();
        const auto gpu = qwen3::Device::cuda(0), cpu = qwen3::Device::cpu();
        qwen3::SafetensorsCheckpoint sharded(golden_dir() / "safetensors_sharded");
        const std::vector<std::string> names{"b.weight", "a.weight", "b.scale", "a.bias"};
        const auto on_gpu = sharded.load_many(names, gpu);
        const auto on_cpu = sharded.load_many(names, cpu);
        for (std::size_t i = 0; i < names.size(); ++i)
            require(on_gpu[i].device() == gpu && same_bytes(on_gpu[i], on_cpu[i]), "sharded tensors on the GPU");

        // a 40 MiB bf16 tensor wraps around the three 8 MiB staging buffers
        const fs::path d = fs::temp_directory_path() / ("q3k_io_gpu_" + std::to_string(::getpid()));
        fs::create_directories(d);
        const std::size_t n = 20u * 1024u * 1024u + 77u;
        std::string header = "{\"big\":{\"dtype\":\"BF16\",\"shape\":[" + std::to_string(n) +
                             "],\"data_offsets\":[0," + std::to_string(2 * n) +
                             "]},\"small\":{\"dtype\":\"F32\",\"shape\":[3],\"data_offsets\":[" + std::to_string(2 * n) +
                             "," + std::to_string(2 * n + 12) + "]}}";
        std::string bytes(8, '\0');
        for (int i = 0; i < 8; ++i)
            bytes[static_cast<std::size_t>(i)] = static_cast<char>((header.size() >> (8 * i)) & 0xff);
        bytes += header;
        std::string data(2 * n + 12, '\0');
        for (std::size_t i = 0; i < data.size(); ++i)
            data[i] = static_cast<char>((i * 2654435761u) >> 13);
        bytes += data;
        {
            std::ofstream f(d / "model.safetensors", std::ios::binary);
            f.write(bytes.data(), static_cast<std::streamsize>(bytes.size()));
        }
        qwen3::SafetensorsLoader loader(d / "model.safetensors");
        const auto many = loader.load_many({"big", "small", "big"}, gpu);
        const qwen3::Tensor big_host = loader.load("big", cpu);
        require(same_bytes(many[0], big_host) && same_bytes(many[2], big_host), "40 MiB tensor through the staging");
        require(same_bytes(many[1], loader.load("small", cpu)), "small tensor after a large one");
        require(same_bytes(loader.load("big", gpu), big_host), "single load to the GPU");
        // a batch large enough for the copy crew: an unknown name fails before any transfer
        test::require_throws<std::out_of_range>([&] { (void)loader.load_many({"big", "missing", "big"}, gpu); },
                                                "unknown name in a crew-sized batch");
        // many chunks: the staging slots wrap several times, the small tensor between two large ones
        const auto again = loader.load_many({"big", "big", "small", "big", "big"}, gpu);
        require(again.size() == 5, "five results");
        for (std::size_t i : {0u, 1u, 3u, 4u})
            require(same_bytes(again[i], big_host), "repeated 40 MiB tensor " + std::to_string(i));
        require(same_bytes(again[2], loader.load("small", cpu)), "small tensor among large ones");
        fs::remove_all(d);
        require(test::current_device() == before, "a load changed the current device");
    }
} // namespace

int main() { return test::run("safetensors IO (GPU) test", body); }
