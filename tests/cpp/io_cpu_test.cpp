// The safetensors reader on the host: files written by the official
// safetensors package (tests/golden/safetensors_*), the format errors the
// reference rejects (src/io/safetensors_file.cpp, safetensors_metadata.cpp,
// safetensors_checkpoint.cpp, mapped_file.cpp), and the checkpoint layouts.
#include "qwen3/io/mapped_file.h"
#include "qwen3/io/safetensors_checkpoint.h"
#include "qwen3/io/safetensors_file.h"
#include "qwen3/io/safetensors_loader.h"
#include "qwen3/io/safetensors_metadata.h"
#include "test_util.hpp"

#include <cstdlib>

#include <filesystem>
#include <fstream>
#include <system_error>
#include <unistd.h>

namespace fs = std::filesystem;
using qwen3::DType;
using qwen3::Shape;
using test::require;
using test::require_throws;

namespace
{
    // tests/golden, found from the executable (tests/cpp/build/<name>) or
    // named by Q3K_GOLDEN_DIR for a build elsewhere
    fs::path golden_dir()
    {
        if (const char *d = std::getenv("Q3K_GOLDEN_DIR"))
            return d;
        return fs::canonical("/proc/self/exe").parent_path().parent_path().parent_path() / "golden";
    }

    fs::path scratch_dir()
    {
        fs::path d = fs::temp_directory_path() / ("q3k_io_test_" + std::to_string(::getpid()));
        fs::create_directories(d);
        return d;
    }

    void write_file(const fs::path &p, const std::string &bytes)
    {
        std::ofstream f(p, std::ios::binary | std::ios::trunc);
        f.write(bytes.data(), static_cast<std::streamsize>(bytes.size()));
    }

    // 8-byte little-endian length + header + data
    std::string safetensors_bytes(const std::string &header, const std::string &data, std::uint64_t length = ~0ULL)
    {
        const std::uint64_t n = length == ~0ULL ? header.size() : length;
        std::string out(8, '\0');
        for (int i = 0; i < 8; ++i)
            out[static_cast<std::size_t>(i)] = static_cast<char>((n >> (8 * i)) & 0xff);
        return out + header + data;
    }

    std::uint16_t bf_pattern(std::size_t i) { return q3o_bf16_from_f32(static_cast<float>(static_cast<int>(i % 251) - 125)); }

    void golden_single()
    {
        qwen3::SafetensorsLoader loader(golden_dir() / "safetensors_single" / "model.safetensors");
        const auto &md = loader.metadata();
        require(md.tensor_count() == 4, "four tensors (the __metadata__ entry is skipped)");
        const auto &emb = md.tensor("model.embed_tokens.weight");
        require(emb.dtype == DType::BFloat16 && emb.shape == (Shape{6, 8}) && emb.size_bytes() == 96, "embedding record");
        qwen3::Tensor t = loader.load("model.embed_tokens.weight", qwen3::Device::cpu());
        const auto *v = static_cast<const std::uint16_t *>(t.data());
        for (std::size_t i = 0; i < 48; ++i)
            require(v[i] == bf_pattern(i), "bf16 values");
        qwen3::Tensor f = loader.load("rope.inv_freq", qwen3::Device::cpu());
        require(f.dtype() == DType::Float32 && static_cast<const float *>(f.data())[3] == 0.75F, "f32 values");
        qwen3::Tensor p = loader.load("positions", qwen3::Device::cpu());
        require(p.dtype() == DType::Int32 && static_cast<const std::int32_t *>(p.data())[0] == -2, "i32 values");
        require_throws<std::out_of_range>([&] { (void)md.tensor("missing"); }, "unknown tensor name");
        const auto many = loader.load_many({"model.norm.weight", "positions"}, qwen3::Device::cpu());
        require(many.size() == 2 && many[0].shape() == (Shape{8}), "load_many on the host");
    }

    void golden_checkpoints()
    {
        qwen3::SafetensorsCheckpoint single(golden_dir() / "safetensors_single");
        require(!single.is_sharded() && single.shard_count() == 1 && single.tensor_count() == 4, "single checkpoint");
        qwen3::SafetensorsCheckpoint sharded(golden_dir() / "safetensors_sharded");
        require(sharded.is_sharded() && sharded.shard_count() == 2 && sharded.tensor_count() == 4, "sharded checkpoint");
        require(sharded.tensor_info("b.weight").shape == (Shape{2, 16}), "sharded record");
        const auto ts = sharded.load_many({"b.scale", "a.bias", "b.weight"}, qwen3::Device::cpu());
        require(ts[0].dtype() == DType::Float32 && static_cast<const float *>(ts[0].data())[2] == 1.0F,
                "load_many keeps the requested order (shard 2 first)");
        require(static_cast<const std::uint16_t *>(ts[2].data())[31] == bf_pattern(31), "values from shard 2");
        require_throws<std::out_of_range>([&] { (void)sharded.load("nope", qwen3::Device::cpu()); }, "unknown name");
    }

    void format_errors()
    {
        const fs::path d = scratch_dir();
        const auto expect_format = [&](const std::string &bytes, const char *what) {
            write_file(d / "x.safetensors", bytes);
            require_throws<qwen3::SafetensorsFormatError>(
                [&] {
                    qwen3::SafetensorsFile f(d / "x.safetensors");
                    qwen3::SafetensorsMetadata m(f);
                },
                what);
        };
        expect_format("1234", "file shorter than the length prefix");
        expect_format(safetensors_bytes("", ""), "empty header");
        expect_format(safetensors_bytes("{}", "", 100), "header past the end of the file");
        expect_format(safetensors_bytes(" {}", ""), "header not starting with '{'");
        expect_format(safetensors_bytes("{\"a\":", ""), "invalid JSON");
        expect_format(safetensors_bytes("[1]", ""), "header not an object");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F16","shape":[1],"data_offsets":[0,2]}})", "xx"),
                      "unsupported dtype");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F32","shape":[1]}})", "xxxx"), "missing data_offsets");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}})", "xxxx"),
                      "negative dimension");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}})", "xxxx"),
                      "size mismatch");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F32","shape":[1],"data_offsets":[4,0]}})", "xxxx"),
                      "end before begin");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F32","shape":[1],"data_offsets":[0,8]}})", "xxxx"),
                      "offset past the data");
        expect_format(safetensors_bytes(R"({"a":{"dtype":"F32","shape":[1.0],"data_offsets":[0,4]}})", "xxxx"),
                      "non-integer dimension");
        // accepted: escapes, whitespace, empty shape (scalar), __metadata__
        write_file(d / "ok.safetensors",
                   safetensors_bytes("{ \"__metadata__\" : {\"k\":\"v\"},\n \"t\\u00e9\\n\" : {\"dtype\":\"I32\", "
                                     "\"shape\":[], \"data_offsets\":[0,4]} }",
                                     std::string("\x07\x00\x00\x00", 4)));
        qwen3::SafetensorsLoader ok(d / "ok.safetensors");
        require(ok.metadata().contains("t\xc3\xa9\n"), "escaped names decode to UTF-8");
        require(*static_cast<const std::int32_t *>(ok.load("t\xc3\xa9\n", qwen3::Device::cpu()).data()) == 7,
                "scalar tensor");
        require_throws<std::system_error>([&] { qwen3::MappedFile m(d / "does-not-exist"); }, "missing file");
        require_throws<std::invalid_argument>([&] { qwen3::MappedFile m(d); }, "directory mapped");
        fs::remove_all(d);
    }

    void checkpoint_errors()
    {
        const fs::path d = scratch_dir();
        const fs::path shard_a = golden_dir() / "safetensors_sharded" / "model-00001-of-00002.safetensors";
        const auto make = [&](const std::string &index) {
            fs::remove_all(d);
            fs::create_directories(d);
            fs::copy_file(shard_a, d / "model-00001-of-00002.safetensors");
            write_file(d / "model.safetensors.index.json", index);
        };
        const auto expect_runtime = [&](const std::string &index, const char *what) {
            make(index);
            require_throws<std::runtime_error>([&] { qwen3::SafetensorsCheckpoint c(d); }, what);
        };
        // shard A holds a.weight (3x4 bf16, 24 B) and a.bias (4 bf16, 8 B): 32 bytes
        const std::string wm = R"("weight_map":{"a.weight":"model-00001-of-00002.safetensors","a.bias":"model-00001-of-00002.safetensors"})";
        make("{\"metadata\":{\"total_size\":32}," + wm + "}");
        qwen3::SafetensorsCheckpoint good(d);
        require(good.is_sharded() && good.tensor_count() == 2, "one-shard index");
        expect_runtime("{\"metadata\":{\"total_size\":33}," + wm + "}", "total_size mismatch");
        expect_runtime("{" + wm + "}", "missing metadata");
        expect_runtime(R"({"metadata":{"total_size":8},"weight_map":{"a.bias":"model-00001-of-00002.safetensors"}})",
                       "tensor in a shard but not in the index");
        expect_runtime(R"({"metadata":{"total_size":32},"weight_map":{"a.weight":"../x.safetensors"}})",
                       "shard name with a path");
        expect_runtime(R"({"metadata":{"total_size":32},"weight_map":{"a.weight":"missing.safetensors"}})",
                       "missing shard");
        expect_runtime(R"({"metadata":{"total_size":32},"weight_map":{}})", "empty weight_map");
        expect_runtime("{\"metadata\":{\"total_size\":32}," + wm.substr(0, wm.size() - 1) + ",\"c\":\"model-00001-of-00002.safetensors\"}}",
                       "indexed tensor missing from its shard");
        make("{\"metadata\":{\"total_size\":32}," + wm + "}");
        fs::copy_file(shard_a, d / "model.safetensors");
        require_throws<std::runtime_error>([&] { qwen3::SafetensorsCheckpoint c(d); }, "both layouts present");
        fs::remove_all(d);
        fs::create_directories(d);
        require_throws<std::runtime_error>([&] { qwen3::SafetensorsCheckpoint c(d); }, "neither layout present");
        require_throws<std::invalid_argument>([&] { qwen3::SafetensorsCheckpoint c(d / "nope"); }, "no directory");
        fs::remove_all(d);
    }

    void body()
    {
        golden_single();
        golden_checkpoints();
        format_errors();
        checkpoint_errors();
    }
} // namespace

int main() { return test::run("safetensors IO (CPU) test", body); }
