// qwen3::ModelConfig against the reference's test (model_config_test.cpp:
// the Qwen3-0.6B and Qwen3-8B config.json fixtures, kept as data in
// tests/golden/model_config/) and the loader's contract
// (src/model/config.cpp:18-371 of the reference): every check, in its order,
// with its exception type and message, on edited copies of the 8B fixture.
#include "qwen3/model/config.h"

#include "test_util.hpp"

#include <cmath>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <functional>
#include <iostream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <unistd.h>

namespace fs = std::filesystem;
using test::require;

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
        fs::path d = fs::temp_directory_path() / ("q3k_config_test_" + std::to_string(::getpid()));
        fs::create_directories(d);
        return d;
    }

    std::string read_text(const fs::path &p)
    {
        std::ifstream f(p, std::ios::binary);
        return {std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>()};
    }

    fs::path write_config(const std::string &text)
    {
        static int counter = 0;
        const fs::path p = scratch_dir() / ("config_" + std::to_string(counter++) + ".json");
        std::ofstream f(p, std::ios::binary | std::ios::trunc);
        f << text;
        return p;
    }

    // The fixture's members sit one per line ("key": value, ending at ",\n"
    // or at the closing "\n}"); these edit one member's value or drop it.
    std::pair<std::size_t, std::size_t> member_value(const std::string &text, const std::string &key)
    {
        const std::string tag = "\"" + key + "\": ";
        const std::size_t at = text.find(tag);
        require(at != std::string::npos, "fixture has no member " + key);
        const std::size_t start = at + tag.size();
        const std::size_t end = std::min(text.find(",\n", start), text.find("\n}", start));
        return {start, end};
    }

    std::string with_member(std::string text, const std::string &key, const std::string &json)
    {
        const auto [start, end] = member_value(text, key);
        return text.replace(start, end - start, json);
    }

    std::string without_member(std::string text, const std::string &key)
    {
        const std::size_t line = text.rfind('\n', text.find("\"" + key + "\": "));
        const auto [start, end] = member_value(text, key);
        // drop the member's line with its comma (or the comma before it, for the last member)
        if (text.compare(end, 2, ",\n") == 0)
            return text.erase(line, end + 1 - line);
        const std::size_t comma = text.rfind(',', line);
        return text.erase(comma, end - comma);
    }

    template <typename Exception>
    void expect_error(const std::function<void()> &f, const std::string &message, bool prefix = false)
    {
        try
        {
            f();
        }
        catch (const Exception &e)
        {
            const std::string what = e.what();
            const bool ok = prefix ? what.rfind(message, 0) == 0 : what == message;
            require(ok, "expected \"" + message + "\", got \"" + what + "\"");
            return;
        }
        catch (const std::exception &e)
        {
            require(false, "wrong exception type for \"" + message + "\": " + e.what());
        }
        require(false, "no exception, expected \"" + message + "\"");
    }

    template <typename Exception>
    void load_error(const std::string &text, const std::string &message)
    {
        const fs::path p = write_config(text);
        expect_error<Exception>([&] { (void)qwen3::load_model_config(p); }, message);
    }

    qwen3::ModelConfig load_text(const std::string &text) { return qwen3::load_model_config(write_config(text)); }

    bool same(const qwen3::ModelConfig &a, const qwen3::ModelConfig &b)
    {
        return a.vocab_size == b.vocab_size && a.hidden_size == b.hidden_size &&
               a.intermediate_size == b.intermediate_size && a.num_hidden_layers == b.num_hidden_layers &&
               a.num_attention_heads == b.num_attention_heads && a.num_key_value_heads == b.num_key_value_heads &&
               a.head_dim == b.head_dim && a.max_position_embeddings == b.max_position_embeddings &&
               a.rope_theta == b.rope_theta && a.rms_norm_eps == b.rms_norm_eps && a.bos_token_id == b.bos_token_id &&
               a.eos_token_id == b.eos_token_id && a.attention_bias == b.attention_bias &&
               a.tie_word_embeddings == b.tie_word_embeddings && a.use_sliding_window == b.use_sliding_window;
    }

    void reference_test_cases()
    {
        const qwen3::ModelConfig small = qwen3::load_model_config(golden_dir() / "model_config" / "qwen3_0_6b.json");
        require(small.hidden_size == 1024 && small.num_hidden_layers == 28, "0.6B sizes");
        require(small.q_projection_size() == 2048 && small.kv_projection_size() == 1024, "0.6B projections");
        require(small.query_heads_per_kv_head() == 2 && small.tie_word_embeddings, "0.6B GQA group / tied");
        require(same(small, qwen3::make_qwen3_0_6b_config()), "0.6B fixture differs from make_qwen3_0_6b_config");

        const qwen3::ModelConfig large = qwen3::load_model_config(golden_dir() / "model_config" / "qwen3_8b.json");
        require(large.hidden_size == 4096 && large.num_hidden_layers == 36, "8B sizes");
        require(large.q_projection_size() == 4096 && large.kv_projection_size() == 1024, "8B projections");
        require(large.query_heads_per_kv_head() == 4 && !large.tie_word_embeddings, "8B GQA group / untied");
        require(large.intermediate_size == 12288 && large.vocab_size == 151936 && large.head_dim == 128 &&
                    large.max_position_embeddings == 40960 && large.rope_theta == 1.0e6F &&
                    large.rms_norm_eps == 1.0e-6F && large.bos_token_id == 151643 && large.eos_token_id == 151645,
                "8B values");

        qwen3::ModelConfig invalid = large;
        invalid.num_key_value_heads = 6;
        expect_error<std::invalid_argument>([&] { invalid.validate(); },
                                            "num_attention_heads must be divisible by num_key_value_heads");
    }

    void validate_rules()
    {
        const qwen3::ModelConfig base = qwen3::make_qwen3_0_6b_config();
        auto check = [&](const std::function<void(qwen3::ModelConfig &)> &edit, const std::string &message) {
            qwen3::ModelConfig c = base;
            edit(c);
            expect_error<std::invalid_argument>([&] { c.validate(); }, message);
        };
        // the reference's message has no space after the field name
        check([](auto &c) { c.vocab_size = 0; }, "vocab_sizemust be positive");
        check([](auto &c) { c.hidden_size = -1; }, "hidden_sizemust be positive");
        check([](auto &c) { c.intermediate_size = 0; }, "intermediate_sizemust be positive");
        check([](auto &c) { c.num_hidden_layers = 0; }, "num_hidden_layersmust be positive");
        check([](auto &c) { c.num_attention_heads = 0; }, "num_attention_headsmust be positive");
        check([](auto &c) { c.num_key_value_heads = 0; }, "num_key_value_headsmust be positive");
        check([](auto &c) { c.head_dim = 0; }, "head_dimmust be positive");
        check([](auto &c) { c.max_position_embeddings = 0; }, "max_position_embeddingsmust be positive");
        // first failing rule wins
        check([](auto &c) { c.vocab_size = 0; c.head_dim = 0; }, "vocab_sizemust be positive");
        check([](auto &c) { c.head_dim = 127; }, "head_dim must be even for RoPE");
        check([](auto &c) { c.rope_theta = 0.0F; }, "rope_theta must be finite and positive");
        check([](auto &c) { c.rope_theta = -1.0F; }, "rope_theta must be finite and positive");
        check([](auto &c) { c.rope_theta = INFINITY; }, "rope_theta must be finite and positive");
        check([](auto &c) { c.rope_theta = NAN; }, "rope_theta must be finite and positive");
        check([](auto &c) { c.rms_norm_eps = 0.0F; }, "rms_norm_eps must be finite and positive");
        check([](auto &c) { c.rms_norm_eps = NAN; }, "rms_norm_eps must be finite and positive");
        check([](auto &c) { c.bos_token_id = -1; }, "bos_token_id is outside the vocabulary");
        check([](auto &c) { c.bos_token_id = c.vocab_size; }, "bos_token_id is outside the vocabulary");
        check([](auto &c) { c.eos_token_id = c.vocab_size; }, "eos_token_id is outside the vocabulary");
        check([](auto &c) { c.attention_bias = true; }, "attention bias is not supported");
        check([](auto &c) { c.use_sliding_window = true; }, "sliding-window attention is not supported");

        qwen3::ModelConfig edge = base;
        edge.bos_token_id = 0;
        edge.eos_token_id = edge.vocab_size - 1;
        edge.validate();
        qwen3::ModelConfig no_kv;
        require(no_kv.query_heads_per_kv_head() == 0, "no KV heads gives a group size of 0");
        require(qwen3::ModelConfig{}.bos_token_id == -1 && qwen3::ModelConfig{}.eos_token_id == -1,
                "token id defaults");
    }

    void loader_rules()
    {
        const std::string good = read_text(golden_dir() / "model_config" / "qwen3_8b.json");
        using RE = std::runtime_error;
        using IA = std::invalid_argument;

        // file and document
        const fs::path missing = scratch_dir() / "no_such_config.json";
        expect_error<RE>([&] { (void)qwen3::load_model_config(missing); },
                         "cannot open model config: " + missing.string());
        const fs::path bad = write_config("{\"model_type\": \"qwen3\",");
        expect_error<RE>([&] { (void)qwen3::load_model_config(bad); },
                         "cannot parse model config '" + bad.string() + "': ", true);
        const fs::path empty = write_config("");
        expect_error<RE>([&] { (void)qwen3::load_model_config(empty); },
                         "cannot parse model config '" + empty.string() + "': ", true);
        load_error<RE>("[1, 2]", "model config root must be a JSON object");
        load_error<RE>("\"qwen3\"", "model config root must be a JSON object");
        require(same(load_text("\xEF\xBB\xBF" + good), load_text(good)), "a UTF-8 byte order mark is skipped");
        require(same(load_text(good + "\n{ not json"), load_text(good)), "text after the root value is not read");

        // the checks before the numeric fields, in order
        load_error<RE>(without_member(good, "model_type"), "missing required config field 'model_type'");
        load_error<RE>(with_member(good, "model_type", "3"), "config field 'model_type' must be a string");
        load_error<IA>(with_member(good, "model_type", "\"llama\""), "only Qwen3 Dense models are supported");
        load_error<IA>(with_member(without_member(good, "vocab_size"), "model_type", "\"qwen2\""),
                       "only Qwen3 Dense models are supported");
        load_error<RE>(without_member(good, "architectures"), "missing required config field 'architectures'");
        load_error<RE>(with_member(good, "architectures", "\"Qwen3ForCausalLM\""),
                       "config field 'architechtures' must be an array");
        load_error<IA>(with_member(good, "architectures", "[\"LlamaForCausalLM\", 5]"),
                       "only Qwen3ForCausalLM is supported");
        load_error<IA>(with_member(good, "architectures", "[]"), "only Qwen3ForCausalLM is supported");
        (void)load_text(with_member(good, "architectures", "[5, {\"a\": 1}, \"Qwen3ForCausalLM\"]"));
        load_error<IA>(with_member(good, "hidden_act", "\"gelu\""), "only the SiLU activation is supported");
        load_error<RE>(without_member(good, "hidden_act"), "missing required config field 'hidden_act'");
        load_error<IA>(with_member(good, "torch_dtype", "\"float16\""), "only BF16 Qwen3 checkpoints are supported");
        load_error<IA>(with_member(good, "rope_scaling", "{\"rope_type\": \"yarn\"}"),
                       "config field 'rope_scaling' is not support yet");
        load_error<IA>(with_member(good, "sliding_window", "4096"), "config field 'sliding_window' is not support yet");
        load_error<IA>(with_member(good, "sliding_window", "false"), "config field 'sliding_window' is not support yet");
        load_error<IA>(with_member(good, "use_cache", "true, \"quantization_config\": {}"),
                       "config field 'quantization_config' is not support yet");
        (void)load_text(without_member(without_member(good, "rope_scaling"), "sliding_window"));
        (void)load_text(with_member(good, "use_cache", "true, \"quantization_config\": null"));

        // integers
        load_error<RE>(without_member(good, "vocab_size"), "missing required config field 'vocab_size'");
        load_error<RE>(with_member(good, "vocab_size", "151936.0"), "config field 'vocab_size' must be an integar");
        load_error<RE>(with_member(good, "hidden_size", "4e3"), "config field 'hidden_size' must be an integar");
        load_error<RE>(with_member(good, "head_dim", "\"128\""), "config field 'head_dim' must be an integar");
        load_error<RE>(with_member(good, "head_dim", "true"), "config field 'head_dim' must be an integar");
        load_error<RE>(with_member(good, "num_hidden_layers", "2147483648"),
                       "config field 'num_hidden_layers' is outside the int32 range");
        load_error<RE>(with_member(good, "bos_token_id", "-2147483649"),
                       "config field 'bos_token_id' is outside the int32 range");
        // beyond uint64 / int64 the number is a double, so not an integer
        load_error<RE>(with_member(good, "eos_token_id", "18446744073709551616"),
                       "config field 'eos_token_id' must be an integar");
        load_error<RE>(with_member(good, "eos_token_id", "-9223372036854775809"),
                       "config field 'eos_token_id' must be an integar");
        // a uint64 above INT64_MAX keeps its bits as int64: 2^64 - 1 reads as -1
        load_error<IA>(with_member(good, "eos_token_id", "18446744073709551615"),
                       "eos_token_id is outside the vocabulary");
        require(load_text(with_member(good, "bos_token_id", "-0")).bos_token_id == 0, "-0 is the integer 0");
        require(load_text(with_member(good, "max_position_embeddings", "2147483647")).max_position_embeddings ==
                    2147483647,
                "INT32_MAX is accepted");
        // a repeated key keeps its last value
        require(load_text(with_member(good, "hidden_size", "1, \"hidden_size\": 2048")).hidden_size == 2048,
                "repeated key: the last value");
        // validate() runs after all fields are read
        load_error<IA>(with_member(good, "num_key_value_heads", "6"),
                       "num_attention_heads must be divisible by num_key_value_heads");
        load_error<IA>(with_member(good, "vocab_size", "0"), "vocab_sizemust be positive");

        // floats
        load_error<RE>(with_member(good, "rope_theta", "\"1e6\""), "config field 'rope_theta' must be numeric");
        load_error<RE>(with_member(good, "rope_theta", "null"), "config field 'rope_theta' must be numeric");
        load_error<RE>(with_member(good, "rope_theta", "1e39"), "config field 'rope_theta' cannot be represented as float");
        load_error<RE>(with_member(good, "rms_norm_eps", "-1e400"),
                       "config field 'rms_norm_eps' cannot be represented as float");
        load_error<IA>(with_member(good, "rms_norm_eps", "1e-400"), "rms_norm_eps must be finite and positive");
        load_error<IA>(with_member(good, "rms_norm_eps", "-1e-06"), "rms_norm_eps must be finite and positive");
        require(load_text(with_member(good, "rope_theta", "1.0E+6")).rope_theta == 1.0e6F, "exponent form");
        require(load_text(with_member(good, "rope_theta", "10000")).rope_theta == 10000.0F, "an integer as float");
        require(load_text(with_member(good, "rms_norm_eps", "0.00001")).rms_norm_eps == 1.0e-5F, "decimal form");
        require(load_text(with_member(good, "rope_theta", "3.4028234663852886e38")).rope_theta ==
                    3.4028234663852886e38F,
                "FLT_MAX is accepted");

        // booleans
        load_error<RE>(with_member(good, "attention_bias", "0"), "config field 'attention_bias' must be boolean");
        load_error<RE>(without_member(good, "tie_word_embeddings"),
                       "missing required config field 'tie_word_embeddings'");
        load_error<IA>(with_member(good, "attention_bias", "true"), "attention bias is not supported");
        load_error<IA>(with_member(good, "use_sliding_window", "true"), "sliding-window attention is not supported");
        require(load_text(with_member(good, "tie_word_embeddings", "true")).tie_word_embeddings, "tied flag");

        // the first failing field in the reference's order: vocab_size is read before hidden_size
        load_error<RE>(with_member(with_member(good, "hidden_size", "1.5"), "vocab_size", "\"x\""),
                       "config field 'vocab_size' must be an integar");
        // rope_theta is read before bos_token_id, booleans last
        load_error<RE>(with_member(with_member(good, "attention_bias", "1"), "rope_theta", "\"x\""),
                       "config field 'rope_theta' must be numeric");
    }
} // namespace

int main()
{
    try
    {
        reference_test_cases();
        validate_rules();
        loader_rules();
        std::error_code ec;
        fs::remove_all(scratch_dir(), ec);
        std::cout << "ModelConfig test passed.\n";
        return EXIT_SUCCESS;
    }
    catch (const std::exception &e)
    {
        std::cerr << "ModelConfig test failed: " << e.what() << '\n';
        return EXIT_FAILURE;
    }
}
