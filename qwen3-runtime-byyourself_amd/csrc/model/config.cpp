// ModelConfig: the dense Qwen3 config.json, read with the library's pull
// parser into a table of the root object's members (a repeated key keeps its
// last value, as a JSON object does), then checked field by field.
//
// The reference reads the file with nlohmann::json (src/model/config.cpp:
// helpers :18-143, validate :165-244, load_model_config :246-338, the 0.6B
// values :340-371).  What its checks see of a JSON value is restated here:
//   * an integer is a number written without fraction or exponent that fits
//     int64 (with a minus sign) or uint64 (without); any other number is a
//     double, parsed from its text in the C locale (overflow gives +-inf);
//   * an integer read as int64 keeps its bits (a uint64 above INT64_MAX
//     wraps), then the int32 range is checked;
//   * only the root value is parsed: text after it is not read.
// The checks, their order, exception types and messages are the reference's,
// including its spellings.
#include "qwen3/model/config.h"

#include "../io/json_cursor.hpp"

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <fstream>
#include <iterator>
#include <limits>
#include <locale.h>
#include <map>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace qwen3
{
    namespace
    {
        using io_detail::JsonCursor;

        // One member of the root object, as far as the checks look at it.
        struct Member
        {
            enum class Type
            {
                Object,
                Array,
                String,
                Integer,   // int64
                Unsigned,  // uint64
                Float,
                Bool,
                Null
            };
            Type type = Type::Null;
            std::int64_t integer = 0;
            std::uint64_t unsigned_value = 0;
            double number = 0.0;
            std::string string;
            bool boolean = false;
            std::vector<std::optional<std::string>> items;  // an array's items: a string, or nullopt
        };

        using Members = std::map<std::string, Member>;

        // JSON numbers use '.' whatever LC_NUMERIC the process has set.
        double c_locale_strtod(const std::string &text)
        {
            static const locale_t c_locale = newlocale(LC_ALL_MASK, "C", static_cast<locale_t>(0));
            if (c_locale == static_cast<locale_t>(0))
                return std::strtod(text.c_str(), nullptr);
            return strtod_l(text.c_str(), nullptr, c_locale);
        }

        Member read_number(JsonCursor &cur)
        {
            const JsonCursor::Number n = cur.read_number();
            const std::string text(n.text);
            Member m;
            if (n.integral && !n.negative && n.is_unsigned)
            {
                m.type = Member::Type::Unsigned;
                m.unsigned_value = n.value;
                return m;
            }
            if (n.integral && n.negative)
            {
                errno = 0;
                const long long v = std::strtoll(text.c_str(), nullptr, 10);
                if (errno != ERANGE)
                {
                    m.type = Member::Type::Integer;
                    m.integer = v;
                    return m;
                }
            }
            m.type = Member::Type::Float;
            m.number = c_locale_strtod(text);
            return m;
        }

        Member read_member(JsonCursor &cur)
        {
            Member m;
            switch (cur.peek_kind())
            {
            case JsonCursor::Kind::Object:
                cur.skip_value();
                m.type = Member::Type::Object;
                break;
            case JsonCursor::Kind::Array:
                m.type = Member::Type::Array;
                cur.open_array();
                while (cur.next_item())
                {
                    if (cur.peek_kind() == JsonCursor::Kind::String)
                    {
                        m.items.emplace_back(cur.read_string());
                    }
                    else
                    {
                        cur.skip_value();
                        m.items.emplace_back(std::nullopt);
                    }
                }
                break;
            case JsonCursor::Kind::String:
                m.type = Member::Type::String;
                m.string = cur.read_string();
                break;
            case JsonCursor::Kind::Number: m = read_number(cur); break;
            case JsonCursor::Kind::Bool:
                m.type = Member::Type::Bool;
                m.boolean = cur.read_bool();
                break;
            case JsonCursor::Kind::Null:
                cur.read_null();
                m.type = Member::Type::Null;
                break;
            }
            return m;
        }

        // The root value of the text: its members when it is an object, nullopt
        // for any other (well-formed) value.  Malformed JSON throws the parser's
        // std::runtime_error.
        std::optional<Members> parse_root(std::string_view text)
        {
            JsonCursor cur(text);
            if (cur.peek_kind() != JsonCursor::Kind::Object)
            {
                cur.skip_value();
                return std::nullopt;
            }
            Members members;
            cur.open_object();
            std::string key;
            while (cur.next_key(key))
                members[key] = read_member(cur);
            return members;
        }

        void require_positive(std::int32_t value, const char *name)
        {
            if (value <= 0)
                throw std::invalid_argument(std::string(name) + "must be positive");
        }

        const Member &required_field(const Members &root, const char *key)
        {
            const auto it = root.find(key);
            if (it == root.end())
                throw std::runtime_error("missing required config field '" + std::string{key} + "'");
            return it->second;
        }

        std::int32_t read_int32(const Members &root, const char *key)
        {
            const Member &value = required_field(root, key);
            if (value.type != Member::Type::Integer && value.type != Member::Type::Unsigned)
                throw std::runtime_error("config field '" + std::string{key} + "' must be an integar");
            const std::int64_t number =
                value.type == Member::Type::Integer ? value.integer : static_cast<std::int64_t>(value.unsigned_value);
            if (number < std::numeric_limits<std::int32_t>::min() || number > std::numeric_limits<std::int32_t>::max())
                throw std::runtime_error("config field '" + std::string{key} + "' is outside the int32 range");
            return static_cast<std::int32_t>(number);
        }

        float read_float(const Members &root, const char *key)
        {
            const Member &value = required_field(root, key);
            double number;
            switch (value.type)
            {
            case Member::Type::Integer: number = static_cast<double>(value.integer); break;
            case Member::Type::Unsigned: number = static_cast<double>(value.unsigned_value); break;
            case Member::Type::Float: number = value.number; break;
            default: throw std::runtime_error("config field '" + std::string{key} + "' must be numeric");
            }
            if (!std::isfinite(number) || std::fabs(number) > std::numeric_limits<float>::max())
                throw std::runtime_error("config field '" + std::string{key} + "' cannot be represented as float");
            return static_cast<float>(number);
        }

        bool read_bool(const Members &root, const char *key)
        {
            const Member &value = required_field(root, key);
            if (value.type != Member::Type::Bool)
                throw std::runtime_error("config field '" + std::string{key} + "' must be boolean");
            return value.boolean;
        }

        std::string read_string(const Members &root, const char *key)
        {
            const Member &value = required_field(root, key);
            if (value.type != Member::Type::String)
                throw std::runtime_error("config field '" + std::string{key} + "' must be a string");
            return value.string;
        }

        void reject_non_null_field(const Members &root, const char *key)
        {
            const auto it = root.find(key);
            if (it != root.end() && it->second.type != Member::Type::Null)
                throw std::invalid_argument("config field '" + std::string{key} + "' is not support yet");
        }

        void require_qwen3_architecture(const Members &root)
        {
            const Member &architectures = required_field(root, "architectures");
            if (architectures.type != Member::Type::Array)
                throw std::runtime_error("config field 'architechtures' must be an array");
            for (const auto &item : architectures.items)
                if (item && *item == "Qwen3ForCausalLM")
                    return;
            throw std::invalid_argument("only Qwen3ForCausalLM is supported");
        }
    } // namespace

    std::int64_t ModelConfig::q_projection_size() const noexcept
    {
        return static_cast<std::int64_t>(num_attention_heads) * head_dim;
    }

    std::int64_t ModelConfig::kv_projection_size() const noexcept
    {
        return static_cast<std::int64_t>(num_key_value_heads) * head_dim;
    }

    std::int32_t ModelConfig::query_heads_per_kv_head() const noexcept
    {
        return num_key_value_heads == 0 ? 0 : num_attention_heads / num_key_value_heads;
    }

    void ModelConfig::validate() const
    {
        require_positive(vocab_size, "vocab_size");
        require_positive(hidden_size, "hidden_size");
        require_positive(intermediate_size, "intermediate_size");
        require_positive(num_hidden_layers, "num_hidden_layers");
        require_positive(num_attention_heads, "num_attention_heads");
        require_positive(num_key_value_heads, "num_key_value_heads");
        require_positive(head_dim, "head_dim");
        require_positive(max_position_embeddings, "max_position_embeddings");
        if (num_attention_heads % num_key_value_heads != 0)
            throw std::invalid_argument("num_attention_heads must be divisible by num_key_value_heads");
        if (head_dim % 2 != 0)
            throw std::invalid_argument("head_dim must be even for RoPE");
        if (!std::isfinite(rope_theta) || rope_theta <= 0.0F)
            throw std::invalid_argument("rope_theta must be finite and positive");
        if (!std::isfinite(rms_norm_eps) || rms_norm_eps <= 0.0F)
            throw std::invalid_argument("rms_norm_eps must be finite and positive");
        if (bos_token_id < 0 || bos_token_id >= vocab_size)
            throw std::invalid_argument("bos_token_id is outside the vocabulary");
        if (eos_token_id < 0 || eos_token_id >= vocab_size)
            throw std::invalid_argument("eos_token_id is outside the vocabulary");
        if (attention_bias)
            throw std::invalid_argument("attention bias is not supported");
        if (use_sliding_window)
            throw std::invalid_argument("sliding-window attention is not supported");
    }

    ModelConfig load_model_config(const std::filesystem::path &config_path)
    {
        std::ifstream input{config_path, std::ios::binary};
        if (!input)
            throw std::runtime_error("cannot open model config: " + config_path.string());
        const std::string text{std::istreambuf_iterator<char>(input), std::istreambuf_iterator<char>()};

        std::optional<Members> parsed;
        try
        {
            parsed = parse_root(text);
        }
        catch (const std::runtime_error &error)
        {
            throw std::runtime_error("cannot parse model config '" + config_path.string() + "': " + error.what());
        }
        if (!parsed)
            throw std::runtime_error("model config root must be a JSON object");
        const Members &root = *parsed;

        if (read_string(root, "model_type") != "qwen3")
            throw std::invalid_argument("only Qwen3 Dense models are supported");
        require_qwen3_architecture(root);
        if (read_string(root, "hidden_act") != "silu")
            throw std::invalid_argument("only the SiLU activation is supported");
        if (read_string(root, "torch_dtype") != "bfloat16")
            throw std::invalid_argument("only BF16 Qwen3 checkpoints are supported");
        reject_non_null_field(root, "rope_scaling");
        reject_non_null_field(root, "sliding_window");
        reject_non_null_field(root, "quantization_config");

        ModelConfig config;
        config.vocab_size = read_int32(root, "vocab_size");
        config.hidden_size = read_int32(root, "hidden_size");
        config.intermediate_size = read_int32(root, "intermediate_size");
        config.num_hidden_layers = read_int32(root, "num_hidden_layers");
        config.num_attention_heads = read_int32(root, "num_attention_heads");
        config.num_key_value_heads = read_int32(root, "num_key_value_heads");
        config.head_dim = read_int32(root, "head_dim");
        config.max_position_embeddings = read_int32(root, "max_position_embeddings");
        config.rope_theta = read_float(root, "rope_theta");
        config.rms_norm_eps = read_float(root, "rms_norm_eps");
        config.bos_token_id = read_int32(root, "bos_token_id");
        config.eos_token_id = read_int32(root, "eos_token_id");
        config.attention_bias = read_bool(root, "attention_bias");
        config.tie_word_embeddings = read_bool(root, "tie_word_embeddings");
        config.use_sliding_window = read_bool(root, "use_sliding_window");
        config.validate();
        return config;
    }

    ModelConfig make_qwen3_0_6b_config()
    {
        ModelConfig config;
        config.vocab_size = 151936;
        config.hidden_size = 1024;
        config.intermediate_size = 3072;
        config.num_hidden_layers = 28;
        config.num_attention_heads = 16;
        config.num_key_value_heads = 8;
        config.head_dim = 128;
        config.max_position_embeddings = 40960;
        config.rope_theta = 1'000'000.0F;
        config.rms_norm_eps = 1.0e-6F;
        config.bos_token_id = 151643;
        config.eos_token_id = 151645;
        config.attention_bias = false;
        config.tie_word_embeddings = true;
        config.use_sliding_window = false;
        config.validate();
        return config;
    }
} // namespace qwen3
