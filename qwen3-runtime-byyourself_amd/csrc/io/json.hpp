// A small JSON reader for safetensors headers and checkpoint indexes
// (RFC 8259 values; numbers keep their text, and whether they are an
// unsigned integer that fits 64 bits).  Throws std::runtime_error with the
// byte offset on malformed input.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace qwen3::json
{
    struct Value
    {
        enum class Kind
        {
            Null,
            Bool,
            Number,
            String,
            Array,
            Object
        };
        Kind kind = Kind::Null;
        bool boolean = false;
        std::string text;             // string value, or the number's text
        bool is_unsigned = false;     // number: a non-negative integer below 2^64
        std::uint64_t unsigned_value = 0;
        std::vector<Value> items;                            // array
        std::vector<std::pair<std::string, Value>> members;  // object, in file order

        [[nodiscard]] const Value *find(const std::string &key) const
        {
            for (const auto &m : members)
                if (m.first == key)
                    return &m.second;
            return nullptr;
        }
    };

    class Parser
    {
    public:
        explicit Parser(const std::string &text) : s_(text) {}

        Value parse()
        {
            skip_ws();
            Value v = value(0);
            skip_ws();
            if (i_ != s_.size())
                fail("trailing characters");
            return v;
        }

    private:
        [[noreturn]] void fail(const char *what) const
        {
            throw std::runtime_error(std::string("JSON ") + what + " at byte " + std::to_string(i_));
        }
        void skip_ws()
        {
            while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r'))
                ++i_;
        }
        char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
        void expect(char c)
        {
            if (peek() != c)
                fail("unexpected character");
            ++i_;
        }
        void literal(const char *word)
        {
            for (const char *p = word; *p; ++p)
                expect(*p);
        }

        Value value(int depth)
        {
            if (depth > 64)
                fail("nesting too deep");
            Value v;
            switch (peek())
            {
            case '{': v = object(depth); break;
            case '[': v = array(depth); break;
            case '"':
                v.kind = Value::Kind::String;
                v.text = string();
                break;
            case 't':
                literal("true");
                v.kind = Value::Kind::Bool;
                v.boolean = true;
                break;
            case 'f':
                literal("false");
                v.kind = Value::Kind::Bool;
                break;
            case 'n': literal("null"); break;
            default: v = number(); break;
            }
            return v;
        }

        Value object(int depth)
        {
            Value v;
            v.kind = Value::Kind::Object;
            expect('{');
            skip_ws();
            if (peek() == '}')
            {
                ++i_;
                return v;
            }
            for (;;)
            {
                skip_ws();
                std::string key = string();
                skip_ws();
                expect(':');
                skip_ws();
                v.members.emplace_back(std::move(key), value(depth + 1));
                skip_ws();
                if (peek() == ',')
                {
                    ++i_;
                    continue;
                }
                expect('}');
                return v;
            }
        }

        Value array(int depth)
        {
            Value v;
            v.kind = Value::Kind::Array;
            expect('[');
            skip_ws();
            if (peek() == ']')
            {
                ++i_;
                return v;
            }
            for (;;)
            {
                skip_ws();
                v.items.push_back(value(depth + 1));
                skip_ws();
                if (peek() == ',')
                {
                    ++i_;
                    continue;
                }
                expect(']');
                return v;
            }
        }

        static void put_utf8(std::string &out, std::uint32_t cp)
        {
            if (cp < 0x80)
                out += static_cast<char>(cp);
            else if (cp < 0x800)
            {
                out += static_cast<char>(0xC0 | (cp >> 6));
                out += static_cast<char>(0x80 | (cp & 0x3F));
            }
            else if (cp < 0x10000)
            {
                out += static_cast<char>(0xE0 | (cp >> 12));
                out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
                out += static_cast<char>(0x80 | (cp & 0x3F));
            }
            else
            {
                out += static_cast<char>(0xF0 | (cp >> 18));
                out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
                out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
                out += static_cast<char>(0x80 | (cp & 0x3F));
            }
        }

        std::uint32_t hex4()
        {
            std::uint32_t cp = 0;
            for (int k = 0; k < 4; ++k)
            {
                const char c = peek();
                ++i_;
                cp <<= 4;
                if (c >= '0' && c <= '9')
                    cp |= static_cast<std::uint32_t>(c - '0');
                else if (c >= 'a' && c <= 'f')
                    cp |= static_cast<std::uint32_t>(c - 'a' + 10);
                else if (c >= 'A' && c <= 'F')
                    cp |= static_cast<std::uint32_t>(c - 'A' + 10);
                else
                    fail("bad \\u escape");
            }
            return cp;
        }

        std::string string()
        {
            expect('"');
            std::string out;
            for (;;)
            {
                if (i_ >= s_.size())
                    fail("unterminated string");
                const char c = s_[i_++];
                if (c == '"')
                    return out;
                if (static_cast<unsigned char>(c) < 0x20)
                    fail("control character in string");
                if (c != '\\')
                {
                    out += c;
                    continue;
                }
                const char e = peek();
                ++i_;
                switch (e)
                {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u':
                {
                    std::uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00)
                    {
                        expect('\\');
                        expect('u');
                        const std::uint32_t low = hex4();
                        if (low < 0xDC00 || low >= 0xE000)
                            fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (low - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail("bad escape");
                }
            }
        }

        Value number()
        {
            Value v;
            v.kind = Value::Kind::Number;
            const std::size_t begin = i_;
            if (peek() == '-')
                ++i_;
            if (peek() == '0')
                ++i_;
            else if (peek() >= '1' && peek() <= '9')
                while (peek() >= '0' && peek() <= '9')
                    ++i_;
            else
                fail("unexpected character");
            bool integer = true;
            if (peek() == '.')
            {
                integer = false;
                ++i_;
                if (!(peek() >= '0' && peek() <= '9'))
                    fail("bad number");
                while (peek() >= '0' && peek() <= '9')
                    ++i_;
            }
            if (peek() == 'e' || peek() == 'E')
            {
                integer = false;
                ++i_;
                if (peek() == '+' || peek() == '-')
                    ++i_;
                if (!(peek() >= '0' && peek() <= '9'))
                    fail("bad number");
                while (peek() >= '0' && peek() <= '9')
                    ++i_;
            }
            v.text = s_.substr(begin, i_ - begin);
            if (integer && v.text[0] != '-')
            {
                std::uint64_t acc = 0;
                bool fits = true;
                for (const char c : v.text)
                {
                    const std::uint64_t d = static_cast<std::uint64_t>(c - '0');
                    if (acc > (UINT64_MAX - d) / 10)
                    {
                        fits = false;
                        break;
                    }
                    acc = acc * 10 + d;
                }
                v.is_unsigned = fits;
                v.unsigned_value = acc;
            }
            return v;
        }

        const std::string &s_;
        std::size_t i_ = 0;
    };

    inline Value parse(const std::string &text) { return Parser(text).parse(); }
} // namespace qwen3::json
