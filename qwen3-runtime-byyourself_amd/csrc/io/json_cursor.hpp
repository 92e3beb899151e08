// A pull parser over RFC 8259 JSON text.  The caller walks the document
// value by value (open_object / next_key, open_array / next_item,
// read_string / read_number / skip_value), so a safetensors header or a
// checkpoint index is checked while it is read, without building a tree.
//
// Strings are returned as UTF-8 (escapes decoded, surrogate pairs joined;
// lone surrogates, raw control characters and ill-formed UTF-8 rejected).
// A number reports whether it is an unsigned integer that fits 64 bits: no
// sign, fraction or exponent ("-0", "1.0" and "1e3" are not), and carries
// its text for callers that need other readings of it.  Malformed
// input throws std::runtime_error("JSON <reason> at byte <offset>").
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace qwen3::io_detail
{
    class JsonCursor final
    {
    public:
        enum class Kind
        {
            Object,
            Array,
            String,
            Number,
            Bool,
            Null
        };

        struct Number
        {
            bool is_unsigned = false;  // a non-negative integer below 2^64
            std::uint64_t value = 0;   // valid when is_unsigned
            bool integral = false;     // no fraction and no exponent
            bool negative = false;     // a leading minus sign
            std::string_view text;     // the number as written (valid while the text is)
        };

        // A leading UTF-8 byte order mark (EF BB BF) is skipped, as nlohmann's
        // lexer does for every document the reference parses.
        explicit JsonCursor(std::string_view text) : text_(text)
        {
            if (text_.size() >= 3 && static_cast<unsigned char>(text_[0]) == 0xEF &&
                static_cast<unsigned char>(text_[1]) == 0xBB && static_cast<unsigned char>(text_[2]) == 0xBF)
                at_ = 3;
        }

        // Kind of the next value (whitespace skipped); throws at end of input
        // or on a character that cannot start a value.
        Kind peek_kind()
        {
            skip_ws();
            if (at_ >= text_.size())
                fail("value expected, end of input found");
            switch (text_[at_])
            {
            case '{': return Kind::Object;
            case '[': return Kind::Array;
            case '"': return Kind::String;
            case 't':
            case 'f': return Kind::Bool;
            case 'n': return Kind::Null;
            default:
                if (text_[at_] == '-' || (text_[at_] >= '0' && text_[at_] <= '9'))
                    return Kind::Number;
                fail("unexpected character");
            }
        }

        void open_object() { open('{'); }
        void open_array() { open('['); }

        // Moves to the next member of the innermost open object: true with
        // its key (the cursor then sits on the member's value), false after
        // consuming the closing brace.
        bool next_key(std::string &key)
        {
            if (!next_in('}'))
                return false;
            skip_ws();
            if (at_ >= text_.size() || text_[at_] != '"')
                fail("object key expected");
            key = read_string();
            skip_ws();
            expect(':');
            return true;
        }

        // Moves to the next item of the innermost open array: true when one
        // follows (not consumed), false after consuming the closing bracket.
        bool next_item() { return next_in(']'); }

        std::string read_string()
        {
            skip_ws();
            expect('"');
            std::string out;
            for (;;)
            {
                if (at_ >= text_.size())
                    fail("unterminated string");
                const auto c = static_cast<unsigned char>(text_[at_]);
                if (c == '"')
                {
                    ++at_;
                    return out;
                }
                if (c < 0x20)
                    fail("control character in string");
                if (c == '\\')
                {
                    ++at_;
                    escape(out);
                }
                else if (c < 0x80)
                {
                    out.push_back(static_cast<char>(c));
                    ++at_;
                }
                else
                {
                    utf8_sequence(out);
                }
            }
        }

        Number read_number()
        {
            skip_ws();
            const std::size_t start = at_;
            Number n;
            bool negative = false, integral = true, fits = true;
            std::uint64_t v = 0;
            if (peek() == '-')
            {
                negative = true;
                ++at_;
            }
            if (peek() == '0')
            {
                ++at_;
                if (is_digit(peek()))
                    fail("leading zero in number");
            }
            else if (is_digit(peek()))
            {
                while (is_digit(peek()))
                {
                    const std::uint64_t d = static_cast<std::uint64_t>(text_[at_] - '0');
                    if (v > (UINT64_MAX - d) / 10)
                        fits = false;
                    else
                        v = v * 10 + d;
                    ++at_;
                }
            }
            else
            {
                fail("digit expected");
            }
            if (peek() == '.')
            {
                integral = false;
                ++at_;
                digits("digit expected after decimal point");
            }
            if (peek() == 'e' || peek() == 'E')
            {
                integral = false;
                ++at_;
                if (peek() == '+' || peek() == '-')
                    ++at_;
                digits("digit expected in exponent");
            }
            n.is_unsigned = !negative && integral && fits;
            n.value = n.is_unsigned ? v : 0;
            n.integral = integral;
            n.negative = negative;
            n.text = text_.substr(start, at_ - start);
            return n;
        }

        bool read_bool()
        {
            skip_ws();
            if (peek() == 't')
            {
                word("true");
                return true;
            }
            word("false");
            return false;
        }

        void read_null()
        {
            skip_ws();
            word("null");
        }

        // Consumes the next value, whatever its kind, checking its syntax.
        void skip_value()
        {
            switch (peek_kind())
            {
            case Kind::Object:
            {
                open_object();
                std::string key;
                while (next_key(key))
                    skip_value();
                break;
            }
            case Kind::Array:
                open_array();
                while (next_item())
                    skip_value();
                break;
            case Kind::String: (void)read_string(); break;
            case Kind::Number: (void)read_number(); break;
            case Kind::Bool: (void)read_bool(); break;
            case Kind::Null: read_null(); break;
            }
        }

        // After the top-level value: only whitespace may follow.
        void finish()
        {
            skip_ws();
            if (at_ != text_.size())
                fail("trailing characters after the document");
        }

    private:
        static constexpr std::size_t kMaxDepth = 256;

        // Per open container: whether no member or item was read yet.
        std::string_view text_;
        std::size_t at_ = 0;
        std::vector<bool> first_;

        [[noreturn]] void fail(const char *reason) const
        {
            throw std::runtime_error(std::string("JSON ") + reason + " at byte " + std::to_string(at_));
        }

        static bool is_digit(char c) { return c >= '0' && c <= '9'; }
        char peek() const { return at_ < text_.size() ? text_[at_] : '\0'; }

        void skip_ws()
        {
            while (at_ < text_.size() &&
                   (text_[at_] == ' ' || text_[at_] == '\t' || text_[at_] == '\n' || text_[at_] == '\r'))
                ++at_;
        }

        void expect(char c)
        {
            if (peek() != c || at_ >= text_.size())
                fail(c == ':' ? "':' expected" : c == ',' ? "',' expected" : "unexpected character");
            ++at_;
        }

        void word(const char *w)
        {
            for (const char *p = w; *p != '\0'; ++p)
            {
                if (peek() != *p)
                    fail("invalid literal");
                ++at_;
            }
        }

        void digits(const char *reason)
        {
            if (!is_digit(peek()))
                fail(reason);
            while (is_digit(peek()))
                ++at_;
        }

        void open(char c)
        {
            skip_ws();
            expect(c);
            if (first_.size() >= kMaxDepth)
                fail("nesting too deep");
            first_.push_back(true);
        }

        // Shared comma / close logic of objects and arrays.
        bool next_in(char close)
        {
            if (first_.empty())
                fail("no open container");
            skip_ws();
            if (peek() == close && at_ < text_.size())
            {
                ++at_;
                first_.pop_back();
                return false;
            }
            if (!first_.back())
                expect(',');
            first_.back() = false;
            return true;
        }

        static void put_utf8(std::string &out, std::uint32_t cp)
        {
            if (cp < 0x80)
            {
                out.push_back(static_cast<char>(cp));
            }
            else if (cp < 0x800)
            {
                out.push_back(static_cast<char>(0xC0 | (cp >> 6)));
                out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            }
            else if (cp < 0x10000)
            {
                out.push_back(static_cast<char>(0xE0 | (cp >> 12)));
                out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
                out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            }
            else
            {
                out.push_back(static_cast<char>(0xF0 | (cp >> 18)));
                out.push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
                out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
                out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            }
        }

        std::uint32_t hex4()
        {
            std::uint32_t v = 0;
            for (int i = 0; i < 4; ++i)
            {
                const char c = peek();
                std::uint32_t d;
                if (c >= '0' && c <= '9')
                    d = static_cast<std::uint32_t>(c - '0');
                else if (c >= 'a' && c <= 'f')
                    d = static_cast<std::uint32_t>(c - 'a' + 10);
                else if (c >= 'A' && c <= 'F')
                    d = static_cast<std::uint32_t>(c - 'A' + 10);
                else
                    fail("invalid \\u escape");
                v = v * 16 + d;
                ++at_;
            }
            return v;
        }

        // After a backslash.
        void escape(std::string &out)
        {
            const char c = peek();
            ++at_;
            switch (c)
            {
            case '"': out.push_back('"'); return;
            case '\\': out.push_back('\\'); return;
            case '/': out.push_back('/'); return;
            case 'b': out.push_back('\b'); return;
            case 'f': out.push_back('\f'); return;
            case 'n': out.push_back('\n'); return;
            case 'r': out.push_back('\r'); return;
            case 't': out.push_back('\t'); return;
            case 'u': break;
            default: --at_; fail("invalid escape");
            }
            std::uint32_t cp = hex4();
            if (cp >= 0xDC00 && cp <= 0xDFFF)
                fail("unpaired low surrogate");
            if (cp >= 0xD800 && cp <= 0xDBFF)
            {
                if (peek() != '\\' || at_ + 1 >= text_.size() || text_[at_ + 1] != 'u')
                    fail("high surrogate without a low surrogate");
                at_ += 2;
                const std::uint32_t lo = hex4();
                if (lo < 0xDC00 || lo > 0xDFFF)
                    fail("high surrogate without a low surrogate");
                cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            }
            put_utf8(out, cp);
        }

        // One multi-byte UTF-8 sequence (RFC 3629: shortest form, no
        // surrogates, at most U+10FFFF), copied unchanged.
        void utf8_sequence(std::string &out)
        {
            const auto b0 = static_cast<unsigned char>(text_[at_]);
            int extra;
            std::uint32_t cp, min;
            if ((b0 & 0xE0) == 0xC0)
            {
                extra = 1;
                cp = b0 & 0x1F;
                min = 0x80;
            }
            else if ((b0 & 0xF0) == 0xE0)
            {
                extra = 2;
                cp = b0 & 0x0F;
                min = 0x800;
            }
            else if ((b0 & 0xF8) == 0xF0)
            {
                extra = 3;
                cp = b0 & 0x07;
                min = 0x10000;
            }
            else
            {
                fail("ill-formed UTF-8");
            }
            if (at_ + static_cast<std::size_t>(extra) >= text_.size())
                fail("ill-formed UTF-8");
            for (int i = 1; i <= extra; ++i)
            {
                const auto b = static_cast<unsigned char>(text_[at_ + static_cast<std::size_t>(i)]);
                if ((b & 0xC0) != 0x80)
                    fail("ill-formed UTF-8");
                cp = (cp << 6) | (b & 0x3F);
            }
            if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
                fail("ill-formed UTF-8");
            out.append(text_.substr(at_, static_cast<std::size_t>(extra) + 1));
            at_ += static_cast<std::size_t>(extra) + 1;
        }
    };
} // namespace qwen3::io_detail
