// Tensor table of a safetensors header, built in one pass of a pull parser
// over the header bytes.  Each tensor record is captured field by field as
// it is read ("draft"), then judged against an ordered rule list; the
// verdicts are kept by name (a repeated name keeps its last record, as a
// JSON object does) and, once the whole header has parsed, the first failing
// record in name order raises its error, as a header parsed into a sorted
// JSON object and then checked would (src/io/safetensors_metadata.cpp:
// 64-178 of the reference).  The rules, their order and messages are that
// file's contract; the exception type is SafetensorsFormatError throughout.
#include "qwen3/io/safetensors_metadata.h"

#include "json_cursor.hpp"

#include <limits>
#include <map>
#include <optional>
#include <vector>

namespace qwen3
{
    namespace
    {
        using io_detail::JsonCursor;

        // How a field of a record looked in the header.
        enum class Seen
        {
            Absent,
            WrongKind,  // present but not the JSON kind the rule wants
            Present,
        };

        // One array of numbers (shape, data_offsets): its items as read.
        struct NumberList
        {
            Seen seen = Seen::Absent;
            std::vector<std::optional<JsonCursor::Number>> items;  // nullopt: an item that is not a number
        };

        // Everything a record said, before any rule is applied.
        struct Draft
        {
            bool is_object = false;
            Seen dtype_seen = Seen::Absent;
            std::string dtype;
            NumberList shape;
            NumberList offsets;
        };

        // A draft under judgement: the rules fill these in as they pass.
        struct Judgement
        {
            const Draft &draft;
            std::size_t data_size;
            DType dtype = DType::BFloat16;
            std::vector<Shape::Dimension> dims;
            std::size_t begin = 0;
            std::size_t end = 0;
            std::size_t numel = 0;
        };

        using Rule = std::optional<std::string> (*)(Judgement &);

        std::optional<std::string> unsigned_items(const NumberList &list, const char *field, std::vector<std::uint64_t> &out)
        {
            for (const auto &item : list.items)
            {
                if (!item || !item->is_unsigned)
                    return "'" + std::string(field) + "' must contain unsigned integers";
                if (item->value > static_cast<std::uint64_t>(std::numeric_limits<std::size_t>::max()))
                    return "'" + std::string(field) + "' contains a value too large for size_t";
                out.push_back(item->value);
            }
            return std::nullopt;
        }

        // The checks of a record, in the order they are applied.
        const Rule kRules[] = {
            [](Judgement &j) -> std::optional<std::string> {
                if (!j.draft.is_object)
                    return "metadata must be a JSON object";
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                const Draft &d = j.draft;
                if (d.dtype_seen == Seen::Absent || d.shape.seen == Seen::Absent || d.offsets.seen == Seen::Absent)
                    return "missing dtype, shape or data_offsets";
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                if (j.draft.dtype_seen != Seen::Present)
                    return "'dtype' must be a string";
                const std::string &n = j.draft.dtype;
                if (n == "BF16")
                    j.dtype = DType::BFloat16;
                else if (n == "F32")
                    j.dtype = DType::Float32;
                else if (n == "I32")
                    j.dtype = DType::Int32;
                else
                    return "unsupported dtype '" + n + "'";
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                if (j.draft.shape.seen != Seen::Present)
                    return "'shape' must be an array";
                std::vector<std::uint64_t> v;
                if (auto e = unsigned_items(j.draft.shape, "shape", v))
                    return e;
                for (const std::uint64_t d : v)
                {
                    if (d > static_cast<std::uint64_t>(std::numeric_limits<Shape::Dimension>::max()))
                        return "'shape' contains a value too large for a dimension";
                    j.dims.push_back(static_cast<Shape::Dimension>(d));
                }
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                if (j.draft.offsets.seen != Seen::Present || j.draft.offsets.items.size() != 2)
                    return "'data_offsets' must contain exactly two integers";
                std::vector<std::uint64_t> v;
                if (auto e = unsigned_items(j.draft.offsets, "data_offsets", v))
                    return e;
                j.begin = static_cast<std::size_t>(v[0]);
                j.end = static_cast<std::size_t>(v[1]);
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                if (j.end < j.begin)
                    return "end offset is smaller than begin offset";
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                if (j.end > j.data_size)
                    return "data offset exceeds the weight data buffer";
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                try
                {
                    j.numel = static_cast<std::size_t>(Shape{j.dims}.numel());
                }
                catch (const std::overflow_error &)
                {
                    return "shape element count overflow";
                }
                return std::nullopt;
            },
            [](Judgement &j) -> std::optional<std::string> {
                const std::size_t element = dtype_size(j.dtype);
                if (j.numel != 0 && element > std::numeric_limits<std::size_t>::max() / j.numel)
                    return "tensor byte size overflow";
                if (j.numel * element != j.end - j.begin)
                    return "shape and data_offsets describe different byte sizes";
                return std::nullopt;
            },
        };

        // Reads an array of numbers into `list` (the cursor sits on it).
        void read_numbers(JsonCursor &cur, NumberList &list)
        {
            list.items.clear();
            if (cur.peek_kind() != JsonCursor::Kind::Array)
            {
                list.seen = Seen::WrongKind;
                cur.skip_value();
                return;
            }
            list.seen = Seen::Present;
            cur.open_array();
            while (cur.next_item())
            {
                if (cur.peek_kind() == JsonCursor::Kind::Number)
                {
                    list.items.emplace_back(cur.read_number());
                }
                else
                {
                    list.items.emplace_back(std::nullopt);
                    cur.skip_value();
                }
            }
        }

        // Reads one record (the cursor sits on its value).  Fields other than
        // dtype, shape and data_offsets are skipped; a repeated field keeps
        // its last value.
        Draft read_draft(JsonCursor &cur)
        {
            Draft d;
            if (cur.peek_kind() != JsonCursor::Kind::Object)
            {
                cur.skip_value();
                return d;
            }
            d.is_object = true;
            cur.open_object();
            std::string field;
            while (cur.next_key(field))
            {
                if (field == "dtype")
                {
                    if (cur.peek_kind() == JsonCursor::Kind::String)
                    {
                        d.dtype_seen = Seen::Present;
                        d.dtype = cur.read_string();
                    }
                    else
                    {
                        d.dtype_seen = Seen::WrongKind;
                        cur.skip_value();
                    }
                }
                else if (field == "shape")
                {
                    read_numbers(cur, d.shape);
                }
                else if (field == "data_offsets")
                {
                    read_numbers(cur, d.offsets);
                }
                else
                {
                    cur.skip_value();
                }
            }
            return d;
        }

        // The outcome for one tensor name: its record, or the first rule it broke.
        struct Verdict
        {
            std::optional<SafetensorsTensorInfo> info;
            std::string error;
        };

        Verdict judge(const Draft &draft, std::size_t data_size)
        {
            Judgement j{draft, data_size};
            for (const Rule rule : kRules)
                if (auto e = rule(j))
                    return Verdict{std::nullopt, std::move(*e)};
            return Verdict{SafetensorsTensorInfo{j.dtype, Shape{std::move(j.dims)}, j.begin, j.end}, {}};
        }
    } // namespace

    SafetensorsMetadata::SafetensorsMetadata(const SafetensorsFile &file)
    {
        const ConstByteView header = file.header_bytes();
        const std::size_t data_size = file.data_bytes().size_bytes();
        // name order, last record of a repeated name (what a JSON object keeps)
        std::map<std::string, Verdict> verdicts;
        try
        {
            JsonCursor cur(std::string_view(reinterpret_cast<const char *>(header.data()), header.size_bytes()));
            if (cur.peek_kind() != JsonCursor::Kind::Object)
            {
                cur.skip_value();
                cur.finish();
                throw SafetensorsFormatError("Safetensors header must be a JSON object");
            }
            cur.open_object();
            std::string name;
            while (cur.next_key(name))
            {
                if (name == "__metadata__")
                {
                    cur.skip_value();  // creator information, not a tensor
                    continue;
                }
                verdicts.insert_or_assign(name, judge(read_draft(cur), data_size));
            }
            cur.finish();
        }
        catch (const SafetensorsFormatError &)
        {
            throw;
        }
        catch (const std::runtime_error &e)
        {
            throw SafetensorsFormatError(std::string("invalid Safetensor JSON header: ") + e.what());
        }
        for (const auto &[name, verdict] : verdicts)
            if (!verdict.info)
                throw SafetensorsFormatError("tensor '" + name + "': " + verdict.error);
        tensors_.reserve(verdicts.size());
        for (auto &[name, verdict] : verdicts)
            tensors_.emplace(name, std::move(*verdict.info));
    }

    bool SafetensorsMetadata::contains(std::string_view name) const { return tensors_.count(std::string(name)) != 0; }

    const SafetensorsTensorInfo &SafetensorsMetadata::tensor(std::string_view name) const
    {
        const auto it = tensors_.find(std::string(name));
        if (it == tensors_.end())
            throw std::out_of_range("Safetensors tensor not found: " + std::string(name));
        return it->second;
    }
} // namespace qwen3
