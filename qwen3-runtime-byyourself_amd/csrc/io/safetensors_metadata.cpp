// Tensor records of a safetensors header (checks and messages of the
// reference's src/io/safetensors_metadata.cpp; a repeated key keeps its last
// value, as a JSON object does).
#include "qwen3/io/safetensors_metadata.h"

#include "json.hpp"

#include <limits>
#include <vector>

namespace qwen3
{
    namespace
    {
        [[noreturn]] void tensor_error(const std::string &name, const std::string &message)
        {
            throw SafetensorsFormatError("tensor '" + name + "': " + message);
        }

        DType parse_dtype(const json::Value &v, const std::string &name)
        {
            if (v.kind != json::Value::Kind::String)
                tensor_error(name, "'dtype' must be a string");
            if (v.text == "BF16")
                return DType::BFloat16;
            if (v.text == "F32")
                return DType::Float32;
            if (v.text == "I32")
                return DType::Int32;
            tensor_error(name, "unsupported dtype '" + v.text + "'");
        }

        std::size_t parse_size(const json::Value &v, const std::string &name, const std::string &field)
        {
            if (v.kind != json::Value::Kind::Number || !v.is_unsigned)
                tensor_error(name, "'" + field + "' must contain unsigned integers");
            if (v.unsigned_value > static_cast<std::uint64_t>(std::numeric_limits<std::size_t>::max()))
                tensor_error(name, "'" + field + "' contains a value too large for size_t");
            return static_cast<std::size_t>(v.unsigned_value);
        }
    } // namespace

    SafetensorsMetadata::SafetensorsMetadata(const SafetensorsFile &file)
    {
        const ConstByteView header = file.header_bytes();
        const std::size_t data_size = file.data_bytes().size_bytes();
        json::Value root;
        try
        {
            root = json::parse(std::string(reinterpret_cast<const char *>(header.data()), header.size_bytes()));
        }
        catch (const std::runtime_error &e)
        {
            throw SafetensorsFormatError(std::string("invalid Safetensors JSON header: ") + e.what());
        }
        if (root.kind != json::Value::Kind::Object)
            throw SafetensorsFormatError("Safetensors header must be a JSON object");
        for (const auto &member : root.members)
        {
            const std::string &name = member.first;
            if (name == "__metadata__")
                continue;
            const json::Value &record = member.second;
            if (record.kind != json::Value::Kind::Object)
                tensor_error(name, "metadata must be a JSON object");
            const json::Value *dtype_v = record.find("dtype");
            const json::Value *shape_v = record.find("shape");
            const json::Value *offsets_v = record.find("data_offsets");
            if (dtype_v == nullptr || shape_v == nullptr || offsets_v == nullptr)
                tensor_error(name, "missing dtype, shape or data_offsets");
            const DType dtype = parse_dtype(*dtype_v, name);
            if (shape_v->kind != json::Value::Kind::Array)
                tensor_error(name, "'shape' must be an array");
            std::vector<Shape::Dimension> dims;
            dims.reserve(shape_v->items.size());
            for (const json::Value &d : shape_v->items)
            {
                const std::size_t n = parse_size(d, name, "shape");
                if (n > static_cast<std::size_t>(std::numeric_limits<Shape::Dimension>::max()))
                    tensor_error(name, "'shape' contains a value too large for a dimension");
                dims.push_back(static_cast<Shape::Dimension>(n));
            }
            Shape shape{std::move(dims)};
            if (offsets_v->kind != json::Value::Kind::Array || offsets_v->items.size() != 2)
                tensor_error(name, "'data_offsets' must contain exactly two integers");
            const std::size_t begin = parse_size(offsets_v->items[0], name, "data_offsets");
            const std::size_t end = parse_size(offsets_v->items[1], name, "data_offsets");
            if (end < begin)
                tensor_error(name, "end offset is smaller than begin offset");
            if (end > data_size)
                tensor_error(name, "data offset exceeds the weight data buffer");
            std::size_t numel = 0;
            try
            {
                numel = static_cast<std::size_t>(shape.numel());
            }
            catch (const std::overflow_error &)
            {
                tensor_error(name, "shape element count overflow");
            }
            const std::size_t element = dtype_size(dtype);
            if (numel != 0 && element > std::numeric_limits<std::size_t>::max() / numel)
                tensor_error(name, "tensor byte size overflow");
            if (numel * element != end - begin)
                tensor_error(name, "shape and data_offsets describe different byte sizes");
            tensors_.insert_or_assign(name, SafetensorsTensorInfo{dtype, std::move(shape), begin, end});
        }
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
