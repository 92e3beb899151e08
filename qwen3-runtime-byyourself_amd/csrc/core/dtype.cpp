#include "qwen3/core/dtype.h"

#include <stdexcept>

namespace qwen3
{
    std::size_t dtype_size(DType dtype)
    {
        switch (dtype)
        {
        case DType::Float32: return 4;
        case DType::BFloat16: return 2;
        case DType::Int32: return 4;
        }
        throw std::invalid_argument("unknown dtype");
    }

    std::string_view dtype_name(DType dtype)
    {
        switch (dtype)
        {
        case DType::Float32: return "float32";
        case DType::BFloat16: return "bfloat16";
        case DType::Int32: return "int32";
        }
        throw std::invalid_argument("unknown dtype");
    }
} // namespace qwen3
