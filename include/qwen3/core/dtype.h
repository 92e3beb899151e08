#pragma once

// Element types of the runtime's tensors.  Contract pinned by the reference's
// tests/unit/core_metadata_test.cpp:41-54 (its src/core is absent from the
// snapshot): dtype_size 4/2/4, dtype_name "float32"/"bfloat16"/"int32".

#include <cstddef>
#include <string_view>

namespace qwen3
{
    enum class DType
    {
        Float32,
        BFloat16,
        Int32,
    };

    [[nodiscard]] std::size_t dtype_size(DType dtype);

    [[nodiscard]] std::string_view dtype_name(DType dtype);
} // namespace qwen3
