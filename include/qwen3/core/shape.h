#pragma once

// Tensor dimensions.  Contract pinned by tests/unit/core_metadata_test.cpp:85-135
// of the reference: negative dimensions throw std::invalid_argument, numel()
// throws std::overflow_error, Shape{} is a rank-0 scalar with one element.

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <string>
#include <vector>

namespace qwen3
{
    class Shape
    {
    public:
        using Dimension = std::int64_t;

        Shape() = default;
        Shape(std::initializer_list<Dimension> dimensions);
        explicit Shape(std::vector<Dimension> dimensions);

        [[nodiscard]] std::size_t rank() const noexcept { return dimensions_.size(); }
        // Throws std::out_of_range for axis >= rank().
        [[nodiscard]] Dimension operator[](std::size_t axis) const;
        [[nodiscard]] Dimension numel() const;
        [[nodiscard]] bool is_scalar() const noexcept { return dimensions_.empty(); }
        [[nodiscard]] bool has_zero_dimension() const noexcept;
        [[nodiscard]] const std::vector<Dimension> &dimensions() const noexcept { return dimensions_; }
        // "[2, 8, 1024]"
        [[nodiscard]] std::string to_string() const;

        friend bool operator==(const Shape &a, const Shape &b) noexcept { return a.dimensions_ == b.dimensions_; }
        friend bool operator!=(const Shape &a, const Shape &b) noexcept { return !(a == b); }

    private:
        void validate() const;

        std::vector<Dimension> dimensions_;
    };
} // namespace qwen3
