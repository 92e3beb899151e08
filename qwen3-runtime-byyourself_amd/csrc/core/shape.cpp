#include "qwen3/core/shape.h"

#include <limits>
#include <stdexcept>
#include <utility>

namespace qwen3
{
    Shape::Shape(std::initializer_list<Dimension> dimensions) : dimensions_(dimensions) { validate(); }

    Shape::Shape(std::vector<Dimension> dimensions) : dimensions_(std::move(dimensions)) { validate(); }

    void Shape::validate() const
    {
        for (const Dimension d : dimensions_)
        {
            if (d < 0)
                throw std::invalid_argument("Shape dimensions cannot be negative");
        }
    }

    Shape::Dimension Shape::operator[](std::size_t axis) const
    {
        if (axis >= dimensions_.size())
            throw std::out_of_range("Shape axis out of range");
        return dimensions_[axis];
    }

    Shape::Dimension Shape::numel() const
    {
        Dimension n = 1;
        for (const Dimension d : dimensions_)
        {
            if (d == 0)
                return 0;
        }
        for (const Dimension d : dimensions_)
        {
            if (n > std::numeric_limits<Dimension>::max() / d)
                throw std::overflow_error("Shape element count overflows int64");
            n *= d;
        }
        return n;
    }

    bool Shape::has_zero_dimension() const noexcept
    {
        for (const Dimension d : dimensions_)
        {
            if (d == 0)
                return true;
        }
        return false;
    }

    std::string Shape::to_string() const
    {
        std::string s = "[";
        for (std::size_t i = 0; i < dimensions_.size(); ++i)
        {
            if (i)
                s += ", ";
            s += std::to_string(dimensions_[i]);
        }
        return s + "]";
    }
} // namespace qwen3
