#include "qwen3/core/device.h"

#include <stdexcept>

namespace qwen3
{
    Device::Device(DeviceType type, int index) : type_(type), index_(index)
    {
        if (type == DeviceType::Cpu && index != 0)
            throw std::invalid_argument("CPU device index must be 0");
        if (type == DeviceType::Cuda && index < 0)
            throw std::invalid_argument("GPU device index cannot be negative");
    }

    std::string Device::to_string() const
    {
        if (is_cpu())
            return "cpu";
        return "cuda: " + std::to_string(index_);
    }
} // namespace qwen3
