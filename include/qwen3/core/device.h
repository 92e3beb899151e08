#pragma once

// Where a tensor lives.  DeviceType::Cuda / Device::cuda(i) / is_cuda() keep
// the reference's names (tests/unit/core_metadata_test.cpp:56-83) because the
// runtime's callers use them; on this build the device is a HIP GPU.

#include <string>

namespace qwen3
{
    enum class DeviceType
    {
        Cpu,
        Cuda,
    };

    class Device
    {
    public:
        // Throws std::invalid_argument for a negative GPU index or a non-zero CPU index.
        Device(DeviceType type, int index);

        [[nodiscard]] static Device cpu() { return Device{DeviceType::Cpu, 0}; }
        [[nodiscard]] static Device cuda(int index) { return Device{DeviceType::Cuda, index}; }

        [[nodiscard]] DeviceType type() const noexcept { return type_; }
        [[nodiscard]] int index() const noexcept { return index_; }
        [[nodiscard]] bool is_cpu() const noexcept { return type_ == DeviceType::Cpu; }
        [[nodiscard]] bool is_cuda() const noexcept { return type_ == DeviceType::Cuda; }

        // "cpu" or "cuda: <index>"
        [[nodiscard]] std::string to_string() const;

        friend bool operator==(const Device &a, const Device &b) noexcept
        {
            return a.type_ == b.type_ && a.index_ == b.index_;
        }
        friend bool operator!=(const Device &a, const Device &b) noexcept { return !(a == b); }

    private:
        DeviceType type_;
        int index_;
    };
} // namespace qwen3
