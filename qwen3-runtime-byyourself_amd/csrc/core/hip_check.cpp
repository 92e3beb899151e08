#include "qwen3/hip/hip_check.h"

#include <sstream>
#include <stdexcept>

namespace qwen3::hip
{
    void check(hipError_t status, const char *expression, const char *file, int line)
    {
        if (status == hipSuccess)
            return;
        std::ostringstream message;
        message << "HIP call failed: " << expression << '\n'
                << hipGetErrorName(status) << ": " << hipGetErrorString(status) << '\n'
                << "at " << file << ':' << line;
        throw std::runtime_error(message.str());
    }

    DeviceGuard::DeviceGuard(int device) : previous_(0), changed_(false)
    {
        QWEN3_HIP_CHECK(hipGetDevice(&previous_));
        if (previous_ != device)
        {
            QWEN3_HIP_CHECK(hipSetDevice(device));
            changed_ = true;
        }
    }

    DeviceGuard::~DeviceGuard()
    {
        if (changed_)
            static_cast<void>(hipSetDevice(previous_));
    }

    void DeviceGuard::restore()
    {
        if (changed_)
        {
            changed_ = false;
            QWEN3_HIP_CHECK(hipSetDevice(previous_));
        }
    }
} // namespace qwen3::hip
