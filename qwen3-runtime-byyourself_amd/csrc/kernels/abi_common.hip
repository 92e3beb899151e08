// Error slot, version string and the host-side RoPE table builder of the
// C ABI (q3k_abi.h).
#include "q3k_common.hpp"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <vector>

namespace q3k
{
    namespace
    {
        thread_local char g_last_error[512] = "no error";
    }

    int set_error(int status, const char *fmt, ...)
    {
        va_list args;
        va_start(args, fmt);
        std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
        va_end(args);
        return status;
    }

    int check_launch(const char *kernel_name)
    {
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess)
        {
            return set_error(Q3K_ERR_HIP, "HIP launch of %s failed: %s: %s", kernel_name,
                             hipGetErrorName(err), hipGetErrorString(err));
        }
        return Q3K_OK;
    }
} // namespace q3k

extern "C" const char *q3k_last_error_string(void)
{
    return q3k::g_last_error;
}

extern "C" const char *q3k_version(void)
{
    return "0.1.0";
}

// Same recipe as src/ops/rope.cu:267-296: one double inverse frequency per
// pair, the angle position * inv_freq in double, cos/sin in double, then a
// single rounding to float.
extern "C" int q3k_build_rope_cache_f32(float *host_cache, int64_t P, int32_t D, float theta)
{
    using namespace q3k;
    if (P <= 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE max_positions must be positive");
    if (D <= 0 || D % 2 != 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE head_dim must be a positive even number");
    if (!std::isfinite(theta) || theta <= 0.0f)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE theta must be finite and positive");
    if (host_cache == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RoPE cache output pointer is null");
    const int64_t half = D / 2;
    if (P > INT64_MAX / D)
        return set_error(Q3K_ERR_OVERFLOW, "RoPE cache size overflows");

    std::vector<double> inv_freq(static_cast<size_t>(half));
    for (int64_t i = 0; i < half; ++i)
    {
        const double exponent = (2.0 * static_cast<double>(i)) / static_cast<double>(D);
        inv_freq[static_cast<size_t>(i)] = std::pow(static_cast<double>(theta), -exponent);
    }
    for (int64_t p = 0; p < P; ++p)
    {
        float *row = host_cache + p * D;
        for (int64_t i = 0; i < half; ++i)
        {
            const double angle = static_cast<double>(p) * inv_freq[static_cast<size_t>(i)];
            row[2 * i] = static_cast<float>(std::cos(angle));
            row[2 * i + 1] = static_cast<float>(std::sin(angle));
        }
    }
    return Q3K_OK;
}
