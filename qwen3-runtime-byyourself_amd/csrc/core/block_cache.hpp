// Internal control of the small-block device cache behind qwen3::Buffer.
#pragma once

namespace qwen3::detail
{
    // While an instance lives, device Buffers made on this thread get fresh
    // device memory instead of a block kept for reuse.  For writers on a
    // stream other than the default one (the weight upload): a reused block
    // may still be read by work queued on the default stream, and a fresh
    // one cannot be.
    class FreshDeviceBlocks
    {
    public:
        FreshDeviceBlocks() noexcept;
        ~FreshDeviceBlocks();
        FreshDeviceBlocks(const FreshDeviceBlocks &) = delete;
        FreshDeviceBlocks &operator=(const FreshDeviceBlocks &) = delete;
    };
} // namespace qwen3::detail
