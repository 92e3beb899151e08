// Argmax over the last dimension for gfx950 (src/ops/argmax.cu:28-100 of the
// reference: bf16 rows, NaN counts as -inf, ties go to the smaller index,
// int32 indices).
//
// Every candidate becomes one 64-bit key: the bf16 bits mapped to an
// order-preserving unsigned value (NaN -> -inf, -0 -> +0, since the
// reference's float compare treats them as equal) in the high word and
// ~index in the low word, so "larger value, then smaller index" is a plain
// unsigned max.  One block of 1024 threads per row (rows strided over the
// grid): 128-bit loads when the row allows, wave max by lane shuffles, block
// max through LDS.  When there are too few rows to fill the GPU and the
// caller gives a workspace, each row is cut into slices of whole 8-column
// vectors: one block per (row, slice) writes the slice's best key, and a
// second kernel takes the maximum over the slices of each row (the key
// order is total, so the result is the same).
#include "q3k_common.hpp"

#include <mutex>

namespace q3k
{
    namespace
    {
        constexpr int kArgmaxBlock = 1024;

        __device__ __forceinline__ uint64_t argmax_key(uint32_t b, uint32_t index)
        {
            if ((b & 0x7fffu) > 0x7f80u)
                b = 0xff80u; // NaN -> -inf
            if (b == 0x8000u)
                b = 0u; // -0 -> +0
            const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
            return (static_cast<uint64_t>(ord) << 32) | (0xffffffffu - index);
        }

        __device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

        // This thread's best key over columns [begin, end) of row r; with
        // VEC, r is 16-byte aligned and begin a multiple of 8.
        template <bool VEC>
        __device__ __forceinline__ uint64_t thread_best(const uint16_t *r, int64_t begin, int64_t end)
        {
            uint64_t best = 0; // below every candidate
            int64_t tail = begin;
            if constexpr (VEC)
            {
                const int64_t v_end = end / 8;
                const Vec8 *rv = reinterpret_cast<const Vec8 *>(r);
                // groups of four 16-byte loads per thread, the last group
                // partial, all issued before any is used
                constexpr int U = 4;
                for (int64_t i = begin / 8 + threadIdx.x; i < v_end; i += U * kArgmaxBlock)
                {
                    Vec8 v[U];
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        if (i + u * kArgmaxBlock < v_end)
                            v[u] = rv[i + u * kArgmaxBlock];
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        if (i + u * kArgmaxBlock < v_end)
                        {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                            {
                                const uint32_t idx = static_cast<uint32_t>(8 * (i + u * kArgmaxBlock) + 2 * j);
                                best = max_u64(best, argmax_key(v[u].d[j] & 0xffffu, idx));
                                best = max_u64(best, argmax_key(v[u].d[j] >> 16, idx + 1));
                            }
                        }
                }
                tail = v_end * 8 > begin ? v_end * 8 : begin;
            }
            for (int64_t c = tail + threadIdx.x; c < end; c += kArgmaxBlock)
                best = max_u64(best, argmax_key(r[c], static_cast<uint32_t>(c)));
            return best;
        }

        // Block maximum of the threads' keys, valid in thread 0; wave_best is
        // free again when the call returns.
        __device__ __forceinline__ uint64_t block_best(uint64_t best, uint64_t *wave_best)
        {
            const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
            for (int off = 32; off > 0; off /= 2)
                best = max_u64(best, __shfl_xor(best, off, kWave));
            if (lane == 0)
                wave_best[wave] = best;
            __syncthreads();
            if (wave == 0)
            {
                best = lane < kArgmaxBlock / kWave ? wave_best[lane] : 0;
#pragma unroll
                for (int off = 8; off > 0; off /= 2)
                    best = max_u64(best, __shfl_xor(best, off, kWave));
            }
            __syncthreads();
            return best;
        }

        __device__ __forceinline__ int32_t key_index(uint64_t key)
        {
            return static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(key));
        }

        template <bool VEC>
        __global__ __launch_bounds__(kArgmaxBlock) void argmax_kernel(const uint16_t *__restrict__ x,
                                                                      int32_t *__restrict__ out, int64_t rows,
                                                                      int64_t stride, int64_t n)
        {
            __shared__ uint64_t wave_best[kArgmaxBlock / kWave];
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                const uint64_t best = block_best(thread_best<VEC>(x + row * stride, 0, n), wave_best);
                if (threadIdx.x == 0)
                    out[row] = key_index(best);
            }
        }

        // One block per (row, slice): part[row * slices + slice] = the best
        // key of columns [slice * slice_len, min(n, (slice + 1) * slice_len)).
        template <bool VEC>
        __global__ __launch_bounds__(kArgmaxBlock) void argmax_slice_kernel(const uint16_t *__restrict__ x,
                                                                            uint64_t *__restrict__ part,
                                                                            int64_t stride, int64_t n,
                                                                            int32_t slices, int64_t slice_len)
        {
            __shared__ uint64_t wave_best[kArgmaxBlock / kWave];
            const int64_t row = blockIdx.x / slices;
            const int64_t begin = (blockIdx.x % slices) * slice_len;
            const int64_t end = begin + slice_len < n ? begin + slice_len : n;
            const uint64_t best = block_best(thread_best<VEC>(x + row * stride, begin, end), wave_best);
            if (threadIdx.x == 0)
                part[blockIdx.x] = best;
        }

        // One wave per row: the maximum of its slice keys (slices <= 64).
        __global__ __launch_bounds__(kBlock) void argmax_merge_kernel(const uint64_t *__restrict__ part,
                                                                      int32_t *__restrict__ out, int64_t rows,
                                                                      int32_t slices)
        {
            const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
            if (row >= rows)
                return;
            const int lane = threadIdx.x % kWave;
            uint64_t best = lane < slices ? part[row * slices + lane] : 0;
#pragma unroll
            for (int off = 32; off > 0; off /= 2)
                best = max_u64(best, __shfl_xor(best, off, kWave));
            if (lane == 0)
                out[row] = key_index(best);
        }

        // Rows are cut into slices when fewer than kTargetBlocks blocks would
        // run; a slice keeps at least kMinSlice columns (8 per thread).
        constexpr int64_t kTargetBlocks = 512;
        constexpr int64_t kMinSlice = 8 * kArgmaxBlock;
        constexpr int kMaxSlices = kWave;

        struct SlicePlan
        {
            int32_t slices = 1;
            int64_t slice_len = 0;
            int64_t bytes = 0;
        };

        SlicePlan plan_slices(int64_t rows, int64_t n)
        {
            SlicePlan p;
            if (rows <= 0 || rows >= kTargetBlocks)
                return p;
            int64_t want = (kTargetBlocks + rows - 1) / rows;
            if (want > n / kMinSlice)
                want = n / kMinSlice;
            if (want > kMaxSlices)
                want = kMaxSlices;
            if (want < 2)
                return p;
            const int64_t len = ((n + want - 1) / want + 7) / 8 * 8;
            const int64_t slices = (n + len - 1) / len;
            if (slices < 2 || rows > INT32_MAX / slices)
                return p;
            p.slices = static_cast<int32_t>(slices);
            p.slice_len = len;
            p.bytes = rows * slices * static_cast<int64_t>(sizeof(uint64_t));
            return p;
        }
    } // namespace
} // namespace q3k

namespace q3k
{
    namespace
    {
        // Shared checks of both argmax entry points (src/ops/argmax.cu:104-161).
        int validate_argmax(const uint16_t *x, const int32_t *out, int64_t rows, int64_t row_stride,
                            int64_t search_size)
        {
            if (rows < 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax row count cannot be negative");
            if (row_stride <= 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax reduction dimension must be positive");
            if (row_stride > INT32_MAX)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax reduction dimension exceeds Int32 index range");
            if (search_size <= 0 || search_size > row_stride)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "valid reduction size is outside the last dimension");
            if (rows == 0)
                return Q3K_OK;
            if (x == nullptr || out == nullptr)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax received a null pointer");
            if (!aligned_to(x, 2) || !aligned_to(out, 4))
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax pointers must be aligned to their element size");
            if (rows > INT64_MAX / row_stride)
                return set_error(Q3K_ERR_OVERFLOW, "argmax input size overflows");
            return Q3K_OK;
        }

        // Launches for checked arguments: the sliced kernels when `part`
        // (8-byte aligned, room for plan.bytes) is given and the plan slices,
        // else one block per row.
        int launch_argmax(const uint16_t *x, int32_t *out, int64_t rows, int64_t row_stride, int64_t search_size,
                          const SlicePlan &plan, uint64_t *part, hipStream_t s)
        {
            const bool vec = aligned16(x) && row_stride % 8 == 0;
            if (plan.slices > 1 && part != nullptr)
            {
                const dim3 grid(static_cast<unsigned>(rows * plan.slices));
                if (vec)
                    argmax_slice_kernel<true><<<grid, dim3(kArgmaxBlock), 0, s>>>(x, part, row_stride, search_size,
                                                                                  plan.slices, plan.slice_len);
                else
                    argmax_slice_kernel<false><<<grid, dim3(kArgmaxBlock), 0, s>>>(x, part, row_stride, search_size,
                                                                                   plan.slices, plan.slice_len);
                const int64_t per_block = kBlock / kWave;
                argmax_merge_kernel<<<dim3(static_cast<unsigned>((rows + per_block - 1) / per_block)), dim3(kBlock), 0,
                                      s>>>(part, out, rows, plan.slices);
                return check_launch("argmax_last_dimension");
            }
            const unsigned grid = static_cast<unsigned>(rows < 65535 ? rows : 65535);
            if (vec)
                argmax_kernel<true><<<dim3(grid), dim3(kArgmaxBlock), 0, s>>>(x, out, rows, row_stride, search_size);
            else
                argmax_kernel<false><<<dim3(grid), dim3(kArgmaxBlock), 0, s>>>(x, out, rows, row_stride, search_size);
            return check_launch("argmax_last_dimension");
        }

        // The slice results of q3k_argmax_bf16_noalloc: a fixed array in
        // device memory, one copy per GPU, held until the process ends.  The
        // slice plan needs rows * slices * 8 bytes with rows * slices < 1024
        // (rows < 512, slices <= ceil(512 / rows)), so 8 KiB covers every
        // input; the array has twice that.  Every entry a call reads is
        // written by the same call first, so nothing needs clearing.
        constexpr int64_t kArgmaxScratchBytes = 16384;
        constexpr int kMaxScratchDevices = 64;
        std::mutex g_scratch_mutex;
        void *g_scratch_address[kMaxScratchDevices];  // per device, from hipGetSymbolAddress
    } // namespace

    static __device__ __align__(256) uint64_t scratch[kArgmaxScratchBytes / sizeof(uint64_t)];

    namespace
    {
        // The device address of `scratch` on the current GPU, looked up on
        // the first call per GPU (the host-side name is not a device address).
        int scratch_address(void **address)
        {
            int device = 0;
            if (hipGetDevice(&device) != hipSuccess)
                return set_error(Q3K_ERR_HIP, "argmax: no current GPU");
            if (device < 0 || device >= kMaxScratchDevices)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax scratch supports GPUs 0 .. %d", kMaxScratchDevices - 1);
            std::lock_guard<std::mutex> lock(g_scratch_mutex);
            if (g_scratch_address[device] == nullptr)
            {
                void *p = nullptr;
                const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
                if (e != hipSuccess || p == nullptr)
                    return set_error(Q3K_ERR_HIP, "argmax scratch lookup failed on GPU %d: %s", device,
                                     hipGetErrorString(e));
                g_scratch_address[device] = p;
            }
            *address = g_scratch_address[device];
            return Q3K_OK;
        }
    } // namespace
} // namespace q3k

extern "C" int q3k_argmax_bf16(const uint16_t *x, int32_t *out, int64_t rows, int64_t row_stride,
                               int64_t search_size, void *workspace, int64_t workspace_bytes,
                               q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_argmax(x, out, rows, row_stride, search_size))
        return st;
    if (workspace_bytes < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "argmax workspace size cannot be negative");
    if (rows == 0)
        return Q3K_OK;
    const SlicePlan plan = plan_slices(rows, search_size);
    const bool sliced = plan.slices > 1 && workspace != nullptr && workspace_bytes >= plan.bytes &&
                        aligned_to(workspace, 8);
    return launch_argmax(x, out, rows, row_stride, search_size, plan,
                         sliced ? static_cast<uint64_t *>(workspace) : nullptr, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int q3k_argmax_bf16_noalloc(const uint16_t *x, int32_t *out, int64_t rows, int64_t row_stride,
                                       int64_t search_size, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_argmax(x, out, rows, row_stride, search_size))
        return st;
    if (rows == 0)
        return Q3K_OK;
    const SlicePlan plan = plan_slices(rows, search_size);
    uint64_t *part = nullptr;
    if (plan.slices > 1)
    {
        if (plan.bytes > kArgmaxScratchBytes)
            return set_error(Q3K_ERR_INVALID_ARGUMENT,
                             "argmax needs %lld bytes of scratch, more than the library's fixed %lld",
                             static_cast<long long>(plan.bytes), static_cast<long long>(kArgmaxScratchBytes));
        void *address = nullptr;
        if (const int st = scratch_address(&address))
            return st;
        part = static_cast<uint64_t *>(address);
    }
    return launch_argmax(x, out, rows, row_stride, search_size, plan, part, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int64_t q3k_argmax_workspace_bytes(int64_t rows, int64_t search_size)
{
    return q3k::plan_slices(rows, search_size).bytes;
}
