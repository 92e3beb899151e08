// Top-k candidate selection for gfx950: the GPU half of sampling.  The
// reference copies every [B, V] logit to the host and runs temperature,
// top-k (nth_element, keeping every token whose score ties the k-th),
// sort, softmax, top-p and the draw there (src/generation/sampler.cpp:
// 134-265, 288-312).  Temperature scaling is monotone, so the top-k set is
// "every logit >= the k-th largest logit"; this kernel finds that value
// with a two-pass radix select over order-preserving 16-bit keys (high
// byte, then low byte, 256-bin LDS histograms) and compacts the tokens at
// or above it (index and bf16 bits, any order), so the host finishes the
// reference's steps on about k candidates instead of V logits.
//
// One block of 1024 threads per row (rows strided over the grid).  Logits of
// a row share few exponents, so most increments hit a handful of bins: each
// wave counts into its own histogram and the 16 are summed before the bin
// search.  A row with a non-finite logit is flagged (the reference throws
// for it).
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        constexpr int kSelBlock = 1024;

        // order-preserving key of a finite bf16 value; -0 and +0 share a key
        // (the reference compares the scores as doubles)
        __device__ __forceinline__ uint32_t sel_key(uint32_t b)
        {
            if (b == 0x8000u)
                b = 0u;
            return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
        }

        // the bin holding the k-th largest key, counting down from bin 255, and
        // the rank of that key inside the bin (single thread; 256 bins)
        __device__ __forceinline__ void find_bin(const uint32_t *hist, uint32_t k, uint32_t *bin_out,
                                                 uint32_t *rank_out)
        {
            uint32_t above = 0;
            int bin = 255;
            for (; bin > 0; --bin)
            {
                if (above + hist[bin] >= k)
                    break;
                above += hist[bin];
            }
            *bin_out = static_cast<uint32_t>(bin);
            *rank_out = k - above;
        }

        constexpr int kSelWaves = kSelBlock / kWave;

        __global__ __launch_bounds__(kSelBlock) void topk_select_kernel(const uint16_t *__restrict__ x, int64_t rows,
                                                                        int64_t stride, int64_t n, uint32_t k,
                                                                        int32_t cap, int32_t *__restrict__ count,
                                                                        int32_t *__restrict__ cand_index,
                                                                        uint16_t *__restrict__ cand_logit,
                                                                        int32_t *__restrict__ nonfinite)
        {
            __shared__ uint32_t wave_hist[kSelWaves][256];
            __shared__ uint32_t hist[256];
            __shared__ uint32_t sel[2];
            __shared__ uint32_t found, bad;
            const int tid = threadIdx.x;
            const int wave = tid / kWave;
            uint32_t *my_hist = wave_hist[wave];
            auto clear = [&]() {
                for (int i = tid; i < kSelWaves * 256; i += kSelBlock)
                    (&wave_hist[0][0])[i] = 0u;
            };
            auto merge = [&]() {
                if (tid < 256)
                {
                    uint32_t sum = 0u;
#pragma unroll
                    for (int w = 0; w < kSelWaves; ++w)
                        sum += wave_hist[w][tid];
                    hist[tid] = sum;
                }
            };
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                const uint16_t *r = x + row * stride;
                clear();
                if (tid == 0)
                {
                    found = 0u;
                    bad = 0u;
                }
                __syncthreads();
                uint32_t my_bad = 0u;
                for (int64_t c = tid; c < n; c += kSelBlock)
                {
                    const uint32_t b = r[c];
                    my_bad |= (b & 0x7f80u) == 0x7f80u ? 1u : 0u;
                    atomicAdd(&my_hist[sel_key(b) >> 8], 1u);
                }
                if (my_bad)
                    atomicOr(&bad, 1u);
                __syncthreads();
                merge();
                __syncthreads();
                if (tid == 0)
                    find_bin(hist, k, &sel[0], &sel[1]);
                clear();
                __syncthreads();
                const uint32_t hi = sel[0], rank = sel[1];
                for (int64_t c = tid; c < n; c += kSelBlock)
                {
                    const uint32_t key = sel_key(r[c]);
                    if ((key >> 8) == hi)
                        atomicAdd(&my_hist[key & 255u], 1u);
                }
                __syncthreads();
                merge();
                __syncthreads();
                if (tid == 0)
                {
                    uint32_t lo, unused;
                    find_bin(hist, rank, &lo, &unused);
                    sel[0] = (hi << 8) | lo;
                }
                __syncthreads();
                const uint32_t kth = sel[0];
                for (int64_t c = tid; c < n; c += kSelBlock)
                {
                    const uint32_t b = r[c];
                    if (sel_key(b) >= kth)
                    {
                        const uint32_t slot = atomicAdd(&found, 1u);
                        if (slot < static_cast<uint32_t>(cap))
                        {
                            cand_index[row * cap + slot] = static_cast<int32_t>(c);
                            cand_logit[row * cap + slot] = static_cast<uint16_t>(b);
                        }
                    }
                }
                __syncthreads();
                if (tid == 0)
                {
                    count[row] = static_cast<int32_t>(found);
                    nonfinite[row] = static_cast<int32_t>(bad);
                }
                __syncthreads(); // the shared counters are reset for the next row
            }
        }
    } // namespace
} // namespace q3k

extern "C" int q3k_topk_candidates_bf16(const uint16_t *logits, int64_t rows, int64_t row_stride,
                                        int64_t search_size, int32_t k, int32_t cap, int32_t *count,
                                        int32_t *cand_index, uint16_t *cand_logit, int32_t *nonfinite,
                                        q3k_stream_t stream)
{
    using namespace q3k;
    if (rows < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "top-k row count cannot be negative");
    if (row_stride <= 0 || row_stride > INT32_MAX)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "top-k vocabulary size must be in [1, 2^31)");
    if (search_size <= 0 || search_size > row_stride)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "valid_vocab_size is outside the logits vocabulary");
    if (k <= 0 || k > search_size)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "top_k must be in [1, valid_vocab_size]");
    if (cap <= 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "candidate capacity must be positive");
    if (rows == 0)
        return Q3K_OK;
    if (logits == nullptr || count == nullptr || cand_index == nullptr || cand_logit == nullptr ||
        nonfinite == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "top-k selection received a null pointer");
    if (!aligned_to(logits, 2) || !aligned_to(count, 4) || !aligned_to(cand_index, 4) ||
        !aligned_to(cand_logit, 2) || !aligned_to(nonfinite, 4))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "top-k pointers must be aligned to their element size");
    if (rows > INT64_MAX / row_stride || rows > INT64_MAX / cap)
        return set_error(Q3K_ERR_OVERFLOW, "top-k sizes overflow");
    const unsigned grid = static_cast<unsigned>(rows < 65535 ? rows : 65535);
    topk_select_kernel<<<dim3(grid), dim3(kSelBlock), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        logits, rows, row_stride, search_size, static_cast<uint32_t>(k), cap, count, cand_index, cand_logit,
        nonfinite);
    return check_launch("topk_candidates");
}
