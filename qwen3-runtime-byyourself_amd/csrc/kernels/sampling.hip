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
// One block of 1024 threads per row (rows strided over the grid), usually
// two reads of the row:
//   1. each thread's largest logit (16-byte loads when the row is aligned)
//      and the non-finite flag;
//   2. T = the k-th largest of those 1024 maxima.  The k threads whose maxima
//      are >= T each hold a logit >= T, so the k-th largest logit is >= T
//      and every top-k token is among the logits >= T, which the second read
//      appends to an LDS list (wave-aggregated slots);
//   3. the exact k-th largest comes from a radix select over that short
//      list, and the list entries at or above it are written out.
// When k exceeds the thread count or more than kCandMax logits reach T (many
// ties), the row takes the three-read radix select over the whole row: logits
// of a row share few exponents, so most increments hit a handful of bins and
// each wave counts into its own histogram.  A row with a non-finite logit is
// flagged (the reference throws for it).
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        constexpr int kSelBlock = 1024;
        constexpr int kSelWaves = kSelBlock / kWave;
        constexpr int kCandMax = 4096;

        // order-preserving key of a finite bf16 value; -0 and +0 share a key
        // (the reference compares the scores as doubles)
        __device__ __forceinline__ uint32_t sel_key(uint32_t b)
        {
            if (b == 0x8000u)
                b = 0u;
            return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
        }

        // the bf16 bits whose key is `key` (the +0 representative for 0)
        __device__ __forceinline__ uint32_t key_bits(uint32_t key)
        {
            return (key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu);
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

        // k-th largest (1 <= k <= n) of the 16-bit keys key_at(0 .. n - 1),
        // block-wide, by two 8-bit radix passes over one shared histogram
        template <typename KeyAt>
        __device__ uint32_t block_kth(KeyAt key_at, int n, uint32_t k, uint32_t *hist, uint32_t *sel)
        {
            const int tid = threadIdx.x;
            if (tid < 256)
                hist[tid] = 0u;
            __syncthreads();
            for (int i = tid; i < n; i += kSelBlock)
                atomicAdd(&hist[key_at(i) >> 8], 1u);
            __syncthreads();
            if (tid == 0)
                find_bin(hist, k, &sel[0], &sel[1]);
            __syncthreads();
            const uint32_t hi = sel[0], rank = sel[1];
            if (tid < 256)
                hist[tid] = 0u;
            __syncthreads();
            for (int i = tid; i < n; i += kSelBlock)
            {
                const uint32_t key = key_at(i);
                if ((key >> 8) == hi)
                    atomicAdd(&hist[key & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0)
            {
                uint32_t lo, unused;
                find_bin(hist, rank, &lo, &unused);
                sel[2] = (hi << 8) | lo;
            }
            __syncthreads();
            return sel[2];
        }

        __device__ __forceinline__ float bf_val(uint32_t b) { return __uint_as_float(b << 16); }

        // Visits logits c = 0 .. n - 1 of a row, each thread its share:
        // 16-byte chunks (chunk j to thread j % kSelBlock) when the row is
        // 16-byte aligned, kSelUnroll chunks loaded before any is visited (one
        // block per row: its loads in flight set the row's read rate); single
        // logits otherwise.  f(c, bits).
        constexpr int kSelUnroll = 4;
        template <typename F>
        __device__ __forceinline__ void for_row(const uint16_t *r, int64_t n, F f)
        {
            const int tid = threadIdx.x;
            if ((reinterpret_cast<uintptr_t>(r) & 15u) == 0)
            {
                const int64_t chunks = n / 8;
                const Vec8 *rv = reinterpret_cast<const Vec8 *>(r);
                auto visit = [&](int64_t j, const Vec8 &v) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        f(8 * j + e, (e % 2 == 0) ? (v.d[e / 2] & 0xffffu) : (v.d[e / 2] >> 16));
                };
                int64_t j = tid;
                for (; j + (kSelUnroll - 1) * kSelBlock < chunks; j += kSelUnroll * kSelBlock)
                {
                    Vec8 v[kSelUnroll];
#pragma unroll
                    for (int u = 0; u < kSelUnroll; ++u)
                        v[u] = load8<false>(rv + j + u * kSelBlock);
#pragma unroll
                    for (int u = 0; u < kSelUnroll; ++u)
                        visit(j + u * kSelBlock, v[u]);
                }
                for (; j < chunks; j += kSelBlock)
                    visit(j, load8<false>(rv + j));
                for (int64_t c = 8 * chunks + tid; c < n; c += kSelBlock)
                    f(c, static_cast<uint32_t>(r[c]));
            }
            else
            {
                for (int64_t c = tid; c < n; c += kSelBlock)
                    f(c, static_cast<uint32_t>(r[c]));
            }
        }

        __global__ __launch_bounds__(kSelBlock) void topk_select_kernel(const uint16_t *__restrict__ x, int64_t rows,
                                                                        int64_t stride, int64_t n, uint32_t k,
                                                                        int32_t cap, int32_t *__restrict__ count,
                                                                        int32_t *__restrict__ cand_index,
                                                                        uint16_t *__restrict__ cand_logit,
                                                                        int32_t *__restrict__ nonfinite)
        {
            __shared__ uint32_t wave_hist[kSelWaves][256];
            __shared__ uint32_t hist[256];
            __shared__ uint32_t thread_max[kSelBlock];
            __shared__ uint32_t list_bits[kCandMax];
            __shared__ int32_t list_index[kCandMax];
            __shared__ uint32_t sel[3];
            __shared__ uint32_t found, bad, listed;
            const int tid = threadIdx.x;
            const int lane = tid % kWave;
            const int wave = tid / kWave;
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                const uint16_t *r = x + row * stride;
                if (tid == 0)
                {
                    found = 0u;
                    bad = 0u;
                    listed = 0u;
                }
                __syncthreads();
                // 1. per-thread maximum and non-finite flag
                float tmax = -__builtin_huge_valf();
                uint32_t my_bad = 0u;
                for_row(r, n, [&](int64_t, uint32_t b) {
                    my_bad |= (b & 0x7f80u) == 0x7f80u ? 1u : 0u;
                    tmax = fmaxf(tmax, bf_val(b));
                });
                // a thread without logits counts as key 0, below every finite key
                thread_max[tid] = tmax == -__builtin_huge_valf() ? 0u : sel_key(__float_as_uint(tmax) >> 16);
                if (my_bad)
                    atomicOr(&bad, 1u);
                __syncthreads();
                bool exact = false;
                uint32_t kth = 0u;
                // rows with a non-finite logit keep the whole-row select
                if (k <= static_cast<uint32_t>(kSelBlock) && bad == 0u)
                {
                    // 2. lower bound and the list of logits at or above it; fewer
                    // than k threads holding logits gives key 0: take every logit
                    const uint32_t t_key = block_kth([&](int i) { return thread_max[i]; }, kSelBlock, k, hist, sel);
                    const float t_val = t_key == 0u ? -__builtin_huge_valf() : bf_val(key_bits(t_key));
                    for_row(r, n, [&](int64_t c, uint32_t b) {
                        const bool take = bf_val(b) >= t_val;
                        const uint64_t ballot = __ballot(take);
                        if (ballot == 0)
                            return;
                        const int leader = __ffsll(static_cast<unsigned long long>(ballot)) - 1;
                        uint32_t base = 0u;
                        if (lane == leader)
                            base = atomicAdd(&listed, static_cast<uint32_t>(__popcll(ballot)));
                        base = __shfl(base, leader);
                        if (take)
                        {
                            const uint32_t pos =
                                base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ballot >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo(
                                                                     static_cast<uint32_t>(ballot), 0u));
                            if (pos < static_cast<uint32_t>(kCandMax))
                            {
                                list_bits[pos] = b;
                                list_index[pos] = static_cast<int32_t>(c);
                            }
                        }
                    });
                    __syncthreads();
                    const uint32_t nl = listed;
                    if (nl <= static_cast<uint32_t>(kCandMax))
                    {
                        // 3. exact k-th over the list (k <= nl: the bound holds)
                        kth = block_kth([&](int i) { return sel_key(list_bits[i]); }, static_cast<int>(nl), k, hist,
                                        sel);
                        for (int i = tid; i < static_cast<int>(nl); i += kSelBlock)
                        {
                            const uint32_t b = list_bits[i];
                            if (sel_key(b) >= kth)
                            {
                                const uint32_t slot = atomicAdd(&found, 1u);
                                if (slot < static_cast<uint32_t>(cap))
                                {
                                    cand_index[row * cap + slot] = list_index[i];
                                    cand_logit[row * cap + slot] = static_cast<uint16_t>(b);
                                }
                            }
                        }
                        exact = true;
                    }
                }
                if (!exact)
                {
                    // radix select over the whole row: per-wave histograms
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
                    clear();
                    __syncthreads();
                    for_row(r, n, [&](int64_t, uint32_t b) { atomicAdd(&my_hist[sel_key(b) >> 8], 1u); });
                    __syncthreads();
                    merge();
                    __syncthreads();
                    if (tid == 0)
                        find_bin(hist, k, &sel[0], &sel[1]);
                    clear();
                    __syncthreads();
                    const uint32_t hi = sel[0], rank = sel[1];
                    for_row(r, n, [&](int64_t, uint32_t b) {
                        const uint32_t key = sel_key(b);
                        if ((key >> 8) == hi)
                            atomicAdd(&my_hist[key & 255u], 1u);
                    });
                    __syncthreads();
                    merge();
                    __syncthreads();
                    if (tid == 0)
                    {
                        uint32_t lo, unused;
                        find_bin(hist, rank, &lo, &unused);
                        sel[2] = (hi << 8) | lo;
                    }
                    __syncthreads();
                    kth = sel[2];
                    for_row(r, n, [&](int64_t c, uint32_t b) {
                        if (sel_key(b) >= kth)
                        {
                            const uint32_t slot = atomicAdd(&found, 1u);
                            if (slot < static_cast<uint32_t>(cap))
                            {
                                cand_index[row * cap + slot] = static_cast<int32_t>(c);
                                cand_logit[row * cap + slot] = static_cast<uint16_t>(b);
                            }
                        }
                    });
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
