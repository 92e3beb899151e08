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
//
// With few rows and a caller workspace, each row is cut into slices: one
// block per (row, slice) finds the slice's bound and lists its logits at or
// above it (steps 1-2 on the slice), and one block per row keeps the listed
// logits at or above the largest slice bound and finishes with step 3 (or
// the whole-row select when a slice saw a non-finite logit or its list
// overflowed).  The candidate set is the same either way.
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

        // The bin holding the k-th largest key, counting down from bin 255, and
        // the rank of that key inside the bin (bin 0 when bins 255 .. 1 hold
        // fewer than k keys).  Called by every lane of one wave: lane l holds
        // bins 255 - 4l .. 252 - 4l, a prefix sum over the lanes gives the
        // keys above each lane's bins, and the first lane whose bins reach k
        // walks its four bins and writes the result.
        __device__ __forceinline__ void find_bin(const uint32_t *hist, uint32_t k, uint32_t *bin_out,
                                                 uint32_t *rank_out)
        {
            const int lane = threadIdx.x % kWave;
            const int top = 255 - 4 * lane;
            uint32_t c[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                c[j] = hist[top - j];
            const uint32_t local = c[0] + c[1] + c[2] + c[3];
            uint32_t incl = local;
#pragma unroll
            for (int off = 1; off < kWave; off *= 2)
            {
                const uint32_t v = __shfl_up(incl, off, kWave);
                if (lane >= off)
                    incl += v;
            }
            const uint64_t hit = __ballot(incl >= k);
            const int owner = hit == 0 ? kWave - 1 : __ffsll(static_cast<unsigned long long>(hit)) - 1;
            if (lane == owner)
            {
                uint32_t above = incl - local;
                int j = 0;
                for (; j < 3; ++j)
                {
                    if (above + c[j] >= k)
                        break;
                    above += c[j];
                }
                *bin_out = static_cast<uint32_t>(top - j);
                *rank_out = k - above;
            }
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
            if (tid < kWave)
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
            if (tid < kWave)
            {
                uint32_t unused;
                find_bin(hist, rank, &sel[2], &unused);   // the low byte
            }
            __syncthreads();
            if (tid == 0)
                sel[2] = (hi << 8) | sel[2];
            __syncthreads();
            return sel[2];
        }

        __device__ __forceinline__ float bf_val(uint32_t b) { return __uint_as_float(b << 16); }

        // Visits logits c = begin .. end - 1 of a row, each thread its share:
        // 16-byte chunks (chunk j to thread j % kSelBlock) when the row is
        // 16-byte aligned (begin is then a multiple of 8), kSelUnroll chunks
        // loaded before any is visited (one block per row or slice: its loads
        // in flight set the read rate); single logits otherwise.  f(c, bits).
        constexpr int kSelUnroll = 4;
        template <typename F>
        __device__ __forceinline__ void for_row(const uint16_t *r, int64_t begin, int64_t end, F f)
        {
            const int tid = threadIdx.x;
            if ((reinterpret_cast<uintptr_t>(r) & 15u) == 0)
            {
                const int64_t chunk_end = end / 8;
                const Vec8 *rv = reinterpret_cast<const Vec8 *>(r);
                auto visit = [&](int64_t j, const Vec8 &v) __attribute__((always_inline)) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        f(8 * j + e, (e % 2 == 0) ? (v.d[e / 2] & 0xffffu) : (v.d[e / 2] >> 16));
                };
                // groups of kSelUnroll chunks, the last one partial: a
                // thread's loads of a group are all issued before any visit
                for (int64_t j = begin / 8 + tid; j < chunk_end; j += kSelUnroll * kSelBlock)
                {
                    Vec8 v[kSelUnroll];
#pragma unroll
                    for (int u = 0; u < kSelUnroll; ++u)
                        if (j + u * kSelBlock < chunk_end)
                            v[u] = load8<false>(rv + j + u * kSelBlock);
#pragma unroll
                    for (int u = 0; u < kSelUnroll; ++u)
                        if (j + u * kSelBlock < chunk_end)
                            visit(j + u * kSelBlock, v[u]);
                }
                const int64_t tail = 8 * chunk_end > begin ? 8 * chunk_end : begin;
                for (int64_t c = tail + tid; c < end; c += kSelBlock)
                    f(c, static_cast<uint32_t>(r[c]));
            }
            else
            {
                for (int64_t c = begin + tid; c < end; c += kSelBlock)
                    f(c, static_cast<uint32_t>(r[c]));
            }
        }

        // LDS of one selection block.
        struct SelShared
        {
            uint32_t wave_hist[kSelWaves][256];
            uint32_t hist[256];
            uint32_t thread_max[kSelBlock];
            uint32_t list_bits[kCandMax];
            int32_t list_index[kCandMax];
            uint32_t sel[3];
            uint32_t found, bad, listed, bound, overflow;
        };

        // Where a row's candidates go.
        struct CandOut
        {
            int32_t cap;
            int32_t *cand_index;
            uint16_t *cand_logit;
        };

        // Each thread's largest logit of [begin, end) as a key in thread_max
        // (a thread without logits counts as key 0, below every finite key),
        // and the non-finite flag in sh.bad; ends with a barrier.
        __device__ __forceinline__ void thread_maxima(const uint16_t *r, int64_t begin, int64_t end, SelShared &sh)
        {
            float tmax = -__builtin_huge_valf();
            uint32_t my_bad = 0u;
            for_row(r, begin, end, [&](int64_t, uint32_t b) __attribute__((always_inline)) {
                my_bad |= (b & 0x7f80u) == 0x7f80u ? 1u : 0u;
                tmax = fmaxf(tmax, bf_val(b));
            });
            sh.thread_max[threadIdx.x] = tmax == -__builtin_huge_valf() ? 0u : sel_key(__float_as_uint(tmax) >> 16);
            if (my_bad)
                atomicOr(&sh.bad, 1u);
            __syncthreads();
        }

        // Appends (bits, index) to the LDS list when `take`: one LDS atomic per
        // wave, slots by lane rank; entries past kCandMax are counted, not kept.
        __device__ __forceinline__ void list_append(SelShared &sh, bool take, uint32_t b, int32_t index)
        {
            const uint64_t ballot = __ballot(take);
            if (ballot == 0)
                return;
            const int lane = threadIdx.x % kWave;
            const int leader = __ffsll(static_cast<unsigned long long>(ballot)) - 1;
            uint32_t base = 0u;
            if (lane == leader)
                base = atomicAdd(&sh.listed, static_cast<uint32_t>(__popcll(ballot)));
            base = __shfl(base, leader);
            if (take)
            {
                const uint32_t pos = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ballot >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo(
                                                                          static_cast<uint32_t>(ballot), 0u));
                if (pos < static_cast<uint32_t>(kCandMax))
                {
                    sh.list_bits[pos] = b;
                    sh.list_index[pos] = index;
                }
            }
        }

        // The list entries at or above its k-th largest (k <= nl <= kCandMax)
        // go to the row's candidates, counted in sh.found.
        __device__ __forceinline__ void emit_list(SelShared &sh, uint32_t nl, uint32_t k, int64_t row,
                                                  const CandOut &co)
        {
            const uint32_t kth = block_kth([&](int i) { return sel_key(sh.list_bits[i]); }, static_cast<int>(nl), k,
                                           sh.hist, sh.sel);
            for (int i = threadIdx.x; i < static_cast<int>(nl); i += kSelBlock)
            {
                const uint32_t b = sh.list_bits[i];
                if (sel_key(b) >= kth)
                {
                    const uint32_t slot = atomicAdd(&sh.found, 1u);
                    if (slot < static_cast<uint32_t>(co.cap))
                    {
                        co.cand_index[row * co.cap + slot] = sh.list_index[i];
                        co.cand_logit[row * co.cap + slot] = static_cast<uint16_t>(b);
                    }
                }
            }
        }

        // Radix select over the whole row (per-wave histograms), then every
        // logit at or above the k-th largest goes to the candidates.
        __device__ void whole_row_select(const uint16_t *r, int64_t n, uint32_t k, int64_t row, const CandOut &co,
                                         SelShared &sh)
        {
            const int tid = threadIdx.x;
            uint32_t *my_hist = sh.wave_hist[tid / kWave];
            auto clear = [&]() __attribute__((always_inline)) {
                for (int i = tid; i < kSelWaves * 256; i += kSelBlock)
                    (&sh.wave_hist[0][0])[i] = 0u;
            };
            auto merge = [&]() __attribute__((always_inline)) {
                if (tid < 256)
                {
                    uint32_t sum = 0u;
#pragma unroll
                    for (int w = 0; w < kSelWaves; ++w)
                        sum += sh.wave_hist[w][tid];
                    sh.hist[tid] = sum;
                }
            };
            clear();
            __syncthreads();
            for_row(r, 0, n, [&](int64_t, uint32_t b) __attribute__((always_inline)) {
                atomicAdd(&my_hist[sel_key(b) >> 8], 1u);
            });
            __syncthreads();
            merge();
            __syncthreads();
            if (tid < kWave)
                find_bin(sh.hist, k, &sh.sel[0], &sh.sel[1]);
            clear();
            __syncthreads();
            const uint32_t hi = sh.sel[0], rank = sh.sel[1];
            for_row(r, 0, n, [&](int64_t, uint32_t b) __attribute__((always_inline)) {
                const uint32_t key = sel_key(b);
                if ((key >> 8) == hi)
                    atomicAdd(&my_hist[key & 255u], 1u);
            });
            __syncthreads();
            merge();
            __syncthreads();
            if (tid < kWave)
            {
                uint32_t unused;
                find_bin(sh.hist, rank, &sh.sel[2], &unused);
            }
            __syncthreads();
            if (tid == 0)
                sh.sel[2] = (hi << 8) | sh.sel[2];
            __syncthreads();
            const uint32_t kth = sh.sel[2];
            for_row(r, 0, n, [&](int64_t c, uint32_t b) __attribute__((always_inline)) {
                if (sel_key(b) >= kth)
                {
                    const uint32_t slot = atomicAdd(&sh.found, 1u);
                    if (slot < static_cast<uint32_t>(co.cap))
                    {
                        co.cand_index[row * co.cap + slot] = static_cast<int32_t>(c);
                        co.cand_logit[row * co.cap + slot] = static_cast<uint16_t>(b);
                    }
                }
            });
        }

        // The lower bound of the logits of [begin, end): the k-th largest of
        // the thread maxima as a value (-inf when fewer than k threads hold
        // logits: every logit is then taken), and its key in *key.
        __device__ __forceinline__ float maxima_bound(SelShared &sh, uint32_t k, uint32_t *key)
        {
            const uint32_t t_key = block_kth([&](int i) { return sh.thread_max[i]; }, kSelBlock, k, sh.hist, sh.sel);
            *key = t_key;
            return t_key == 0u ? -__builtin_huge_valf() : bf_val(key_bits(t_key));
        }

        __global__ __launch_bounds__(kSelBlock) void topk_select_kernel(const uint16_t *__restrict__ x, int64_t rows,
                                                                        int64_t stride, int64_t n, uint32_t k,
                                                                        CandOut co, int32_t *__restrict__ count,
                                                                        int32_t *__restrict__ nonfinite)
        {
            __shared__ SelShared sh;
            const int tid = threadIdx.x;
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                const uint16_t *r = x + row * stride;
                if (tid == 0)
                {
                    sh.found = 0u;
                    sh.bad = 0u;
                    sh.listed = 0u;
                }
                __syncthreads();
                // 1. per-thread maxima and the non-finite flag
                thread_maxima(r, 0, n, sh);
                bool exact = false;
                // rows with a non-finite logit keep the whole-row select
                if (k <= static_cast<uint32_t>(kSelBlock) && sh.bad == 0u)
                {
                    // 2. lower bound and the list of logits at or above it
                    uint32_t t_key;
                    const float t_val = maxima_bound(sh, k, &t_key);
                    for_row(r, 0, n, [&](int64_t c, uint32_t b) __attribute__((always_inline)) {
                        list_append(sh, bf_val(b) >= t_val, b, static_cast<int32_t>(c));
                    });
                    __syncthreads();
                    const uint32_t nl = sh.listed;
                    if (nl <= static_cast<uint32_t>(kCandMax))
                    {
                        // 3. exact k-th over the list (k <= nl: the bound holds)
                        emit_list(sh, nl, k, row, co);
                        exact = true;
                    }
                }
                if (!exact)
                    whole_row_select(r, n, k, row, co, sh);
                __syncthreads();
                if (tid == 0)
                {
                    count[row] = static_cast<int32_t>(sh.found);
                    nonfinite[row] = static_cast<int32_t>(sh.bad);
                }
                __syncthreads(); // the shared counters are reset for the next row
            }
        }

        // Sliced rows (few rows, k <= kSelBlock).  Per (row, slice): the
        // slice's bound T_s (k-th largest of its thread maxima) and its logits
        // at or above T_s.  The k threads whose maxima reach T_s hold k logits
        // >= T_s, so the row's k-th largest is >= T_s, and >= T = max_s T_s;
        // every top-k logit is >= the T_s of its own slice, so it is in that
        // slice's list.  The merge keeps the listed logits >= T and selects
        // exactly over them.
        constexpr int kSliceCand = 2048;

        struct SliceWork
        {
            uint32_t *header; // [rows * slices][4]: bound key, listed count, non-finite flag, 0
            uint32_t *bits;   // [rows * slices][kSliceCand]
            int32_t *index;   // [rows * slices][kSliceCand]
            int32_t slices;
            int64_t slice_len;
        };

        __global__ __launch_bounds__(kSelBlock) void topk_slice_kernel(const uint16_t *__restrict__ x, int64_t stride,
                                                                       int64_t n, uint32_t k, SliceWork w)
        {
            __shared__ SelShared sh;
            const int tid = threadIdx.x;
            const int64_t slot = blockIdx.x;
            const int64_t row = slot / w.slices;
            const int64_t begin = (slot % w.slices) * w.slice_len;
            const int64_t end = begin + w.slice_len < n ? begin + w.slice_len : n;
            const uint16_t *r = x + row * stride;
            if (tid == 0)
            {
                sh.bad = 0u;
                sh.listed = 0u;
            }
            __syncthreads();
            thread_maxima(r, begin, end, sh);
            uint32_t t_key = 0u;
            if (sh.bad == 0u)
            {
                const float t_val = maxima_bound(sh, k, &t_key);
                for_row(r, begin, end, [&](int64_t c, uint32_t b) __attribute__((always_inline)) {
                    list_append(sh, bf_val(b) >= t_val, b, static_cast<int32_t>(c));
                });
                __syncthreads();
                const uint32_t nl = sh.listed;
                const int kept = static_cast<int>(nl < static_cast<uint32_t>(kSliceCand) ? nl : kSliceCand);
                for (int i = tid; i < kept; i += kSelBlock)
                {
                    w.bits[slot * kSliceCand + i] = sh.list_bits[i];
                    w.index[slot * kSliceCand + i] = sh.list_index[i];
                }
            }
            if (tid == 0)
            {
                w.header[4 * slot + 0] = t_key;
                w.header[4 * slot + 1] = sh.listed;
                w.header[4 * slot + 2] = sh.bad;
                w.header[4 * slot + 3] = 0u;
            }
        }

        __global__ __launch_bounds__(kSelBlock) void topk_merge_kernel(const uint16_t *__restrict__ x, int64_t stride,
                                                                       int64_t n, uint32_t k, SliceWork w, CandOut co,
                                                                       int32_t *__restrict__ count,
                                                                       int32_t *__restrict__ nonfinite)
        {
            __shared__ SelShared sh;
            const int tid = threadIdx.x;
            const int64_t row = blockIdx.x;
            const uint32_t *hdr = w.header + 4 * row * w.slices;
            if (tid == 0)
            {
                sh.found = 0u;
                sh.bad = 0u;
                sh.listed = 0u;
                sh.bound = 0u;
                sh.overflow = 0u;
            }
            __syncthreads();
            if (tid < w.slices)
            {
                atomicMax(&sh.bound, hdr[4 * tid + 0]);
                if (hdr[4 * tid + 1] > static_cast<uint32_t>(kSliceCand))
                    atomicOr(&sh.overflow, 1u);
                if (hdr[4 * tid + 2] != 0u)
                    atomicOr(&sh.bad, 1u);
            }
            __syncthreads();
            bool exact = false;
            if (sh.bad == 0u && sh.overflow == 0u)
            {
                // each slice's list is read by its own group of threads, so
                // the lists of all slices are in flight together
                const uint32_t bound = sh.bound;
                const int per = kSelBlock / w.slices;
                const int sp = tid / per;
                if (sp < w.slices)
                {
                    const int64_t slot = row * w.slices + sp;
                    const int listed = static_cast<int>(hdr[4 * sp + 1]);
                    for (int i = tid % per; i < listed; i += per)
                    {
                        const uint32_t b = w.bits[slot * kSliceCand + i];
                        list_append(sh, sel_key(b) >= bound, b, w.index[slot * kSliceCand + i]);
                    }
                }
                __syncthreads();
                const uint32_t nl = sh.listed;
                if (nl <= static_cast<uint32_t>(kCandMax))
                {
                    emit_list(sh, nl, k, row, co);
                    exact = true;
                }
            }
            if (!exact)
                whole_row_select(x + row * stride, n, k, row, co, sh);
            __syncthreads();
            if (tid == 0)
            {
                count[row] = static_cast<int32_t>(sh.found);
                nonfinite[row] = static_cast<int32_t>(sh.bad);
            }
        }

        // Rows are cut into slices when fewer than kTargetBlocks blocks would
        // run (and k <= kSelBlock); a slice keeps at least kMinSlice logits.
        constexpr int64_t kTargetBlocks = 512;
        constexpr int64_t kMinSlice = 8 * kSelBlock;
        constexpr int kMaxSlices = kWave;

        struct SlicePlan
        {
            int32_t slices = 1;
            int64_t slice_len = 0;
            int64_t bytes = 0;
        };

        SlicePlan plan_slices(int64_t rows, int64_t n, int32_t k)
        {
            SlicePlan p;
            if (rows <= 0 || rows >= kTargetBlocks || k <= 0 || k > kSelBlock)
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
            if (slices < 2)
                return p;
            p.slices = static_cast<int32_t>(slices);
            p.slice_len = len;
            p.bytes = rows * slices * (4 * static_cast<int64_t>(sizeof(uint32_t)) + kSliceCand * 8);
            return p;
        }
    } // namespace
} // namespace q3k

extern "C" int q3k_topk_candidates_bf16(const uint16_t *logits, int64_t rows, int64_t row_stride,
                                        int64_t search_size, int32_t k, int32_t cap, int32_t *count,
                                        int32_t *cand_index, uint16_t *cand_logit, int32_t *nonfinite,
                                        void *workspace, int64_t workspace_bytes, q3k_stream_t stream)
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
    if (workspace_bytes < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "top-k workspace size cannot be negative");
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
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const CandOut co{cap, cand_index, cand_logit};
    const SlicePlan plan = plan_slices(rows, search_size, k);
    if (plan.slices > 1 && workspace != nullptr && workspace_bytes >= plan.bytes && aligned_to(workspace, 16))
    {
        const int64_t slots = rows * plan.slices;
        SliceWork w;
        w.header = static_cast<uint32_t *>(workspace);
        w.bits = w.header + 4 * slots;
        w.index = reinterpret_cast<int32_t *>(w.bits + slots * kSliceCand);
        w.slices = plan.slices;
        w.slice_len = plan.slice_len;
        topk_slice_kernel<<<dim3(static_cast<unsigned>(slots)), dim3(kSelBlock), 0, s>>>(
            logits, row_stride, search_size, static_cast<uint32_t>(k), w);
        topk_merge_kernel<<<dim3(static_cast<unsigned>(rows)), dim3(kSelBlock), 0, s>>>(
            logits, row_stride, search_size, static_cast<uint32_t>(k), w, co, count, nonfinite);
        return check_launch("topk_candidates");
    }
    const unsigned grid = static_cast<unsigned>(rows < 65535 ? rows : 65535);
    topk_select_kernel<<<dim3(grid), dim3(kSelBlock), 0, s>>>(logits, rows, row_stride, search_size,
                                                               static_cast<uint32_t>(k), co, count, nonfinite);
    return check_launch("topk_candidates");
}

extern "C" int64_t q3k_topk_workspace_bytes(int64_t rows, int64_t search_size, int32_t k)
{
    return q3k::plan_slices(rows, search_size, k).bytes;
}
