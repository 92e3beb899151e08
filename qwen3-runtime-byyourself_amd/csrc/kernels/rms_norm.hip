// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Fast path (N % 8 == 0, N <= 16384, 16-byte aligned pointers): each row is
// held in registers between its load and its stores, so x (and the residual
// delta) is read from HBM exactly once.  Rows are split into 128-bit vectors
// (8 bf16); vector j sits in thread j % P, slot j / P of the P threads that
// own the row, so every load instruction of a wave covers 1 KiB of
// contiguous memory.  Narrow rows (<= 256 elements, e.g. per-head Q/K norm
// over 128) give each row an aligned group of lanes and reduce the sum of
// squares with DPP inside the wave; rows up to 1024 elements use one wave;
// wider rows (hidden 2048 .. 16384) use one block of up to eight waves per
// row whose wave sums meet in LDS behind one barrier.  Loads and stores are
// non-temporal.  The mapping per width was chosen by measurement on MI355X.
//
// Generic path (any N, any alignment): one 256-thread block per row, scalar
// loads, two passes over the row (reference structure, wave64 reduction).
//
// Arithmetic follows src/ops/rms_norm.cu:82-121 and
// src/ops/elementwise.cu:28-35: fp32 sum of squares, mean = sum / N,
// inv = rsqrt(mean + eps), y = RNE(RNE(x * inv) * w); the fused form adds
// h = RNE(h + d) first and normalises the rounded h.
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        // Normalise the row slice held by this thread: h = RNE(h + d) (ADD),
        // then the partial sum of squares of the rounded values.
        template <int VPT, bool ADD>
        __device__ __forceinline__ float add_and_square(Vec8 (&x)[VPT], const Vec8 (&dv)[VPT], const bool (&live)[VPT])
        {
            float partial = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                if (!live[i])
                    continue;
                if constexpr (ADD)
                {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        x[i].d[k] = pack_rne(bf_lo(x[i].d[k]) + bf_lo(dv[i].d[k]), bf_hi(x[i].d[k]) + bf_hi(dv[i].d[k]));
                }
                partial += sum_sq8(x[i]);
            }
            return partial;
        }

        // Group of G lanes per row (G <= 64), VPT vectors per lane.
        template <int G, int VPT, bool ADD, int NTM>
        __global__ __launch_bounds__(kBlock) void rms_rows_kernel(
            uint16_t *__restrict__ h, const uint16_t *__restrict__ d,
            const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
            int64_t rows, int nvec, float inv_n, float eps)
        {
            constexpr int kRowsPerBlock = kBlock / G;
            const int lane = threadIdx.x % G;
            const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / G;
            if (row >= rows)
                return;

            const int64_t row_offset = row * static_cast<int64_t>(nvec);
            Vec8 *hrow = reinterpret_cast<Vec8 *>(h) + row_offset;
            const Vec8 *wvec = reinterpret_cast<const Vec8 *>(w);
            Vec8 *yrow = reinterpret_cast<Vec8 *>(y) + row_offset;

            // Issue every load of the row (and the weights) before any use.
            Vec8 x[VPT], dv[VPT], wv[VPT];
            bool live[VPT];
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                const int j = lane + i * G;
                live[i] = j < nvec;
                if (live[i])
                {
                    x[i] = load8<nt_load(NTM)>(hrow + j);
                    if constexpr (ADD)
                        dv[i] = load8<nt_load(NTM)>(reinterpret_cast<const Vec8 *>(d) + row_offset + j);
                    wv[i] = wvec[j];
                }
            }
            const float partial = add_and_square<VPT, ADD>(x, dv, live);
            if constexpr (ADD)
            {
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                    if (live[i])
                        store8<nt_store(NTM)>(hrow + lane + i * G, x[i]);
            }
            const float inv = inverse_rms(group_sum<G>(partial), inv_n, eps);
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (live[i])
                    store8<nt_store(NTM)>(yrow + lane + i * G, norm_scale8(x[i], wv[i], inv));
        }

        // WPR waves per row, R consecutive rows per block, VPT vectors per
        // lane and row; the wave sums of all R rows meet in LDS behind one
        // barrier.  PR > 0 raises the wave priority while the loads are issued.
        template <int WPR, int VPT, int R, bool ADD, int NTM, int PR, bool REMAP>
        __global__ __launch_bounds__(WPR * kWave) void rms_block_kernel(
            uint16_t *__restrict__ h, const uint16_t *__restrict__ d,
            const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
            int64_t rows, int nvec, float inv_n, float eps)
        {
            constexpr int kThreads = WPR * kWave;
            __shared__ float wave_sums[R][WPR];
            const int t = threadIdx.x;
            const int64_t row0 = static_cast<int64_t>(tile_index<REMAP>(blockIdx.x, gridDim.x)) * R;
            const Vec8 *wvec = reinterpret_cast<const Vec8 *>(w);

            Vec8 x[R][VPT], dv[R][VPT], wv[VPT];
            bool live[VPT];
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(PR);
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                const int j = t + i * kThreads;
                live[i] = j < nvec;
                if (live[i])
                    wv[i] = wvec[j];
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
            {
                const int64_t row = row0 + r;
                if (row >= rows)
                    break;
                const int64_t row_offset = row * static_cast<int64_t>(nvec);
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                {
                    const int j = t + i * kThreads;
                    if (live[i])
                    {
                        x[r][i] = load8<nt_load(NTM)>(reinterpret_cast<const Vec8 *>(h) + row_offset + j);
                        if constexpr (ADD)
                            dv[r][i] = load8<nt_load(NTM)>(reinterpret_cast<const Vec8 *>(d) + row_offset + j);
                    }
                }
            }
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(0);

            float total[R];
#pragma unroll
            for (int r = 0; r < R; ++r)
            {
                total[r] = 0.0f;
                const int64_t row = row0 + r;
                if (row >= rows)
                    break;
                const float partial = add_and_square<VPT, ADD>(x[r], dv[r], live);
                if constexpr (ADD)
                {
#pragma unroll
                    for (int i = 0; i < VPT; ++i)
                        if (live[i])
                            store8<nt_store(NTM)>(reinterpret_cast<Vec8 *>(h) + row * nvec + t + i * kThreads, x[r][i]);
                }
                total[r] = group_sum<kWave>(partial);
            }
            if constexpr (WPR > 1)
            {
                if (t % kWave == 0)
                {
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        wave_sums[r][t / kWave] = total[r];
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < R; ++r)
                {
                    total[r] = 0.0f;
#pragma unroll
                    for (int k = 0; k < WPR; ++k)
                        total[r] += wave_sums[r][k];
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
            {
                const int64_t row = row0 + r;
                if (row >= rows)
                    break;
                const float inv = inverse_rms(total[r], inv_n, eps);
                Vec8 *yrow = reinterpret_cast<Vec8 *>(y) + row * static_cast<int64_t>(nvec);
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                    if (live[i])
                        store8<nt_store(NTM)>(yrow + t + i * kThreads, norm_scale8(x[r][i], wv[i], inv));
            }
        }

        // Block-wide sum for the generic kernel: wave sums through LDS, then
        // every thread adds the wave partials in the same order.
        __device__ float block_sum(float v, float *scratch)
        {
            v = group_sum<kWave>(v);
            const int wave = threadIdx.x / kWave;
            if (threadIdx.x % kWave == 0)
                scratch[wave] = v;
            __syncthreads();
            float total = 0.0f;
            const int waves = blockDim.x / kWave;
            for (int i = 0; i < waves; ++i)
                total += scratch[i];
            __syncthreads();
            return total;
        }

        template <bool ADD>
        __global__ __launch_bounds__(kBlock) void rms_rows_generic_kernel(
            uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
            int64_t rows, int64_t n, float eps)
        {
            __shared__ float scratch[kBlock / kWave];
            const float inv_n = 1.0f / static_cast<float>(n);
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                uint16_t *hr = h + row * n;
                const uint16_t *dr = d + row * n;
                uint16_t *yr = y + row * n;
                float partial = 0.0f;
                for (int64_t c = threadIdx.x; c < n; c += blockDim.x)
                {
                    float v = bf_to_f(hr[c]);
                    if constexpr (ADD)
                    {
                        const uint16_t s = f_to_bf(v + bf_to_f(dr[c]));
                        hr[c] = s;
                        v = bf_to_f(s);
                    }
                    partial += v * v;
                }
                const float inv = inverse_rms(block_sum(partial, scratch), inv_n, eps);
                for (int64_t c = threadIdx.x; c < n; c += blockDim.x)
                {
                    const float nrm = bf_to_f(f_to_bf(bf_to_f(hr[c]) * inv));
                    yr[c] = f_to_bf(nrm * bf_to_f(w[c]));
                }
            }
        }

        // Non-temporal mode bits (loads | stores), measured on MI355X with
        // input cycles far above the Infinity Cache: non-temporal loads and
        // stores for every row width, except narrow rows without the fused
        // add, where plain loads are faster.
        constexpr int kNtmBlock = 3;
        template <bool ADD>
        constexpr int ntm_rows() { return ADD ? 3 : 2; }

        template <int G, int VPT, bool ADD>
        void launch_rows(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                         int64_t rows, int nvec, float inv_n, float eps, hipStream_t stream)
        {
            constexpr int kRowsPerBlock = kBlock / G;
            const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
            rms_rows_kernel<G, VPT, ADD, ntm_rows<ADD>()><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream>>>(
                h, d, w, y, rows, nvec, inv_n, eps);
        }

        // Rows per block and load priority of the block kernel (measured).
        constexpr int kRowsPerBlockAdd = 1;
        constexpr int kRowsPerBlockNorm = 1;
        constexpr int kPrioAdd = 1;
        constexpr int kPrioNorm = 0;
        constexpr bool kRemapRows = false;  // XCD-contiguous rows measured slower

        template <int WPR, int VPT, bool ADD>
        void launch_block(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                          int64_t rows, int nvec, float inv_n, float eps, hipStream_t stream)
        {
            constexpr int R = ADD ? kRowsPerBlockAdd : kRowsPerBlockNorm;
            const int64_t blocks = (rows + R - 1) / R;
            rms_block_kernel<WPR, VPT, R, ADD, kNtmBlock, ADD ? kPrioAdd : kPrioNorm, kRemapRows>
                <<<dim3(static_cast<unsigned>(blocks)), dim3(WPR * kWave), 0, stream>>>(h, d, w, y, rows, nvec, inv_n, eps);
        }

        template <int VPT, bool ADD>
        bool launch_block_waves(int waves, uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                                int64_t rows, int nvec, float inv_n, float eps, hipStream_t stream)
        {
            switch (waves)
            {
            case 1: launch_block<1, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 2: launch_block<2, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 3: launch_block<3, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 4: launch_block<4, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 5: launch_block<5, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 6: launch_block<6, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 7: launch_block<7, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            case 8: launch_block<8, VPT, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream); return true;
            default: return false;
            }
        }

        // Row-to-lane mapping by row width, in 128-bit vectors (measured on MI355X):
        //   nvec <= 32:   a group of pow2 >= nvec lanes per row, several rows per wave
        //                 (per-head norms, 128 elements = 16 lanes);
        //   nvec <= 128:  one wave per row, 1-2 vectors per lane (hidden 1024);
        //   nvec <= 2048: one row per block of up to 8 waves; one vector per lane
        //                 for the fused add when nvec <= 512 (hidden <= 4096),
        //                 else two (four beyond 8192 elements).
        template <bool ADD>
        bool launch_fast(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                         int64_t rows, int64_t n, float eps, hipStream_t stream)
        {
            const int nvec = static_cast<int>(n / 8);
            const float inv_n = 1.0f / static_cast<float>(n);
            if (nvec <= 1)
                launch_rows<1, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 2)
                launch_rows<2, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 4)
                launch_rows<4, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 8)
                launch_rows<8, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 16)
                launch_rows<16, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 32)
                launch_rows<32, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 64)
                launch_rows<64, 1, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 128)
                launch_rows<64, 2, ADD>(h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (ADD && nvec <= 512)
                return launch_block_waves<1, ADD>((nvec + 63) / 64, h, d, w, y, rows, nvec, inv_n, eps, stream);
            else if (nvec <= 1024)
                return launch_block_waves<2, ADD>((nvec + 127) / 128, h, d, w, y, rows, nvec, inv_n, eps, stream);
            else
                return launch_block_waves<4, ADD>((nvec + 255) / 256, h, d, w, y, rows, nvec, inv_n, eps, stream);
            return true;
        }

        constexpr int64_t kMaxFastN = 8 * kWave * 4 * 8; // 16384 elements per row
        constexpr int64_t kMaxGenericBlocks = 1 << 20;

        template <bool ADD>
        int rms_dispatch(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                         int64_t rows, int64_t n, float eps, hipStream_t stream, const char *name)
        {
            const bool fast = (n % 8 == 0) && n <= kMaxFastN && aligned16(h) && aligned16(w) && aligned16(y) &&
                              (!ADD || aligned16(d)) && rows < (int64_t{1} << 31);
            if (!(fast && launch_fast<ADD>(h, d, w, y, rows, n, eps, stream)))
            {
                const int64_t blocks = rows < kMaxGenericBlocks ? rows : kMaxGenericBlocks;
                rms_rows_generic_kernel<ADD><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream>>>(
                    h, d, w, y, rows, n, eps);
            }
            return check_launch(name);
        }

        int validate_common(const void *x, const void *w, const void *y, int64_t rows, int64_t n, float eps)
        {
            if (rows < 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm row count cannot be negative");
            if (n <= 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm normalized size must be positive");
            if (!(eps > 0.0f) || eps == __builtin_huge_valf())
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm epsilon must be finite and positive");
            if (rows > 0 && (x == nullptr || w == nullptr || y == nullptr))
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm received a null pointer");
            if (rows > INT64_MAX / n)
                return set_error(Q3K_ERR_OVERFLOW, "RMSNorm element count overflows");
            if (!aligned_to(x, 2) || !aligned_to(w, 2) || !aligned_to(y, 2))
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm pointers must be 2-byte aligned");
            return Q3K_OK;
        }
    } // namespace

    // In-place generic RMSNorm (y = x), used by the fused Q/K op's fallback.
    int launch_rms_generic(uint16_t *x, const uint16_t *w, int64_t rows, int64_t n, float eps, hipStream_t stream)
    {
        if (rows == 0)
            return Q3K_OK;
        const int64_t blocks = rows < kMaxGenericBlocks ? rows : kMaxGenericBlocks;
        rms_rows_generic_kernel<false><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream>>>(
            x, nullptr, w, x, rows, n, eps);
        return check_launch("rms_norm (generic)");
    }
} // namespace q3k

extern "C" int q3k_rms_norm_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y,
                                 int64_t rows, int64_t N, float eps, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_common(x, w, y, rows, N, eps))
        return st;
    if (rows == 0)
        return Q3K_OK;
    // The fast kernels read x through the h slot; x is never written when ADD is false.
    return rms_dispatch<false>(const_cast<uint16_t *>(x), nullptr, w, y, rows, N, eps,
                               reinterpret_cast<hipStream_t>(stream), "rms_norm");
}

extern "C" int q3k_add_rms_norm_bf16(uint16_t *h, const uint16_t *d, const uint16_t *w,
                                     uint16_t *y, int64_t rows, int64_t N, float eps,
                                     q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_common(h, w, y, rows, N, eps))
        return st;
    if (rows > 0 && d == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "add_rms_norm delta pointer is null");
    if (!aligned_to(d, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm pointers must be 2-byte aligned");
    if (rows == 0)
        return Q3K_OK;
    return rms_dispatch<true>(h, d, w, y, rows, N, eps, reinterpret_cast<hipStream_t>(stream), "add_rms_norm");
}
