// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Fast path (N % 8 == 0, N <= 8192, 16-byte aligned pointers): a group of G
// lanes owns one row and keeps it in registers, so x (and the residual
// delta) is read from HBM exactly once.  Each lane holds VPT 128-bit
// vectors (8 bf16 each); vector j of a row sits in lane j % G, slot j / G, so
// every load instruction of a group reads G * 16 contiguous bytes.  The row
// sum of squares is reduced across the group with DPP (G <= 16) or
// cross-lane shuffles, with no LDS and no barrier.  G = 64 is one wave per
// row (hidden rows of 1024..8192); G = 16 packs four head rows of 128 into a
// wave (per-head Q/K norm).
//
// Generic path (any N, any alignment): one 256-thread block per row, scalar
// loads, two passes over the row (reference structure, wave64 reduction).
//
// Arithmetic follows src/ops/rms_norm.cu:82-121 and
// src/ops/elementwise.cu:28-35: fp32 sum of squares, mean = sum / N,
// inv = 1/sqrt(mean + eps), y = RNE(RNE(x * inv) * w); the fused form adds
// h = RNE(h + d) first and normalises the rounded h.
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        template <int G, int VPT, bool ADD>
        __global__ __launch_bounds__(kBlock) void rms_rows_kernel(
            uint16_t *__restrict__ h, const uint16_t *__restrict__ d,
            const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
            int64_t rows, int nvec, float n_float, float eps)
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
            Vec8 x[VPT];
            Vec8 dv[VPT];
            Vec8 wv[VPT];
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                const int j = lane + i * G;
                if (j < nvec)
                {
                    x[i] = hrow[j];
                    if constexpr (ADD)
                        dv[i] = reinterpret_cast<const Vec8 *>(d)[row_offset + j];
                    wv[i] = wvec[j];
                }
            }

            if constexpr (ADD)
            {
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                {
                    const int j = lane + i * G;
                    if (j < nvec)
                    {
                        Vec8 s;
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            s.d[k] = pack_rne(bf_lo(x[i].d[k]) + bf_lo(dv[i].d[k]),
                                              bf_hi(x[i].d[k]) + bf_hi(dv[i].d[k]));
                        x[i] = s;
                        hrow[j] = s;
                    }
                }
            }

            float partial = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                const int j = lane + i * G;
                if (j < nvec)
                    partial += sum_sq8(x[i]);
            }
            const float total = group_sum<G>(partial);
            const float inv = inverse_rms(total, n_float, eps);

#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                const int j = lane + i * G;
                if (j < nvec)
                    yrow[j] = norm_scale8(x[i], wv[i], inv);
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
            const float n_float = static_cast<float>(n);
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
                const float inv = inverse_rms(block_sum(partial, scratch), n_float, eps);
                for (int64_t c = threadIdx.x; c < n; c += blockDim.x)
                {
                    const float nrm = bf_to_f(f_to_bf(bf_to_f(hr[c]) * inv));
                    yr[c] = f_to_bf(nrm * bf_to_f(w[c]));
                }
            }
        }

        template <int G, int VPT, bool ADD>
        void launch_rows(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                         int64_t rows, int nvec, float n_float, float eps, hipStream_t stream)
        {
            constexpr int kRowsPerBlock = kBlock / G;
            const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
            rms_rows_kernel<G, VPT, ADD><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream>>>(
                h, d, w, y, rows, nvec, n_float, eps);
        }

        template <bool ADD>
        bool launch_fast(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                         int64_t rows, int64_t n, float eps, hipStream_t stream)
        {
            const int nvec = static_cast<int>(n / 8);
            const float nf = static_cast<float>(n);
            if (nvec <= 1)
                launch_rows<1, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream);
            else if (nvec <= 2)
                launch_rows<2, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream);
            else if (nvec <= 4)
                launch_rows<4, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream);
            else if (nvec <= 8)
                launch_rows<8, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream);
            else if (nvec <= 16)
                launch_rows<16, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream);
            else if (nvec <= 32)
                launch_rows<32, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream);
            else
            {
                switch ((nvec + kWave - 1) / kWave)
                {
                case 1: launch_rows<64, 1, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 2: launch_rows<64, 2, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 3: launch_rows<64, 3, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 4: launch_rows<64, 4, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 5: launch_rows<64, 5, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 6: launch_rows<64, 6, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 7: launch_rows<64, 7, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 8: launch_rows<64, 8, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 9: launch_rows<64, 9, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 10: launch_rows<64, 10, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 11: launch_rows<64, 11, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 12: launch_rows<64, 12, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 13: launch_rows<64, 13, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 14: launch_rows<64, 14, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 15: launch_rows<64, 15, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                case 16: launch_rows<64, 16, ADD>(h, d, w, y, rows, nvec, nf, eps, stream); break;
                default: return false;
                }
            }
            return true;
        }

        constexpr int64_t kMaxFastN = 16 * kWave * 8; // 8192 elements per row
        constexpr int64_t kMaxGenericBlocks = 1 << 20;

        template <bool ADD>
        int rms_dispatch(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                         int64_t rows, int64_t n, float eps, hipStream_t stream, const char *name)
        {
            const bool fast = (n % 8 == 0) && n <= kMaxFastN && aligned16(h) && aligned16(w) && aligned16(y) &&
                              (!ADD || aligned16(d)) && rows <= (int64_t{1} << 31);
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
