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
        // What a launch normalises.  kNorm: y = rms_norm(x); kAddNorm:
        // h = RNE(h + d) written back, y = rms_norm(h); kGatherNorm: the row
        // is table[ids[i]] (zero when the id is outside [0, vocab)), written
        // to h as the residual stream, and y = rms_norm(row).
        enum RowMode
        {
            kNorm = 0,
            kAddNorm = 1,
            kGatherNorm = 2,
        };

        // Output row i (of y, and of h in gather mode) reads input row
        // first + i * stride of h and d; plain launches use first 0, stride 1.
        struct RowMap
        {
            int64_t first;
            int64_t stride;
            const int32_t *ids;
            const uint16_t *table;
            int64_t vocab;
        };

        // Source of output row `out_row`: its input vectors, or nullptr for a
        // gathered row whose id is out of range (the row is zero).
        template <int MODE>
        __device__ __forceinline__ const Vec8 *row_source(const uint16_t *h, const RowMap &map, int64_t out_row,
                                                          int nvec)
        {
            if constexpr (MODE == kGatherNorm)
            {
                const int32_t id = map.ids[out_row];
                if (id < 0 || static_cast<int64_t>(id) >= map.vocab)
                    return nullptr;
                return reinterpret_cast<const Vec8 *>(map.table) + static_cast<int64_t>(id) * nvec;
            }
            else
            {
                return reinterpret_cast<const Vec8 *>(h) + (map.first + out_row * map.stride) * nvec;
            }
        }

        // Where the updated residual of output row `out_row` goes (kAddNorm,
        // kGatherNorm).
        template <int MODE>
        __device__ __forceinline__ Vec8 *residual_row(uint16_t *h, const RowMap &map, int64_t out_row, int nvec)
        {
            if constexpr (MODE == kGatherNorm)
                return reinterpret_cast<Vec8 *>(h) + out_row * nvec;
            else
                return reinterpret_cast<Vec8 *>(h) + (map.first + out_row * map.stride) * nvec;
        }

        // h = RNE(h + d) for the add mode, then the partial sum of squares of
        // the (rounded) values held by this thread.
        template <int VPT, int MODE>
        __device__ __forceinline__ float add_and_square(Vec8 (&x)[VPT], const Vec8 (&dv)[VPT], const bool (&live)[VPT])
        {
            float partial = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                if (!live[i])
                    continue;
                if constexpr (MODE == kAddNorm)
                {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        x[i].d[k] = pack_rne(bf_lo(x[i].d[k]) + bf_lo(dv[i].d[k]), bf_hi(x[i].d[k]) + bf_hi(dv[i].d[k]));
                }
                partial += sum_sq8(x[i]);
            }
            return partial;
        }

        // Loads of one row slice: every x vector first, then d (add mode),
        // then the weights (issuing the HBM streams ahead of the weight reads,
        // which hit the cache, measured faster).  FULL: the slice covers the
        // row exactly, so no vector needs a bounds test.
        template <int VPT, int MODE, int NTM, bool FULL>
        __device__ __forceinline__ void load_row(const Vec8 *src, const uint16_t *d, const RowMap &map, int64_t out_row,
                                                 int nvec, const Vec8 *wvec, int first_vec, int vec_step, Vec8 (&x)[VPT],
                                                 Vec8 (&dv)[VPT], Vec8 (&wv)[VPT], bool (&live)[VPT])
        {
            const Vec8 zero = {{0u, 0u, 0u, 0u}};
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                live[i] = FULL || first_vec + i * vec_step < nvec;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
            {
                if (!live[i])
                    continue;
                const int j = first_vec + i * vec_step;
                if constexpr (MODE == kGatherNorm)
                    x[i] = src != nullptr ? load8<false>(src + j) : zero;
                else
                    x[i] = load8<nt_load(NTM)>(src + j);
            }
            if constexpr (MODE == kAddNorm)
            {
                const Vec8 *drow = reinterpret_cast<const Vec8 *>(d) + (map.first + out_row * map.stride) * nvec;
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                    if (live[i])
                        dv[i] = load8<nt_load(NTM)>(drow + first_vec + i * vec_step);
            }
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (live[i])
                    wv[i] = wvec[first_vec + i * vec_step];
        }

        // Group of G lanes per row (G <= 64), VPT vectors per lane, RPG rows
        // per lane group, BLOCK lanes per block.  The rows of a wave are
        // contiguous: lane group j of wave w takes rows
        // w * (64 / G) * RPG + j + (64 / G) * r, r < RPG, so each load
        // instruction covers 64 / G whole rows.  Every x load (of all RPG rows)
        // is issued first, then d, then the weights once.
        template <int G, int VPT, int RPG, int MODE, int NTM, bool FULL, int BLOCK>
        __global__ __launch_bounds__(BLOCK) void rms_rows_kernel(
            uint16_t *__restrict__ h, const uint16_t *__restrict__ d,
            const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
            int64_t rows, int nvec, float inv_n, float eps, RowMap map)
        {
            constexpr int kGroups = kWave / G;
            const int lane = threadIdx.x % G;
            const int64_t wave = static_cast<int64_t>(blockIdx.x) * (BLOCK / kWave) + threadIdx.x / kWave;
            const int64_t row0 = wave * kGroups * RPG + (threadIdx.x % kWave) / G;
            if (row0 >= rows)
                return;
            const Vec8 zero = {{0u, 0u, 0u, 0u}};
            Vec8 x[RPG][VPT], dv[RPG][VPT], wv[VPT];
            bool live[RPG][VPT];
            const Vec8 *src[RPG];
#pragma unroll
            for (int r = 0; r < RPG; ++r)
            {
                const int64_t row = row0 + kGroups * r;
                src[r] = row < rows ? row_source<MODE>(h, map, row, nvec) : nullptr;
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                    live[r][i] = row < rows && (FULL || lane + i * G < nvec);
            }
#pragma unroll
            for (int r = 0; r < RPG; ++r)
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                {
                    if (!live[r][i])
                        continue;
                    if constexpr (MODE == kGatherNorm)
                        x[r][i] = src[r] != nullptr ? load8<false>(src[r] + lane + i * G) : zero;
                    else
                        x[r][i] = load8<nt_load(NTM)>(src[r] + lane + i * G);
                }
            if constexpr (MODE == kAddNorm)
            {
#pragma unroll
                for (int r = 0; r < RPG; ++r)
                {
                    const Vec8 *drow =
                        reinterpret_cast<const Vec8 *>(d) + (map.first + (row0 + kGroups * r) * map.stride) * nvec;
#pragma unroll
                    for (int i = 0; i < VPT; ++i)
                        if (live[r][i])
                            dv[r][i] = load8<nt_load(NTM)>(drow + lane + i * G);
                }
            }
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (FULL || lane + i * G < nvec)
                    wv[i] = reinterpret_cast<const Vec8 *>(w)[lane + i * G];
#pragma unroll
            for (int r = 0; r < RPG; ++r)
            {
                const int64_t row = row0 + kGroups * r;
                if (row >= rows)
                    continue;
                const float partial = add_and_square<VPT, MODE>(x[r], dv[r], live[r]);
                if constexpr (MODE != kNorm)
                {
                    Vec8 *hrow = residual_row<MODE>(h, map, row, nvec);
#pragma unroll
                    for (int i = 0; i < VPT; ++i)
                        if (live[r][i])
                            store8<nt_store(NTM)>(hrow + lane + i * G, x[r][i]);
                }
                const float inv = inverse_rms(group_sum<G>(partial), inv_n, eps);
                Vec8 *yrow = reinterpret_cast<Vec8 *>(y) + row * nvec;
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                    if (live[r][i])
                        store8<nt_store(NTM)>(yrow + lane + i * G, norm_scale8(x[r][i], wv[i], inv));
            }
        }

        // One row per block of WPR waves, VPT vectors per lane; the wave sums
        // meet in LDS behind one barrier.  PR > 0 raises the wave priority
        // while the loads are issued.
        template <int WPR, int VPT, int MODE, int NTM, int PR, bool REMAP, bool FULL>
        __global__ __launch_bounds__(WPR * kWave) void rms_block_kernel(
            uint16_t *__restrict__ h, const uint16_t *__restrict__ d,
            const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
            int64_t rows, int nvec, float inv_n, float eps, RowMap map)
        {
            constexpr int kThreads = WPR * kWave;
            __shared__ float wave_sums[WPR];
            const int t = threadIdx.x;
            const int64_t row = tile_index<REMAP>(blockIdx.x, gridDim.x);

            Vec8 x[VPT], dv[VPT], wv[VPT];
            bool live[VPT];
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(PR);
            load_row<VPT, MODE, NTM, FULL>(row_source<MODE>(h, map, row, nvec), d, map, row, nvec,
                                           reinterpret_cast<const Vec8 *>(w), t, kThreads, x, dv, wv, live);
            if constexpr (PR > 0)
                __builtin_amdgcn_s_setprio(0);

            const float partial = add_and_square<VPT, MODE>(x, dv, live);
            if constexpr (MODE != kNorm)
            {
                Vec8 *hrow = residual_row<MODE>(h, map, row, nvec);
#pragma unroll
                for (int i = 0; i < VPT; ++i)
                    if (live[i])
                        store8<nt_store(NTM)>(hrow + t + i * kThreads, x[i]);
            }
            float total = group_sum<kWave>(partial);
            if constexpr (WPR > 1)
            {
                if (t % kWave == 0)
                    wave_sums[t / kWave] = total;
                __syncthreads();
                total = 0.0f;
#pragma unroll
                for (int k = 0; k < WPR; ++k)
                    total += wave_sums[k];
            }
            const float inv = inverse_rms(total, inv_n, eps);
            Vec8 *yrow = reinterpret_cast<Vec8 *>(y) + row * nvec;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (live[i])
                    store8<nt_store(NTM)>(yrow + t + i * kThreads, norm_scale8(x[i], wv[i], inv));
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

        // Any width, any alignment: one 256-thread block per row, scalar
        // accesses, two passes over the row.
        template <int MODE>
        __global__ __launch_bounds__(kBlock) void rms_rows_generic_kernel(
            uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
            int64_t rows, int64_t n, float eps, RowMap map)
        {
            __shared__ float scratch[kBlock / kWave];
            const float inv_n = 1.0f / static_cast<float>(n);
            for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
            {
                const uint16_t *src;
                uint16_t *hr;
                bool zero = false;
                if constexpr (MODE == kGatherNorm)
                {
                    const int32_t id = map.ids[row];
                    zero = id < 0 || static_cast<int64_t>(id) >= map.vocab;
                    src = map.table + (zero ? 0 : static_cast<int64_t>(id) * n);
                    hr = h + row * n;
                }
                else
                {
                    hr = h + (map.first + row * map.stride) * n;
                    src = hr;
                }
                const uint16_t *dr = d + (map.first + row * map.stride) * n;
                uint16_t *yr = y + row * n;
                float partial = 0.0f;
                for (int64_t c = threadIdx.x; c < n; c += blockDim.x)
                {
                    float v = zero ? 0.0f : bf_to_f(src[c]);
                    if constexpr (MODE == kAddNorm)
                    {
                        const uint16_t s = f_to_bf(v + bf_to_f(dr[c]));
                        hr[c] = s;
                        v = bf_to_f(s);
                    }
                    else if constexpr (MODE == kGatherNorm)
                    {
                        hr[c] = zero ? uint16_t{0} : src[c];
                    }
                    partial += v * v;
                }
                const float inv = inverse_rms(block_sum(partial, scratch), inv_n, eps);
                for (int64_t c = threadIdx.x; c < n; c += blockDim.x)
                {
                    // reads back the (rounded) residual this thread wrote in pass 1
                    const float x = MODE == kNorm ? bf_to_f(src[c]) : bf_to_f(hr[c]);
                    const float nrm = bf_to_f(f_to_bf(x * inv));
                    yr[c] = f_to_bf(nrm * bf_to_f(w[c]));
                }
            }
        }

        // Non-temporal mode bits (loads | stores), measured on MI355X with
        // input cycles far above the Infinity Cache: non-temporal loads and
        // stores for every row width (128-wide rows, 262144 of them: 75.5%
        // of peak against 73.7% with plain loads; 1024-wide, 65536 rows:
        // 78.2% against 75.3%).  Gathered rows use plain loads (random rows,
        // as in the embedding kernel).
        template <int MODE>
        constexpr int ntm_block() { return MODE == kGatherNorm ? 2 : 3; }
        template <int MODE>
        constexpr int ntm_rows() { return MODE == kGatherNorm ? 2 : 3; }
        // Wave priority while the loads are issued: raised priority helped the
        // fused add while stores were written back from L2 at the end of each
        // kernel; with write-through stores the default is faster (77.7%
        // against 76.3% of peak for add + norm at T = 8192, H = 4096).
        template <int MODE>
        constexpr int prio_block() { return 0; }
        constexpr bool kRemapRows = false;  // XCD-contiguous rows measured slower

        struct Launch
        {
            uint16_t *h;
            const uint16_t *d;
            const uint16_t *w;
            uint16_t *y;
            int64_t rows;
            int nvec;
            float inv_n;
            float eps;
            RowMap map;
            hipStream_t stream;
        };

        // A launch that writes at most kSmallLaunchBytes of y (a decode step)
        // stores with write-through (`sc1`) instead of streaming stores.
        inline bool small_launch(const Launch &l) { return l.rows * l.nvec * 16 <= kSmallLaunchBytes; }

        template <int G, int VPT, int RPG, int MODE, int NTM, int BLOCK>
        void launch_rows_ntm(const Launch &l, const dim3 &grid)
        {
            if (l.nvec == G * VPT)
                rms_rows_kernel<G, VPT, RPG, MODE, NTM, true, BLOCK><<<grid, dim3(BLOCK), 0, l.stream>>>(
                    l.h, l.d, l.w, l.y, l.rows, l.nvec, l.inv_n, l.eps, l.map);
            else
                rms_rows_kernel<G, VPT, RPG, MODE, NTM, false, BLOCK><<<grid, dim3(BLOCK), 0, l.stream>>>(
                    l.h, l.d, l.w, l.y, l.rows, l.nvec, l.inv_n, l.eps, l.map);
        }

        template <int G, int VPT, int RPG, int MODE, int BLOCK = kRmsRowsBlock>
        bool launch_rows_rpg(const Launch &l)
        {
            constexpr int kRowsPerBlock = BLOCK / G * RPG;
            if (!rms_rows_fit(l.rows, G, BLOCK))
                return false;
            const dim3 grid(static_cast<unsigned>(blocks_for(l.rows, kRowsPerBlock)));
            if (small_launch(l))
                launch_rows_ntm<G, VPT, RPG, MODE, ntm_small(ntm_rows<MODE>()), BLOCK>(l, grid);
            else
                launch_rows_ntm<G, VPT, RPG, MODE, ntm_rows<MODE>(), BLOCK>(l, grid);
            return true;
        }

        // Rows per lane group and lanes per block of the plain norm (measured
        // on MI355X, nt loads, rotations past the Infinity Cache).  One row per
        // lane group in one-wave blocks by default: the per-head Q norm of
        // config 4 (262144 128-wide rows) 20.8 against 21.6 us in four-wave
        // blocks.  128-wide rows take four rows per 16-lane group in four-wave
        // blocks for 16384 .. 65536 rows (the K norm of config 4, 65536 rows:
        // 6.56 us, against 6.72-7.08 us for one, two, four or eight rows in
        // one-wave blocks and 7.4 us for one row in four-wave blocks);
        // 1024-wide rows take two per wave in four-wave blocks from 4096 rows
        // (8192 rows: 6.4 against 7.4 us; 65536 rows: equal).  Fewer rows
        // (decode) keep one, for more waves.
        template <int G, int VPT, int MODE>
        bool launch_rows(const Launch &l)
        {
            if constexpr (MODE == kNorm && G == 16 && VPT == 1)
            {
                if (l.rows >= 16384 && l.rows <= 65536)
                    return launch_rows_rpg<G, VPT, 4, MODE, kBlock>(l);
            }
            if constexpr (MODE == kNorm && G == 64 && VPT == 2)
            {
                if (l.rows >= 4096)
                    return launch_rows_rpg<G, VPT, 2, MODE, kBlock>(l);
            }
            return launch_rows_rpg<G, VPT, 1, MODE>(l);
        }

        template <int WPR, int VPT, int MODE, int NTM>
        void launch_block_ntm(const Launch &l)
        {
            const dim3 grid(static_cast<unsigned>(l.rows)), block(WPR * kWave);
            if (l.nvec == WPR * kWave * VPT)
                rms_block_kernel<WPR, VPT, MODE, NTM, prio_block<MODE>(), kRemapRows, true>
                    <<<grid, block, 0, l.stream>>>(l.h, l.d, l.w, l.y, l.rows, l.nvec, l.inv_n, l.eps, l.map);
            else
                rms_block_kernel<WPR, VPT, MODE, NTM, prio_block<MODE>(), kRemapRows, false>
                    <<<grid, block, 0, l.stream>>>(l.h, l.d, l.w, l.y, l.rows, l.nvec, l.inv_n, l.eps, l.map);
        }

        template <int WPR, int VPT, int MODE>
        bool launch_block(const Launch &l)
        {
            if (!rms_block_fits(l.rows, WPR))
                return false;
            if (small_launch(l))
                launch_block_ntm<WPR, VPT, MODE, ntm_small(ntm_block<MODE>())>(l);
            else
                launch_block_ntm<WPR, VPT, MODE, ntm_block<MODE>()>(l);
            return true;
        }

        template <int VPT, int MODE>
        bool launch_block_waves(int waves, const Launch &l)
        {
            switch (waves)
            {
            case 1: return launch_block<1, VPT, MODE>(l);
            case 2: return launch_block<2, VPT, MODE>(l);
            case 3: return launch_block<3, VPT, MODE>(l);
            case 4: return launch_block<4, VPT, MODE>(l);
            case 5: return launch_block<5, VPT, MODE>(l);
            case 6: return launch_block<6, VPT, MODE>(l);
            case 7: return launch_block<7, VPT, MODE>(l);
            case 8: return launch_block<8, VPT, MODE>(l);
            default: return false;
            }
        }

        // Row-to-lane mapping by row width, in 128-bit vectors (measured on MI355X):
        //   nvec <= 32:   a group of pow2 >= nvec lanes per row, several rows per wave
        //                 (per-head norms, 128 elements = 16 lanes);
        //   nvec <= 128:  one wave per row, 1-2 vectors per lane (hidden 1024);
        //   nvec <= 2048: one row per block of up to 8 waves; one vector per lane
        //                 when nvec <= 512 (hidden <= 4096), else two (four
        //                 beyond 8192 elements).  One vector per lane streams
        //                 fastest (a 64 MB row copy: 76.4% of peak with one,
        //                 73.7% with two, 70.8% with eight).
        template <int MODE>
        bool launch_fast(const Launch &l)
        {
            const int nvec = l.nvec;
            if (nvec <= 1)
                return launch_rows<1, 1, MODE>(l);
            else if (nvec <= 2)
                return launch_rows<2, 1, MODE>(l);
            else if (nvec <= 4)
                return launch_rows<4, 1, MODE>(l);
            else if (nvec <= 8)
                return launch_rows<8, 1, MODE>(l);
            else if (nvec <= 16)
                return launch_rows<16, 1, MODE>(l);
            else if (nvec <= 32)
                return launch_rows<32, 1, MODE>(l);
            else if (nvec <= 64)
                return launch_rows<64, 1, MODE>(l);
            else if (nvec <= 128)
                return launch_rows<64, 2, MODE>(l);
            else if (nvec <= 512)
                return launch_block_waves<1, MODE>((nvec + 63) / 64, l);
            else if (nvec <= 1024)
                return launch_block_waves<2, MODE>((nvec + 127) / 128, l);
            else
                return launch_block_waves<4, MODE>((nvec + 255) / 256, l);
        }

        constexpr int64_t kMaxFastN = 8 * kWave * 4 * 8; // 16384 elements per row
        constexpr int64_t kMaxGenericBlocks = 1 << 20;

        template <int MODE>
        int rms_dispatch(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y, int64_t rows, int64_t n,
                         float eps, const RowMap &map, hipStream_t stream, const char *name)
        {
            const bool fast = (n % 8 == 0) && n <= kMaxFastN && aligned16(h) && aligned16(w) && aligned16(y) &&
                              (MODE != kAddNorm || aligned16(d)) && (MODE != kGatherNorm || aligned16(map.table)) &&
                              rows < (int64_t{1} << 31);  // each launcher also checks that its grid fits
            const Launch l{h, d, w, y, rows, static_cast<int>(n / 8), 1.0f / static_cast<float>(n), eps, map, stream};
            if (!(fast && launch_fast<MODE>(l)))
            {
                const int64_t blocks = rows < kMaxGenericBlocks ? rows : kMaxGenericBlocks;
                rms_rows_generic_kernel<MODE><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream>>>(
                    h, d, w, y, rows, n, eps, map);
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

        // Rows first + i * stride, i < count, must lie in [0, INT64_MAX / n).
        // A mode that writes the selected rows back (the residual add) also
        // needs them distinct: with stride 0 every selected row would be one
        // row, updated by several rows of the grid at once.
        int validate_rows(int64_t count, int64_t first, int64_t stride, int64_t n, bool writes_rows)
        {
            if (first < 0 || stride < 0)
                return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm row selection cannot be negative");
            if (writes_rows && stride == 0 && count > 1)
                return set_error(Q3K_ERR_INVALID_ARGUMENT,
                                 "add_rms_norm row stride must be positive when more than one row is selected");
            if (count > 0)
            {
                const int64_t limit = INT64_MAX / n;
                if (stride > 0 && count - 1 > (limit - 1 - first) / stride)
                    return set_error(Q3K_ERR_OVERFLOW, "RMSNorm row selection overflows");
                if (first >= limit)
                    return set_error(Q3K_ERR_OVERFLOW, "RMSNorm row selection overflows");
            }
            return Q3K_OK;
        }

        constexpr RowMap kPlainRows{0, 1, nullptr, nullptr, 0};
    } // namespace

    // In-place generic RMSNorm (y = x), used by the fused Q/K op's fallback.
    int launch_rms_generic(uint16_t *x, const uint16_t *w, int64_t rows, int64_t n, float eps, hipStream_t stream)
    {
        if (rows == 0)
            return Q3K_OK;
        const int64_t blocks = rows < kMaxGenericBlocks ? rows : kMaxGenericBlocks;
        rms_rows_generic_kernel<kNorm><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream>>>(
            x, nullptr, w, x, rows, n, eps, kPlainRows);
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
    // x is read through the h slot and never written in this mode.
    return rms_dispatch<kNorm>(const_cast<uint16_t *>(x), nullptr, w, y, rows, N, eps, kPlainRows,
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
    return rms_dispatch<kAddNorm>(h, d, w, y, rows, N, eps, kPlainRows, reinterpret_cast<hipStream_t>(stream),
                                  "add_rms_norm");
}

extern "C" int q3k_rms_norm_rows_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y, int64_t count,
                                      int64_t first_row, int64_t row_stride, int64_t N, float eps,
                                      q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_common(x, w, y, count, N, eps))
        return st;
    if (const int st = validate_rows(count, first_row, row_stride, N, false))
        return st;
    if (count == 0)
        return Q3K_OK;
    const RowMap map{first_row, row_stride, nullptr, nullptr, 0};
    return rms_dispatch<kNorm>(const_cast<uint16_t *>(x), nullptr, w, y, count, N, eps, map,
                               reinterpret_cast<hipStream_t>(stream), "rms_norm_rows");
}

extern "C" int q3k_add_rms_norm_rows_bf16(uint16_t *h, const uint16_t *d, const uint16_t *w, uint16_t *y,
                                          int64_t count, int64_t first_row, int64_t row_stride, int64_t N,
                                          float eps, q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_common(h, w, y, count, N, eps))
        return st;
    if (const int st = validate_rows(count, first_row, row_stride, N, true))
        return st;
    if (count > 0 && d == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "add_rms_norm delta pointer is null");
    if (!aligned_to(d, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "RMSNorm pointers must be 2-byte aligned");
    if (count == 0)
        return Q3K_OK;
    const RowMap map{first_row, row_stride, nullptr, nullptr, 0};
    return rms_dispatch<kAddNorm>(h, d, w, y, count, N, eps, map, reinterpret_cast<hipStream_t>(stream),
                                  "add_rms_norm_rows");
}

extern "C" int q3k_embedding_rms_norm_bf16(const int32_t *ids, int64_t T, const uint16_t *table, int64_t V,
                                           int64_t H, const uint16_t *w, float eps, uint16_t *hidden, uint16_t *y,
                                           q3k_stream_t stream)
{
    using namespace q3k;
    if (const int st = validate_common(hidden, w, y, T, H, eps))
        return st;
    if (V <= 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding weight dimensions must be positive");
    if (T == 0)
        return Q3K_OK;
    if (ids == nullptr || table == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding received a null pointer");
    if (!aligned_to(ids, 4) || !aligned_to(table, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "embedding pointers must be aligned to their element size");
    if (V > INT64_MAX / H)
        return set_error(Q3K_ERR_OVERFLOW, "embedding size overflows");
    const RowMap map{0, 1, ids, table, V};
    return rms_dispatch<kGatherNorm>(hidden, nullptr, w, y, T, H, eps, map, reinterpret_cast<hipStream_t>(stream),
                                     "embedding_rms_norm");
}
