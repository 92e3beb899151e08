// Causal grouped-query attention for gfx950 (src/ops/gqa_attention.cu:20-155
// of the reference: query [B, S, Hq * D], key/value cache views
// [B, cached, Hkv, D] with strides, query (b, s) attends to keys
// 0 .. start + s, query head h reads KV head h / (Hq / Hkv)).
//
// Matrix-core path (head_dim 128, unit dim stride, 16-byte rows): a block of
// four waves owns one (batch, KV head) and 128 of its (position, head)
// columns, so every K/V tile it stages in LDS serves 128 query rows.  (A
// decode step with its key range split into short slices runs the same code
// as one-wave blocks, one slice each.)  A wave's
// 32 "columns" are consecutive (position, head) pairs in position-major
// order: 32 / G whole positions when G divides 32; any G up to 32 works (for
// Qwen3-14B's 5 a position's heads may straddle two waves).  Per 32 keys:
//   S^T = K Q^T   with v_mfma_f32_32x32x16_bf16: A = K rows from LDS,
//                 B = the wave's Q fragments (registers for the whole loop);
//   online softmax per column: a lane holds one column, so the key max and
//                 sum need only its own registers and the lane 32 apart
//                 (v_permlane32_swap);
//   O^T += V^T P^T: A = V^T read from the row-major V tile with the LDS
//                 transpose read (ds_read_b64_tr_b16), B = P^T straight from
//                 the S^T registers.  P is split into a bf16 high part and a
//                 bf16 remainder (two MFMAs), so the weights keep about 16
//                 significant bits: the reference accumulates p * v in fp32,
//                 and a single bf16 rounding of p would cost up to half an
//                 output ulp.
// Scores are scaled by scale * log2(e) and exponentiated with v_exp_f32.
// Keys go in tiles of 64 (two S^T halves of 32).  A tile's K and V rows go
// from HBM straight into LDS (buffer_load_dwordx4 ... lds, no registers) while
// the previous tile is computed, into the other of two buffers; one barrier
// per tile.  The P V product of a tile is issued in the next tile's step,
// beside that tile's softmax.  One wave's independent MFMA and VALU work can
// overlap on gfx950, but interleaving them within the wave measured slower
// here than leaving the overlap to the other block's wave on the same SIMD
// (two waves per SIMD at this register count).  Tile rows are 256 bytes with
// the 16-byte chunks XOR-swizzled by row so that the K fragment reads
// (ds_read_b128) and the V transpose reads hit distinct LDS banks.  Prefill
// grids are renumbered so that the query blocks of one (batch, KV head) run on
// one XCD and share its L2.
//
// Generic path (any head_dim <= 256, any strides): one wave per query row,
// keys in order, lanes over the head dimension -- the reference's own
// structure with wave reductions.
#include <type_traits>

#include "dispatch.hpp"
#include "q3k_common.hpp"

namespace q3k
{
    namespace
    {
        typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
        typedef float f32x16_t __attribute__((ext_vector_type(16)));

        typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;
        typedef __attribute__((address_space(3))) void lds_void_t;

        constexpr int kAttD = kAttHeadDim;
        constexpr int kKeyTile = kAttKeyTile;                 // keys per pipeline step
        constexpr int kRowBytes = kAttD * 2;                  // one K or V row in LDS
        constexpr int kHalfBytes = kKeyTile * kRowBytes;      // the K (or V) rows of a tile
        constexpr int kRowsPerLoad = kWave * 16 / kRowBytes;  // rows one wave-wide 16-byte load fills
        constexpr int kAhead = 2;                             // LDS fragment reads in flight ahead of use
        constexpr float kLazyMax = 8.0f;                      // log2 headroom before the softmax reference moves
        constexpr int kAttWaves = kAttWavesPerBlock;          // waves per matrix-core block
        constexpr int kAttBlock = kAttWaves * kWave;
        constexpr float kLog2e = 1.4426950408889634f;

        struct AttnArgs
        {
            const uint16_t *q;
            const uint16_t *k;
            const uint16_t *v;
            uint16_t *out;
            int64_t S;
            int64_t start;
            int64_t ks0, ks1, ks2, ks3;
            int64_t vs0, vs1, vs2, vs3;
            int32_t Hq;
            int32_t Hkv;
            int32_t D;
            int32_t qblocks;
            float scale;
            // split-K: the key range is cut into `splits` slices of split_keys
            // keys (a multiple of the tile); slice results (unnormalised O^T,
            // reference max and sum) go to part_o [splits, rows, D] and part_ml
            // [splits, rows, 2] and attn_combine_kernel merges them
            int32_t splits;
            int32_t split_keys;
            float *part_o;
            float *part_ml;
            int64_t rows;
        };

        __device__ __forceinline__ bf16x8_t as_bf8(const Vec8 &v) { return __builtin_bit_cast(bf16x8_t, v); }

        // LDS chunk (16 bytes) holding chunk c of K row r / V row r of a tile.
        // K: lanes 0..31 of a fragment read read rows r..r+31 at one chunk;
        // any 16 consecutive rows put it in 16 different chunk positions.
        // V: a transpose read takes 4 rows x 32 bytes per 16 lanes; rows
        // 4 apart share a bank set.
        __device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
        __device__ __forceinline__ int v_slot(int r, int c) { return c ^ (4 * (r & 3)); }

        // Buffer resource over [base, base + 2 GiB): raw (stride 0), so the
        // offsets the loads give are byte offsets from base.
        __device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void *base)
        {
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7fffffff, 0x00020000);
        }

        // 16 bytes per lane from rsrc + voffset into LDS at lds_wave + 16 * lane
        // (buffer_load_dwordx4 ... lds: no registers, the wave's LDS base in M0)
        __device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, int32_t voffset, unsigned char *lds_wave)
        {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)lds_wave, 16, voffset, 0, 0, 0);
        }

        // Renumbers workgroup ids so that the ids one XCD receives (id % kXcds
        // == x, in dispatch order) become the contiguous range of the x-th
        // share of the grid.
        constexpr unsigned kXcds = 8;
        __device__ __forceinline__ int xcd_contiguous(unsigned id, unsigned n)
        {
            const unsigned x = id % kXcds, k = id / kXcds, q = n / kXcds, r = n % kXcds;
            return static_cast<int>(x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k);
        }

        // max / sum of x over lanes l and l ^ 32, in every lane (one VALU swap,
        // no LDS): after the swap one operand is x and the other its partner
        __device__ __forceinline__ float pair_max(float x)
        {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
            return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
        }
        __device__ __forceinline__ float pair_sum(float x)
        {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
            return __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }

        // ---- tile operations shared by the kernels ------------------------------

        // Loading a key tile's K (or V) rows into LDS from a block of WAVES
        // waves: wave w fills rows (kKeyTile / WAVES) w .. of a buffer,
        // kRowsPerLoad rows per load; lane j lands in slot j % 16 of row j / 16
        // and so fetches the chunk that slot holds.  A tile's loads address from
        // a buffer resource based at its first key, so the per-lane byte offsets
        // (tile_offsets) stay fixed: 32-bit, checked by the launcher.  Rows past
        // n_keys repeat the last key (finite data, later masked or weighted by
        // zero).
        template <int WAVES>
        struct Staging
        {
            static constexpr int kRows = kKeyTile / WAVES;      // rows of a tile per wave
            static constexpr int kLoads = kRows / kRowsPerLoad; // loads per wave per K (or V) tile
        };

        template <int WAVES, typename Slot>
        __device__ __forceinline__ void tile_offsets(int wave, int lane, int32_t byte_stride, Slot slot,
                                                     int32_t (&voff)[Staging<WAVES>::kLoads])
        {
            const int st_row = Staging<WAVES>::kRows * wave + lane / 16;
#pragma unroll
            for (int x = 0; x < Staging<WAVES>::kLoads; ++x)
            {
                const int r = st_row + kRowsPerLoad * x;
                voff[x] = r * byte_stride + 16 * slot(r, lane % 16);
            }
        }

        template <int WAVES, typename Slot>
        __device__ __forceinline__ void load_tile_rows(int tile, unsigned char *buf, const uint16_t *base,
                                                       int64_t row_stride, int32_t byte_stride, int32_t n_keys,
                                                       int wave, int lane, const int32_t (&voff)[Staging<WAVES>::kLoads],
                                                       Slot slot)
        {
            constexpr int kRows = Staging<WAVES>::kRows;
            const int32_t key0 = tile * kKeyTile;
            const __amdgpu_buffer_rsrc_t rs = tile_rsrc(base + static_cast<int64_t>(key0) * row_stride);
            unsigned char *dst = buf + kRows * wave * kRowBytes;
            if (key0 + kKeyTile <= n_keys)
            {
#pragma unroll
                for (int x = 0; x < Staging<WAVES>::kLoads; ++x)
                    dma16(rs, voff[x], dst + kRowsPerLoad * x * kRowBytes);
            }
            else
            {
                const int last = n_keys - 1 - key0;
                const int st_row = kRows * wave + lane / 16;
#pragma unroll
                for (int x = 0; x < Staging<WAVES>::kLoads; ++x)
                {
                    const int r = st_row + kRowsPerLoad * x;
                    const int rr = r < last ? r : last;
                    dma16(rs, rr * byte_stride + 16 * slot(r, lane % 16), dst + kRowsPerLoad * x * kRowBytes);
                }
            }
        }

        // both halves of the staging for one kernel: K and V bases, strides and
        // the per-lane offsets, as lambdas over the kernel's locals
#define Q3K_ATTN_STAGING(WAVES)                                                                                      \
    const uint16_t *kbase = a.k + b * a.ks0 + kvh * a.ks2;                                                            \
    const uint16_t *vbase = a.v + b * a.vs0 + kvh * a.vs2;                                                            \
    const int32_t kstride = static_cast<int32_t>(a.ks1) * 2, vstride = static_cast<int32_t>(a.vs1) * 2;               \
    const auto kslot = [](int r, int c) __attribute__((always_inline)) { return k_slot(r, c); };                                                     \
    const auto vslot = [](int r, int c) __attribute__((always_inline)) { return v_slot(r, c); };                                                     \
    int32_t k_voff[Staging<WAVES>::kLoads], v_voff[Staging<WAVES>::kLoads];                                           \
    tile_offsets<WAVES>(wave, lane, kstride, kslot, k_voff);                                                          \
    tile_offsets<WAVES>(wave, lane, vstride, vslot, v_voff);                                                          \
    auto load_k = [&](int tile, unsigned char *buf) __attribute__((always_inline)) {                                                                 \
        load_tile_rows<WAVES>(tile, buf, kbase, a.ks1, kstride, n_keys, wave, lane, k_voff, kslot);                   \
    };                                                                                                                \
    auto load_v = [&](int tile, unsigned char *buf) __attribute__((always_inline)) {                                                                 \
        load_tile_rows<WAVES>(tile, buf, vbase, a.vs1, vstride, n_keys, wave, lane, v_voff, vslot);                   \
    };

        // Q fragments of the lane's column.  A padding column (s_col >= S) reads
        // the last position's row instead: its scores are always masked (a wave
        // holding one is a partial wave), so only finiteness matters.
        __device__ __forceinline__ void load_q(const AttnArgs &a, int64_t b, int32_t s_col, int h_col, bool col_ok,
                                               int lg, bf16x8_t (&qf)[kAttD / 16])
        {
            const int64_t s_row = col_ok ? s_col : a.S - 1;
            const Vec8 *qrow = reinterpret_cast<const Vec8 *>(a.q + ((b * a.S + s_row) * a.Hq + h_col) * kAttD);
#pragma unroll
            for (int c = 0; c < kAttD / 16; ++c)
                qf[c] = as_bf8(qrow[2 * c + lg]);
        }

        // Per-lane LDS byte offsets of the V transpose reads: the lanes of each
        // 16 give rows 4 lg + j / 4 (+ 8 per 8-key step) and 4 dims
        // 32 dt + 16 ((lane / 16) % 2) + 4 (j % 4) .. + 3, and each lane gets 4
        // consecutive keys of one dim (dim 32 dt + lane % 32).
        __device__ __forceinline__ void v_offsets(int lane, int (&v_off)[kAttD / 32])
        {
            const int tj = lane % 16, lg = lane / 32;
            const int v_row = 4 * lg + tj / 4;
#pragma unroll
            for (int dt = 0; dt < kAttD / 32; ++dt)
                v_off[dt] = v_row * kRowBytes + 16 * v_slot(v_row, 4 * dt + 2 * ((lane / 16) % 2) + (tj % 4) / 2) +
                            8 * (tj % 2);
        }

        // S^T = K Q^T for the 64 keys of a tile (sacc[hh]: keys 32 hh .. + 31).
        // The K fragment reads run kAhead steps ahead of the MFMAs that use them.
        __device__ __forceinline__ void qk_tile(const unsigned char *k_lds, const bf16x8_t (&qf)[kAttD / 16], int li,
                                                int lg, f32x16_t (&sacc)[2])
        {
            auto read_k = [&](int c, int hh) __attribute__((always_inline)) {
                return *reinterpret_cast<const Vec8 *>(k_lds + (32 * hh + li) * kRowBytes +
                                                       16 * k_slot(li, 2 * c + lg));
            };
            sacc[0] = f32x16_t{};
            sacc[1] = f32x16_t{};
            Vec8 kq[kAhead + 1][2];
#pragma unroll
            for (int c = 0; c < kAhead; ++c)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
                    kq[c][hh] = read_k(c, hh);
#pragma unroll
            for (int c = 0; c < kAttD / 16; ++c)
            {
                if (c + kAhead < kAttD / 16)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        kq[(c + kAhead) % (kAhead + 1)][hh] = read_k(c + kAhead, hh);
                __builtin_amdgcn_sched_barrier(0); // keep the reads ahead of these MFMAs
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
                    sacc[hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(kq[c % (kAhead + 1)][hh]), qf[c], sacc[hh],
                                                                       0, 0, 0);
            }
        }

        // Scores of keys past the column's causal limit and of padding columns
        // become -inf (before the max).
        __device__ __forceinline__ void mask_tile(f32x16_t (&sacc)[2], int32_t key0, int lg, int32_t last_key,
                                                  bool col_ok)
        {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int32_t kk = key0 + 32 * hh + 8 * (r / 4) + 4 * lg + (r % 4);
                    if (kk > last_key || !col_ok)
                        sacc[hh][r] = -__builtin_huge_valf();
                }
        }

        // Online softmax of one tile for the lane's column: the weights, split
        // into bf16 high parts and remainders, go to phi / plo, and m, l are
        // updated.  The weights are taken relative to a reference m that moves
        // only when a tile's max exceeds it by more than kLazyMax (log2 units):
        // they stay below 2^kLazyMax, and the rescale of the output is left for
        // the rare tiles that move it.  Returns that rescale factor (1 when m did
        // not move).  An all-masked column keeps m = -inf and weight 0.  The max
        // of the raw scores times the (positive) scale is the max of the scaled
        // ones.
        __device__ __forceinline__ float softmax_tile(const f32x16_t (&sacc)[2], float scale2, float &m, float &l,
                                                      bf16x8_t (&phi)[2][2], bf16x8_t (&plo)[2][2])
        {
            float mloc = sacc[0][0];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    mloc = fmaxf(mloc, sacc[hh][r]);
            mloc = pair_max(mloc);
            const float m_tile = mloc * scale2;
            const bool move = m_tile > m + kLazyMax;
            const float m_new = move ? m_tile : m;
            const float m_use = m_new == -__builtin_huge_valf() ? 0.0f : m_new;
            const float alpha = move ? __builtin_amdgcn_exp2f(m - m_use) : 1.0f;
            float psum = 0.0f;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int mm = 0; mm < 2; ++mm)
                {
                    Vec8 h8, l8;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                    {
                        const float x0 =
                            __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[hh][8 * mm + 2 * j], scale2, -m_use));
                        const float x1 =
                            __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[hh][8 * mm + 2 * j + 1], scale2, -m_use));
                        psum += x0;
                        psum += x1;
                        const uint32_t hp = pack_rne(x0, x1);
                        h8.d[j] = hp;
                        l8.d[j] = pack_rne(x0 - bf_lo(hp), x1 - bf_hi(hp));
                    }
                    phi[hh][mm] = as_bf8(h8);
                    plo[hh][mm] = as_bf8(l8);
                }
            psum = pair_sum(psum);
            l = l * alpha + psum;
            m = m_new;
            return alpha;
        }

        // o *= alpha; multiplying by alpha == 1 changes nothing, so the wave
        // skips it when no lane needs it
        __device__ __forceinline__ void rescale(f32x16_t (&o)[kAttD / 32], float alpha)
        {
            if (__any(alpha != 1.0f))
            {
#pragma unroll
                for (int dt = 0; dt < kAttD / 32; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        o[dt][r] *= alpha;
            }
        }

        // O^T += V^T P^T for one tile: step i covers the 16-key chunk i / 4
        // (hh = i / 8, mm = (i / 4) % 2) and dims 32 (i % 4) .. + 31.  The
        // transpose reads run kAhead steps ahead of the MFMAs that use them.
        __device__ __forceinline__ void pv_tile(const unsigned char *v_lds, const int (&v_off)[kAttD / 32],
                                                const bf16x8_t (&phi)[2][2], const bf16x8_t (&plo)[2][2],
                                                f32x16_t (&o)[kAttD / 32])
        {
            auto read_v = [&](int i) __attribute__((always_inline)) {
                // keys 16 (i / 4) + 8 t + 4 lg + 0..3 in elements 4 t .. 4 t + 3:
                // the keys of the P^T elements this lane holds
                const unsigned char *vp = v_lds + v_off[i % 4] + 16 * (i / 4) * kRowBytes;
                const bf16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t *)(vp));
                const bf16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t *)(vp + 8 * kRowBytes));
                return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            };
            bf16x8_t vq[kAhead + 1];
#pragma unroll
            for (int i = 0; i < kAhead; ++i)
                vq[i] = read_v(i);
#pragma unroll
            for (int i = 0; i < 16; ++i)
            {
                if (i + kAhead < 16)
                    vq[(i + kAhead) % (kAhead + 1)] = read_v(i + kAhead);
                __builtin_amdgcn_sched_barrier(0); // keep the reads ahead of these MFMAs
                const int dt = i % 4, hh = i / 8, mm = (i / 4) % 2;
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vq[i % (kAhead + 1)], phi[hh][mm], o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vq[i % (kAhead + 1)], plo[hh][mm], o[dt], 0, 0, 0);
            }
        }

        // The lane's column of the result: bf16 O / l, or with split keys the
        // slice's unnormalised O^T, reference max and sum for the merge.
        __device__ __forceinline__ void store_column(const AttnArgs &a, int sp, int64_t b, int32_t s_col, int h_col,
                                                     int lg, const f32x16_t (&o)[kAttD / 32], float m, float l)
        {
            if (a.splits > 1)
            {
                const int64_t slot = static_cast<int64_t>(sp) * a.rows + (b * a.S + s_col) * a.Hq + h_col;
                float *po = a.part_o + slot * kAttD;
#pragma unroll
                for (int dt = 0; dt < kAttD / 32; ++dt)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4)
                    {
                        const float4 w = {o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]};
                        *reinterpret_cast<float4 *>(po + dt * 32 + 8 * q4 + 4 * lg) = w;
                    }
                if (lg == 0)
                {
                    a.part_ml[2 * slot] = m;
                    a.part_ml[2 * slot + 1] = l;
                }
                return;
            }
            const float inv = 1.0f / l;
            uint16_t *orow = a.out + ((b * a.S + s_col) * a.Hq + h_col) * kAttD;
#pragma unroll
            for (int dt = 0; dt < kAttD / 32; ++dt)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                {
                    const int d = dt * 32 + 8 * q4 + 4 * lg;
                    uint2 w;
                    w.x = pack_rne(o[dt][4 * q4] * inv, o[dt][4 * q4 + 1] * inv);
                    w.y = pack_rne(o[dt][4 * q4 + 2] * inv, o[dt][4 * q4 + 3] * inv);
                    *reinterpret_cast<uint2 *>(orow + d) = w;
                }
        }

        // ---- the matrix-core kernel ---------------------------------------------

        // G is the group size Hq / Hkv, or 0 for a group size that does not
        // divide 32 (taken from the arguments at run time).  The S * G columns
        // of one (batch, KV head), (position, head) pairs in position-major
        // order, go 32 to a wave and 32 * WAVES to a block; for a G that
        // divides 32 a wave thus holds 32 / G whole positions, otherwise a
        // position's heads may straddle two waves or blocks.
        template <int G, int WAVES>
        __global__ __launch_bounds__(WAVES * kWave) void attn_mfma_kernel(AttnArgs a)
        {
            const int g = G > 0 ? G : a.Hq / a.Hkv;
            constexpr int kBlockCols = 32 * WAVES;
            // K and V tiles, two buffers each.  Tile t's P V product is issued in
            // step t + 1, beside the softmax of tile t + 1, so V(t) stays resident
            // one step longer than K(t); V(t + 1) is loaded into V(t - 1)'s buffer
            // once every wave has passed the barrier that ends step t.  The four
            // buffers are separate objects and the loop below names them
            // statically, so the compiler can tell that the LDS reads of a step do
            // not depend on the loads in flight.
            __shared__ __attribute__((aligned(16))) unsigned char k_a[kHalfBytes];
            __shared__ __attribute__((aligned(16))) unsigned char k_b[kHalfBytes];
            __shared__ __attribute__((aligned(16))) unsigned char v_a[kHalfBytes];
            __shared__ __attribute__((aligned(16))) unsigned char v_b[kHalfBytes];

            const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
            const int lane = threadIdx.x % kWave;
            const int li = lane % 32, lg = lane / 32;

            // block -> (key slice, batch, KV head, query block); the longest query
            // blocks go first.  Workgroups are dealt to the XCDs in turn; when
            // several query blocks read the same keys, block ids are renumbered to
            // give each XCD a contiguous run, so the query blocks of one (batch,
            // KV head) share that XCD's L2.  (Decode blocks share nothing and keep
            // the plain order, which spreads each batch row over the XCDs.)
            int bid = a.qblocks > 1 ? xcd_contiguous(blockIdx.x, gridDim.x) : static_cast<int>(blockIdx.x);
            const int sp = bid % a.splits;
            bid /= a.splits;
            const int qb = a.qblocks - 1 - bid % a.qblocks;
            bid /= a.qblocks;
            const int kvh = bid % a.Hkv;
            const int64_t b = bid / a.Hkv;
            // positions, columns and key indices fit in 32 bits (checked by the
            // launcher: B * S * Hq < 2^31)
            const int32_t S = static_cast<int32_t>(a.S), start = static_cast<int32_t>(a.start);
            const int32_t n_cols = S * g;
            const int64_t block_col = static_cast<int64_t>(qb) * kBlockCols;
            const int32_t block_end = static_cast<int32_t>(block_col + kBlockCols < n_cols ? block_col + kBlockCols : n_cols);
            const int32_t s_last = (block_end - 1) / g;
            const int32_t n_keys = start + s_last + 1;
            // this block's key slice [sp * split_keys, ...) within the causal range
            const int32_t k_begin = sp * a.split_keys;
            const int32_t k_end = n_keys < k_begin + a.split_keys ? n_keys : k_begin + a.split_keys;
            const int tile_begin = k_begin / kKeyTile;
            const int ntiles = k_end > k_begin ? (k_end + kKeyTile - 1) / kKeyTile : tile_begin;

            // this lane's column
            const int64_t wave_col = block_col + 32 * wave;
            const int64_t col = wave_col + li;
            const int32_t wave_s0 = static_cast<int32_t>(wave_col / g);  // the wave's first position
            const int32_t s_col = static_cast<int32_t>(col / g);
            const int h_col = kvh * g + static_cast<int>(col % g);
            const bool col_ok = col < n_cols;
            const int32_t last_key = start + s_col;
            const bool wave_active = wave_col < n_cols;
            const bool wave_partial = wave_col + 32 > n_cols;

            bf16x8_t qf[kAttD / 16];
            load_q(a, b, s_col, h_col, col_ok, lg, qf);
            Q3K_ATTN_STAGING(WAVES)
            int v_off[kAttD / 32];
            v_offsets(lane, v_off);
            f32x16_t o[kAttD / 32];
#pragma unroll
            for (int dt = 0; dt < kAttD / 32; ++dt)
                o[dt] = f32x16_t{};
            float m = -__builtin_huge_valf(), l = 0.0f;
            const float scale2 = a.scale * kLog2e;
            bf16x8_t phi[2][2], plo[2][2]; // P of the tile whose P V is still to be issued

            // One step: load K(tile + 1); S^T = K(tile) Q^T; the P V of the
            // previous tile (WITH_PV); this tile's softmax; after the barrier,
            // load V(tile + 1) into v_prev.
            auto step = [&](auto with_pv, int tile, const unsigned char *k_cur, unsigned char *k_next,
                            unsigned char *v_prev) __attribute__((always_inline)) {
                if (tile + 1 < ntiles)
                    load_k(tile + 1, k_next); // in flight while this tile is computed
                if (wave_active)
                {
                    const int32_t key0 = tile * kKeyTile;
                    f32x16_t sacc[2];
                    // The matrix phase (S = K Q^T, then the previous tile's P V)
                    // runs at raised wave priority, the softmax at the default:
                    // the other block's wave on the SIMD then interleaves its
                    // VALU work instead of competing for issue with the MFMAs
                    // (prefill 4% faster at config 4, decode unchanged).
                    __builtin_amdgcn_s_setprio(1);
                    qk_tile(k_cur, qf, li, lg, sacc);
                    if (key0 + kKeyTile - 1 > start + wave_s0 || wave_partial)
                        mask_tile(sacc, key0, lg, last_key, col_ok);
                    if constexpr (decltype(with_pv)::value)
                        pv_tile(v_prev, v_off, phi, plo, o);
                    __builtin_amdgcn_s_setprio(0);
                    const float alpha = softmax_tile(sacc, scale2, m, l, phi, plo);
                    // o holds the tiles before this one at the previous reference
                    rescale(o, alpha);
                }
                // this wave's loads of K(tile + 1) and V(tile) have landed; after the
                // barrier all have, and every wave is done with K(tile) and V(tile - 1)
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                if (tile + 1 < ntiles)
                    load_v(tile + 1, v_prev);
            };
            using no_pv = std::integral_constant<bool, false>;
            using with_pv = std::integral_constant<bool, true>;
            if (tile_begin < ntiles)
            {
                load_k(tile_begin, k_a);
                load_v(tile_begin, v_a);
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                // V(t) sits in v_a when t - tile_begin is even, else in v_b
                step(no_pv{}, tile_begin, k_a, k_b, v_b);
                for (int tile = tile_begin + 1; tile < ntiles; tile += 2)
                {
                    step(with_pv{}, tile, k_b, k_a, v_a);
                    if (tile + 1 < ntiles)
                        step(with_pv{}, tile + 1, k_a, k_b, v_b);
                }
                if (wave_active)
                {
                    if ((ntiles - 1 - tile_begin) % 2 == 0)
                        pv_tile(v_a, v_off, phi, plo, o);
                    else
                        pv_tile(v_b, v_off, phi, plo, o);
                }
            }
            if (col_ok)
                store_column(a, sp, b, s_col, h_col, lg, o, m, l);
        }

        // Merges the key slices of one query row per block of four waves
        // (splits <= kMaxSplits).  Every load is issued before any is used:
        // lane s of each wave reads slice s's reference max and sum, and wave
        // w the unnormalised O^T of slices w, w + 4, ...  Weights
        // 2^(m_s - max m) (the maxima are in the log2 domain), then
        // sum_s w_s O_s / sum_s w_s l_s; lane t holds dims 2t, 2t + 1, and the
        // four waves' partial sums meet in LDS.
        constexpr int kMaxSplits = kAttMaxSplits;
        constexpr int kCombineWaves = 4;
        constexpr int kSplitsPerWave = kMaxSplits / kCombineWaves;

        __global__ __launch_bounds__(kCombineWaves * kWave) void attn_combine_kernel(const float *__restrict__ part_o,
                                                                                      const float *__restrict__ part_ml,
                                                                                      uint16_t *__restrict__ out,
                                                                                      int64_t rows, int32_t splits)
        {
            __shared__ float2 wave_acc[kCombineWaves][kWave];
            const int64_t row = blockIdx.x;
            const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
            const int lane = threadIdx.x % kWave;
            float2 ml = make_float2(-__builtin_huge_valf(), 0.0f);
            if (lane < splits)
                ml = reinterpret_cast<const float2 *>(part_ml)[static_cast<int64_t>(lane) * rows + row];
            float2 v[kSplitsPerWave];
#pragma unroll
            for (int u = 0; u < kSplitsPerWave; ++u)
            {
                const int sp = wave + kCombineWaves * u;
                if (sp < splits)
                    v[u] = reinterpret_cast<const float2 *>(part_o + (static_cast<int64_t>(sp) * rows + row) * kAttD)[lane];
            }
            float mx = ml.x;
#pragma unroll
            for (int off = kWave / 2; off > 0; off /= 2)
                mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
            const float w = lane < splits ? __builtin_amdgcn_exp2f(ml.x - mx) : 0.0f;
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int u = 0; u < kSplitsPerWave; ++u)
            {
                const int sp = wave + kCombineWaves * u;
                if (sp < splits)
                {
                    const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), sp));
                    a0 += ws * v[u].x;
                    a1 += ws * v[u].y;
                }
            }
            wave_acc[wave][lane] = make_float2(a0, a1);
            const float lsum = group_sum<kWave>(w * ml.y);
            __syncthreads();
            if (wave == 0)
            {
                float2 t = wave_acc[0][lane];
#pragma unroll
                for (int k = 1; k < kCombineWaves; ++k)
                {
                    t.x += wave_acc[k][lane].x;
                    t.y += wave_acc[k][lane].y;
                }
                const float inv = 1.0f / lsum;
                reinterpret_cast<uint32_t *>(out + row * kAttD)[lane] = pack_rne(t.x * inv, t.y * inv);
            }
        }

        // Generic path: one wave per query row (b, s, h); lane t holds head
        // dims t, t + 64, ... (head_dim <= 256); keys in order with the online
        // softmax of the reference.
        __global__ __launch_bounds__(kBlock) void attn_generic_kernel(AttnArgs a, int64_t rows)
        {
            const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) +
                                __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
            if (row >= rows)
                return;
            const int lane = threadIdx.x % kWave;
            const int h = static_cast<int>(row % a.Hq);
            const int64_t bs = row / a.Hq;
            const int64_t s = bs % a.S, b = bs / a.S;
            const int kvh = h / (a.Hq / a.Hkv);
            const int D = a.D;
            float qv[4], acc[4];
#pragma unroll
            for (int x = 0; x < 4; ++x)
            {
                const int d = lane + 64 * x;
                qv[x] = d < D ? bf_to_f(a.q[row * D + d]) : 0.0f;
                acc[x] = 0.0f;
            }
            const uint16_t *kb = a.k + b * a.ks0 + kvh * a.ks2;
            const uint16_t *vb = a.v + b * a.vs0 + kvh * a.vs2;
            float m = -__builtin_huge_valf(), l = 0.0f;
            const int64_t vis = a.start + s + 1;
            for (int64_t j = 0; j < vis; ++j)
            {
                float part = 0.0f;
#pragma unroll
                for (int x = 0; x < 4; ++x)
                {
                    const int d = lane + 64 * x;
                    if (d < D)
                        part = __builtin_fmaf(qv[x], bf_to_f(kb[j * a.ks1 + d * a.ks3]), part);
                }
                const float score = group_sum<64>(part) * a.scale;
                const float nm = fmaxf(m, score);
                const float ow = __expf(m - nm);
                const float nw = __expf(score - nm);
                l = __builtin_fmaf(l, ow, nw);
#pragma unroll
                for (int x = 0; x < 4; ++x)
                {
                    const int d = lane + 64 * x;
                    if (d < D)
                        acc[x] = __builtin_fmaf(bf_to_f(vb[j * a.vs1 + d * a.vs3]), nw, acc[x] * ow);
                }
                m = nm;
            }
#pragma unroll
            for (int x = 0; x < 4; ++x)
            {
                const int d = lane + 64 * x;
                if (d < D)
                    a.out[row * D + d] = f_to_bf(acc[x] / l);
            }
        }

        template <int G>
        int launch_mfma(AttnArgs a, int64_t B, int waves, hipStream_t stream)
        {
            const int64_t cols = a.S * (a.Hq / a.Hkv), block_cols = 32 * kAttWaves;
            a.qblocks = static_cast<int32_t>((cols + block_cols - 1) / block_cols);
            const int64_t blocks = B * a.Hkv * a.qblocks * a.splits;
            if (!launch_fits(blocks, kAttBlock) || (a.splits > 1 && !launch_fits(a.rows, kCombineWaves * kWave)))
                return set_error(Q3K_ERR_OVERFLOW, "GQA grid is too large");
            if (waves == 1)
            {
                // one query position (at most 32 columns) per block either way, so the grid is the same
                static_assert(G == 0 || 32 / G >= 1, "one position per wave at least");
                attn_mfma_kernel<G, 1><<<dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0, stream>>>(a);
            }
            else
                attn_mfma_kernel<G, kAttWaves><<<dim3(static_cast<unsigned>(blocks)), dim3(kAttBlock), 0, stream>>>(a);
            if (a.splits > 1)
                attn_combine_kernel<<<dim3(static_cast<unsigned>(a.rows)), dim3(kCombineWaves * kWave), 0, stream>>>(
                    a.part_o, a.part_ml, a.out, a.rows, a.splits);
            return check_launch("grouped_query_attention");
        }
    } // namespace
} // namespace q3k

extern "C" int q3k_gqa_attention_bf16(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                      uint16_t *out, int64_t B, int64_t S, int32_t Hq, int32_t Hkv, int32_t D,
                                      int64_t cached, int64_t start, const int64_t *k_strides,
                                      const int64_t *v_strides, void *workspace, int64_t workspace_bytes,
                                      q3k_stream_t stream)
{
    using namespace q3k;
    if (B < 0 || S < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA batch and sequence sizes cannot be negative");
    if (Hq <= 0 || Hkv <= 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA head counts must be positive");
    if (Hq % Hkv != 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA query heads must be divisible by key/value heads");
    if (D <= 0 || D > 256)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA head_dim must be between 1 and 256");
    if (start < 0)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA start_position cannot be negative");
    if (start > cached || S != cached - start)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA cache length must equal start_position + sequence_length");
    if (B == 0 || S == 0)
        return Q3K_OK;
    if (k_strides == nullptr || v_strides == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA stride arrays are null");
    for (int i = 0; i < 4; ++i)
        if (k_strides[i] < 0 || v_strides[i] < 0)
            return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA cache strides cannot be negative");
    if (q == nullptr || k_cache == nullptr || v_cache == nullptr || out == nullptr)
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA received a null pointer");
    if (!aligned_to(q, 2) || !aligned_to(k_cache, 2) || !aligned_to(v_cache, 2) || !aligned_to(out, 2))
        return set_error(Q3K_ERR_INVALID_ARGUMENT, "GQA pointers must be 2-byte aligned");
    if (S > INT64_MAX / B || B * S > INT64_MAX / Hq || B * S * Hq > INT32_MAX)
        return set_error(Q3K_ERR_OVERFLOW, "GQA grid is too large");

    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    AttnArgs a{q,
               k_cache,
               v_cache,
               out,
               S,
               start,
               k_strides[0],
               k_strides[1],
               k_strides[2],
               k_strides[3],
               v_strides[0],
               v_strides[1],
               v_strides[2],
               v_strides[3],
               Hq,
               Hkv,
               D,
               0,
               1.0f / __builtin_sqrtf(static_cast<float>(D)),
               1,
               INT32_MAX,
               nullptr,
               nullptr,
               B * S * Hq};
    const AttnPlan plan =
        plan_attention(B, S, Hq, Hkv, D, start, k_strides, v_strides,
                       aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned_to(out, 8),
                       workspace_bytes, workspace != nullptr && aligned16(workspace));
    if (plan.mfma)
    {
        if (plan.split.splits > 1)
        {
            a.splits = plan.split.splits;
            a.split_keys = plan.split.split_keys;
            a.part_o = static_cast<float *>(workspace);
            a.part_ml = a.part_o + static_cast<int64_t>(plan.split.splits) * a.rows * kAttD;
        }
        switch (plan.g_instance)
        {
        case 1: return launch_mfma<1>(a, B, plan.waves, s);
        case 2: return launch_mfma<2>(a, B, plan.waves, s);
        case 4: return launch_mfma<4>(a, B, plan.waves, s);
        case 8: return launch_mfma<8>(a, B, plan.waves, s);
        case 16: return launch_mfma<16>(a, B, plan.waves, s);
        case 32: return launch_mfma<32>(a, B, plan.waves, s);
        default: return launch_mfma<0>(a, B, plan.waves, s);
        }
    }
    const int64_t rows = B * S * Hq;
    const int64_t blocks = blocks_for(rows, kBlock / kWave);
    if (!launch_fits(blocks, kBlock))
        return set_error(Q3K_ERR_OVERFLOW, "GQA grid is too large");
    attn_generic_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s>>>(a, rows);
    return check_launch("grouped_query_attention (generic)");
}

extern "C" int64_t q3k_gqa_attention_workspace_bytes(int64_t B, int64_t S, int32_t Hq, int32_t Hkv, int32_t D,
                                                     int64_t cached)
{
    if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D != q3k::kAttD || cached < S ||
        B * S * Hq > INT32_MAX)
        return 0;
    return q3k::plan_attention_split(B, S, Hq, Hkv, cached).bytes;
}
