// Trunk cache build and register-token gather/scatter for gfx950.
//
// Cache build (model/cache.rs:21-52): at the cached layers the trunk
// concatenates the frame- and inter-block outputs channel-wise and casts the
// result to f32, the heads' input (concat_channels.wesl, then
// cast_f16_to_f32.wesl). hs_cache_build does both in one pass: each output
// row is [frame_out row | inter_out row] converted to f32, so every input
// element is read once and every output element written once (the reference
// writes and rereads the f16 concatenation in between). The single ops are
// exported too, as the reference's surface.
//
// Register gather/scatter (model/trunk.rs:103-116): the register-attention
// layers pull the first PREFIX rows of every frame into one (N*PREFIX, D)
// sequence and later write them back, 2*N copy_rows calls in the reference.
// hs_copy_row_blocks moves all N blocks of rows in one launch.
//
// All kernels move 16-byte vectors (the cache build reads through the
// caches and streams its output; the copies stream both); other shapes and
// alignments take scalar loops.
#include "hs_common.hpp"

namespace hs {
namespace {

constexpr int kBlock = 256;
#ifndef HS_CACHE_NTL
#define HS_CACHE_NTL 0  // non-temporal loads of the cache build's inputs
#endif
#ifndef HS_CACHE_NTS
#define HS_CACHE_NTS 1  // non-temporal stores of its f32 output
#endif
#ifndef HS_CACHE_BPC
#define HS_CACHE_BPC 8  // resident workgroups per CU
#endif

int64_t grid_for(int64_t items) {
    const int64_t cap = static_cast<int64_t>(num_cus()) * HS_CACHE_BPC;
    const int64_t blocks = ceil_div(items, kBlock);
    return blocks < 1 ? 1 : (blocks < cap ? blocks : cap);
}

// One 8-element chunk: same type, copied as one (f16) or two (f32) 16-byte
// vectors; f16 -> f32, one 16-byte read widened exactly into two writes.
template <typename TI, typename TO>
__device__ __forceinline__ void copy_chunk(const TI* src, TO* dst) {
    if constexpr (sizeof(TI) == sizeof(TO)) {
        if constexpr (sizeof(TI) == 4) {
            st_stream(dst, ld_stream(src));
            st_stream(dst + 4, ld_stream(src + 4));
        } else {
            st_stream(dst, ld_stream(src));
        }
    } else {
        const u32x4 v = ld_stream<HS_CACHE_NTL != 0>(src);
        u32x4 lo, hi;
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const f16x2 p = u2h2(v[w]), q = u2h2(v[w + 2]);
            lo[2 * w] = f2u(static_cast<float>(p.x)), lo[2 * w + 1] = f2u(static_cast<float>(p.y));
            hi[2 * w] = f2u(static_cast<float>(q.x)), hi[2 * w + 1] = f2u(static_cast<float>(q.y));
        }
        st_stream<HS_CACHE_NTS != 0>(dst, lo);
        st_stream<HS_CACHE_NTS != 0>(dst + 4, hi);
    }
}

#ifndef HS_CACHE_ROWS
#define HS_CACHE_ROWS 1  // rows per workgroup and iteration
#endif
#ifndef HS_CACHE_DESC
#define HS_CACHE_DESC 1  // 1: workgroups take the rows from the last to the first
#endif

// Workgroups stride over rows, R rows per iteration (rows b, b + step, ...,
// b + (R - 1) step for workgroup b, so each thread has R loads in flight);
// threads stride over the row's 8-element chunks, the first cc1 from a and
// the next cc2 from b (cc* = channels / 8). No per-element index division.
template <typename TI, typename TO, int R>
__global__ __launch_bounds__(kBlock) void concat_vec_kernel(const TI* __restrict__ a,
                                                            const TI* __restrict__ b,
                                                            TO* __restrict__ out, int64_t rows,
                                                            int cc1, int cc2) {
    const int cc = cc1 + cc2;
    const int64_t step = static_cast<int64_t>(gridDim.x);
    for (int64_t r0 = blockIdx.x; r0 < rows; r0 += R * step) {
        for (int k = threadIdx.x; k < cc; k += kBlock) {
            const bool left = k < cc1;
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int64_t ri = r0 + i * step;
                if (ri >= rows) break;
                const int64_t r = HS_CACHE_DESC ? rows - 1 - ri : ri;
                const TI* src = left ? a + (r * cc1 + k) * 8 : b + (r * cc2 + (k - cc1)) * 8;
                copy_chunk(src, out + (r * cc + k) * 8);
            }
        }
    }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void concat_scalar_kernel(const TI* a, const TI* b, TO* out,
                                                               int64_t total, int c1, int c2) {
    const int c = c1 + c2;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
         i += stride) {
        const int64_t r = i / c;
        const int k = static_cast<int>(i - r * c);
        const TI x = k < c1 ? a[r * c1 + k] : b[r * c2 + (k - c1)];
        out[i] = static_cast<TO>(x);
    }
}

// Block j of n: rows_per_block rows of row_bytes from src + (src_row0 + j *
// src_stride) rows to dst + (dst_row0 + j * dst_stride) rows; V-byte units.
template <typename U>
__global__ __launch_bounds__(kBlock) void row_blocks_kernel(const uint8_t* __restrict__ src,
                                                            uint8_t* __restrict__ dst,
                                                            int64_t units, int64_t per_block,
                                                            int64_t src_stride_b,
                                                            int64_t dst_stride_b) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < units;
         i += stride) {
        const int64_t j = i / per_block;
        const int64_t off = (i - j * per_block) * static_cast<int64_t>(sizeof(U));
        *reinterpret_cast<U*>(dst + j * dst_stride_b + off) =
            *reinterpret_cast<const U*>(src + j * src_stride_b + off);
    }
}

template <typename TI, typename TO>
hs_status launch_concat(hipStream_t st, const void* a, const void* b, void* out, int64_t rows,
                        int c1, int c2, const char* op) {
    const auto* A = static_cast<const TI*>(a);
    const auto* B = static_cast<const TI*>(b);
    auto* O = static_cast<TO*>(out);
    const bool vec = c1 % 8 == 0 && c2 % 8 == 0 && aligned16(a) && aligned16(b) && aligned16(out);
    if (vec) {
        // One row per workgroup, all in one round, the last row first, the
        // inputs read through the caches and the f32 output streamed. At
        // 43,968 rows of 1024 + 1024 f16 -> f32 (540 MB) this measured 94.5
        // us back to back (71% of peak, at its f16 -> f32 widening probe)
        // and 82.9 us behind a cache flush (81%), against 106.6 / 108.6 us
        // for two rows per workgroup with streaming loads, 111-127 us for
        // persistent grids. In the trunk the block output it reads is read
        // next by the following block's LayerNorm, from the first row on:
        // walking the rows backwards leaves the first rows the most recently
        // cached (LayerScale write, this build, LayerNorm: 175.6 against
        // 179-183 us for the ascending orders with streaming loads).
        constexpr int R = HS_CACHE_ROWS;
        const int64_t want = ceil_div(rows, int64_t{R}), cap = int64_t{1} << 22;
        const int64_t blocks = want < cap ? want : cap;
        concat_vec_kernel<TI, TO, R><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
            A, B, O, rows, c1 / 8, c2 / 8);
    } else {
        const int64_t total = rows * (c1 + c2);
        concat_scalar_kernel<TI, TO><<<dim3(static_cast<uint32_t>(grid_for(total))), dim3(kBlock), 0, st>>>(
            A, B, O, total, c1, c2);
    }
    return check_launch(op);
}

hs_status check_concat(const char* op, hs_dtype dt, const void* a, const void* b, const void* out,
                       int64_t rows, int32_t c1, int32_t c2, int64_t out_esz) {
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "%s: unknown dtype", op);
    if (rows < 0 || c1 < 0 || c2 < 0)
        return fail(HS_EINVAL, "%s: shape rows=%lld c1=%d c2=%d", op, static_cast<long long>(rows), c1, c2);
    if (rows * (int64_t{c1} + c2) >= (int64_t{1} << 40)) return fail(HS_EINVAL, "%s: tensor too large", op);
    if (rows == 0 || c1 + c2 == 0) return HS_OK;
    if (!out || (c1 > 0 && !a) || (c2 > 0 && !b)) return fail(HS_EINVAL, "%s: null buffer", op);
    const int64_t esz = dtype_size(dt);
    const int64_t out_bytes = rows * (int64_t{c1} + c2) * out_esz;
    if (overlaps(out, out_bytes, a, rows * c1 * esz) || overlaps(out, out_bytes, b, rows * c2 * esz))
        return fail(HS_EINVAL, "%s: out overlaps an input", op);
    return HS_OK;
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_concat_channels(hs_stream_t stream, hs_dtype dt, const void* a,
                                        const void* b, void* out, int64_t rows, int32_t c1,
                                        int32_t c2) {
    using namespace hs;
    const hs_status rc = check_concat("concat_channels", dt, a, b, out, rows, c1, c2, dtype_size(dt));
    if (rc != HS_OK || rows == 0 || c1 + c2 == 0) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16 ? launch_concat<f16, f16>(st, a, b, out, rows, c1, c2, "concat_channels")
                        : launch_concat<float, float>(st, a, b, out, rows, c1, c2, "concat_channels");
}

extern "C" hs_status hs_cast_f16_to_f32(hs_stream_t stream, const void* x, float* out,
                                        int64_t total) {
    using namespace hs;
    if (total < 0) return fail(HS_EINVAL, "cast_f16_to_f32: negative length");
    if (total >= kMaxElems) return fail(HS_EINVAL, "cast_f16_to_f32: tensor too large");
    if (total == 0) return HS_OK;
    if (!x || !out) return fail(HS_EINVAL, "cast_f16_to_f32: null buffer");
    if (overlaps(out, total * 4, x, total * 2)) return fail(HS_EINVAL, "cast_f16_to_f32: out overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // As a concatenation with an empty right side, in the widest rows that
    // divide the length (the vector kernel spreads a row over a workgroup).
    int32_t w = 1;
    for (int32_t cand : {2048, 256, 8})
        if (total % cand == 0) {
            w = cand;
            break;
        }
    return launch_concat<f16, float>(st, x, nullptr, out, total / w, w, 0, "cast_f16_to_f32");
}

extern "C" hs_status hs_cache_build(hs_stream_t stream, hs_dtype in_dt, const void* frame_out,
                                    const void* inter_out, float* out, int64_t rows, int32_t c1,
                                    int32_t c2) {
    using namespace hs;
    const hs_status rc = check_concat("cache_build", in_dt, frame_out, inter_out, out, rows, c1, c2, 4);
    if (rc != HS_OK || rows == 0 || c1 + c2 == 0) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return in_dt == HS_F16
               ? launch_concat<f16, float>(st, frame_out, inter_out, out, rows, c1, c2, "cache_build")
               : launch_concat<float, float>(st, frame_out, inter_out, out, rows, c1, c2, "cache_build");
}

extern "C" hs_status hs_copy_row_blocks(hs_stream_t stream, const void* src, int64_t src_row0,
                                        int64_t src_stride, void* dst, int64_t dst_row0,
                                        int64_t dst_stride, int64_t n_blocks,
                                        int64_t rows_per_block, int64_t row_bytes) {
    using namespace hs;
    if (src_row0 < 0 || dst_row0 < 0 || src_stride < 0 || dst_stride < 0 || n_blocks < 0 ||
        rows_per_block < 0 || row_bytes < 0)
        return fail(HS_EINVAL, "copy_row_blocks: negative argument");
    if (n_blocks == 0 || rows_per_block == 0 || row_bytes == 0) return HS_OK;
    if (!src || !dst) return fail(HS_EINVAL, "copy_row_blocks: null buffer");
    if (n_blocks > 1 && (src_stride < rows_per_block || dst_stride < rows_per_block))
        return fail(HS_EINVAL, "copy_row_blocks: blocks overlap (stride < rows per block)");
    const int64_t block_bytes = rows_per_block * row_bytes;
    if (block_bytes >= (int64_t{1} << 40) || n_blocks >= (int64_t{1} << 31))
        return fail(HS_EINVAL, "copy_row_blocks: too large");
    const auto* s = static_cast<const uint8_t*>(src) + src_row0 * row_bytes;
    auto* d = static_cast<uint8_t*>(dst) + dst_row0 * row_bytes;
    const int64_t src_span = ((n_blocks - 1) * src_stride + rows_per_block) * row_bytes;
    const int64_t dst_span = ((n_blocks - 1) * dst_stride + rows_per_block) * row_bytes;
    if (overlaps(d, dst_span, s, src_span)) return fail(HS_EINVAL, "copy_row_blocks: src and dst overlap");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t sb = src_stride * row_bytes, db = dst_stride * row_bytes;
    if (aligned16(s) && aligned16(d) && block_bytes % 16 == 0 && sb % 16 == 0 && db % 16 == 0) {
        const int64_t per = block_bytes / 16, units = per * n_blocks;
        row_blocks_kernel<u32x4><<<dim3(static_cast<uint32_t>(grid_for(units))), dim3(kBlock), 0, st>>>(
            s, d, units, per, sb, db);
    } else {
        const int64_t units = block_bytes * n_blocks;
        row_blocks_kernel<uint8_t><<<dim3(static_cast<uint32_t>(grid_for(units))), dim3(kBlock), 0, st>>>(
            s, d, units, block_bytes, sb, db);
    }
    return check_launch("copy_row_blocks");
}
