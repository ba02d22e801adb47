// Elementwise per-layer ops for gfx950:
//   bias + erf-GELU        (fc1 epilogue, linear_wmma.wgsl:69-74, + gelu.wesl)
//   bias + LayerScale + residual (proj/fc2 epilogue + residual_ls.wesl)
//   f32 -> f16 cast        (cast_f32_to_f16.wesl)
//   tiled add              (tiled_add.wesl)
//
// The bias/GELU and LayerScale kernels are column-stationary grid-stride loops:
// the grid's stride through the flat (rows, cols) tensor is a multiple of
// cols, so each thread owns the same V consecutive columns (one 16-byte
// vector) for every row it visits and keeps their bias/gamma in registers.
// Each thread issues U independent 16-byte loads per tensor before it
// computes, so a wave keeps U KiB per input stream in flight. The tiled add
// is table-stationary the same way for large tables (each thread owns one
// table vector and walks its repetitions).
#include "hs_common.hpp"

namespace hs {
namespace {

// Launch shape (overridable at build time for tuning sweeps).
// U: 16-byte vectors per input stream per thread per iteration; BPC:
// workgroups launched per CU; ITERS (GELU): a grid sized so that each
// thread visits that many rows instead. Chosen by timing the whole
// aggregator pass, not the op alone. Both ops run fastest with one vector
// per stream per thread and many workgroups: GELU with two visits per
// thread (S=32: 117.3 us against 120.8 for 64 workgroups per CU, ~5
// visits, and 118.0-119.7 for 96-176 workgroups per CU or three or four
// visits; 130 for 256 per CU, 157 for one visit in a one-shot grid),
// LayerScale with 32 workgroups per CU (~3 visits) while one of its
// streams fits in half the 256 MB Infinity Cache (S=32: 90 MB), and with
// two visits per thread beyond that: 32 workgroups per CU give a thread ~17
// visits at S=200, and there the two-visit grid runs 268 against 332 us
// (79% against 63% of peak; S=48 65 against 67 us, S=100 131 against 145,
// S=140 184 against 214), while at S=32 it leaves the op's own time alone
// and makes the pass 0.7% slower. GELU must keep
// non-temporal stores, because with plain stores its output occupies the
// cache and the LayerNorm after it slows by a third.
#ifndef HS_GELU_U
#define HS_GELU_U 1
#endif
#ifndef HS_GELU_BPC
#define HS_GELU_BPC 64
#endif
#ifndef HS_GELU_ITERS
#define HS_GELU_ITERS 2
#endif
#ifndef HS_GELU_NTL
#define HS_GELU_NTL (HS_NT != 0)  // non-temporal loads of the fc1 output
#endif
#ifndef HS_GELU_NTS
#define HS_GELU_NTS (HS_NT != 0)  // non-temporal stores of the activation
#endif
#ifndef HS_LS_U
#define HS_LS_U 1
#endif
#ifndef HS_LS_BPC
#define HS_LS_BPC 32
#endif
#ifndef HS_LS_ITERS
#define HS_LS_ITERS 0  // > 0: visits per thread at every size
#endif
#ifndef HS_LS_BIG_BYTES
#define HS_LS_BIG_BYTES (int64_t{128} << 20)  // one stream's bytes above which...
#endif
#ifndef HS_LS_BIG_ITERS
#define HS_LS_BIG_ITERS 2  // ...the grid gives each thread this many visits (0: never)
#endif
#ifndef HS_LS_NTS
#define HS_LS_NTS (HS_NT != 0)  // non-temporal stores of the LayerScale + residual output
#endif
#ifndef HS_EW_BPC
#define HS_EW_BPC 4  // cast and tiled add
#endif

constexpr int kBlock = 256;
constexpr int kBlocksPerCu = HS_EW_BPC;

// Grid size (in blocks) for a column-stationary launch: the stride
// blocks*kBlock*V must be a multiple of cols. Returns 0 if no such grid of
// useful size exists.
int64_t column_stationary_blocks(int64_t total, int64_t cols, int V, int U, int bpc) {
    const int64_t per_block = static_cast<int64_t>(kBlock) * V;
    int64_t a = per_block, b = cols;
    while (b) {
        int64_t r = a % b;
        a = b;
        b = r;
    }
    const int64_t step = cols / a;  // blocks must be a multiple of this
    const int64_t want = ceil_div(total, per_block * U);
    const int64_t cap = static_cast<int64_t>(num_cus()) * bpc;
    int64_t blocks = want < cap ? want : cap;
    blocks = ceil_div(blocks, step) * step;
    if (blocks > 4 * cap) return 0;
    // a launch holds fewer than 2^32 work-items; the grid-stride loop
    // covers what a smaller grid leaves
    const int64_t limit = ((int64_t{1} << 32) - 1) / kBlock;
    if (blocks > limit) blocks = (limit / step) * step;
    return blocks;
}

template <typename T, bool BIAS, int U>
__global__ __launch_bounds__(kBlock) void bias_gelu_kernel(const T* x, const float* __restrict__ bias,
                                                           T* out, int64_t total, int cols) {
    constexpr int V = Vec<T>::N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * V;
    const int64_t e0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * V;
    // The fc1 bias joins in f32; the reference's GEMM epilogue would have
    // stored x + bias as f16 first (one extra rounding this fused op leaves
    // out). For f16 input the bias is kept halved: h = x * 0.5 + b / 2 is one
    // mixed-precision FMA straight from the f16 half (no conversion, no
    // separate add) and equals 0.5f * (float(x) + b) bit for bit (halving is
    // exact, and x + b is never subnormal: a nonzero f16 x is at least 2^-24,
    // so an f32 b cancels it to 0 or to at least 2^-47).
    constexpr bool kHalfBias = BIAS && sizeof(T) == 2;
    float bv[V];
    if constexpr (BIAS) {
        const int c0 = static_cast<int>(e0 % cols);
#pragma unroll
        for (int k = 0; k < V; k += 4) {
            float4 b4 = ld_f32x4(bias + c0 + k);
            bv[k] = b4.x, bv[k + 1] = b4.y, bv[k + 2] = b4.z, bv[k + 3] = b4.w;
        }
        if constexpr (kHalfBias) {
#pragma unroll
            for (int k = 0; k < V; k++) bv[k] *= 0.5f;
        }
    }
    auto load = [&](u32x4 (&raw)[U], int64_t base) {
#pragma unroll
        for (int u = 0; u < U; u++)
            if (base + u * stride < total) raw[u] = ld_stream<HS_GELU_NTL>(x + base + u * stride);
    };
    auto compute = [&](const u32x4 (&raw)[U], int64_t base) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (base + u * stride >= total) break;
            float f[V];
            unpack(raw[u], f, T{});
#pragma unroll
            for (int k = 0; k < V; k++) {
                if constexpr (kHalfBias)
                    f[k] = gelu_half(fmaf(f[k], 0.5f, bv[k]));
                else if constexpr (BIAS)
                    f[k] = gelu_f(f[k] + bv[k]);
                else
                    f[k] = gelu_f(f[k]);
            }
            st_stream<HS_GELU_NTS>(out + base + u * stride, pack(f, T{}));
        }
    };
    for (int64_t base = e0; base < total; base += stride * U) {
        u32x4 raw[U];
        load(raw, base);
        compute(raw, base);
    }
}

template <typename T, bool BIAS, int U>
__global__ __launch_bounds__(kBlock) void bias_ls_kernel(const T* res, const T* x,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ gamma, T* out,
                                                         int64_t total, int cols) {
    constexpr int V = Vec<T>::N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * V;
    const int64_t e0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * V;
    const int c0 = static_cast<int>(e0 % cols);
    float gv[V], bv[V];
#pragma unroll
    for (int k = 0; k < V; k += 4) {
        float4 g4 = ld_f32x4(gamma + c0 + k);
        gv[k] = g4.x, gv[k + 1] = g4.y, gv[k + 2] = g4.z, gv[k + 3] = g4.w;
        if constexpr (BIAS) {
            float4 b4 = ld_f32x4(bias + c0 + k);
            bv[k] = b4.x, bv[k + 1] = b4.y, bv[k + 2] = b4.z, bv[k + 3] = b4.w;
        }
    }
    for (int64_t base = e0; base < total; base += stride * U) {
        u32x4 rr[U], xr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (base + u * stride < total) {
                rr[u] = ld_stream(res + base + u * stride);
                xr[u] = ld_stream(x + base + u * stride);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (base + u * stride >= total) break;
            float fr[V], fx[V];
            unpack(rr[u], fr, T{});
            unpack(xr[u], fx, T{});
#pragma unroll
            for (int k = 0; k < V; k++) {
                float v = fx[k];
                if constexpr (BIAS) v = storage_round(v + bv[k], T{});
                fr[k] = ls_affine(fr[k], gv[k], v);  // residual_ls.wesl:28
            }
            st_stream<HS_LS_NTS>(out + base + u * stride, pack(fr, T{}));
        }
    }
}

// Scalar fallbacks for shapes or pointers the vector kernels do not cover.
template <typename T>
__global__ __launch_bounds__(kBlock) void bias_gelu_scalar_kernel(const T* x, const float* bias,
                                                                  T* out, int64_t total, int cols) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        float v = load_elem(x + i);
        if (bias) v = v + bias[i % cols];
        store_elem(out + i, gelu_f(v));
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void bias_ls_scalar_kernel(const T* res, const T* x,
                                                                const float* bias,
                                                                const float* gamma, T* out,
                                                                int64_t total, int cols) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const int c = static_cast<int>(i % cols);
        float v = load_elem(x + i);
        if (bias) v = storage_round(v + bias[c], T{});
        store_elem(out + i, ls_affine(load_elem(res + i), gamma[c], v));
    }
}

// f32 -> f16 in a one-shot grid: each wave takes kCastU * 64 consecutive
// 4-float vectors, lane l the vectors l, l + 64, ..., so every load
// instruction reads 1 KiB and every store writes 512 contiguous bytes, all
// kCastU loads in flight before the first store (two per lane: the cast
// probe's fastest shape). Elements past the last
// whole vector (total % 4) are cast by the first lanes of workgroup 0.
#ifndef HS_CAST_U
#define HS_CAST_U 2  // S=32 (45 M floats): 42.4 us against 45.0 for 4, 46.1 for 1, 79.5 for 8
#endif
constexpr int kCastU = HS_CAST_U;

__global__ __launch_bounds__(kBlock) void cast_f32_f16_kernel(const float* x, f16* out, int64_t total) {
    const int64_t n4 = total / 4;
    const int64_t base =
        (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * kCastU + (threadIdx.x & 63);
    u32x4 r[kCastU];
#pragma unroll
    for (int u = 0; u < kCastU; u++)
        if (base + u * 64 < n4) r[u] = ld_stream(x + (base + u * 64) * 4);
#pragma unroll
    for (int u = 0; u < kCastU; u++) {
        if (base + u * 64 >= n4) break;
        float f[4];
        unpack(r[u], f, float{});
        u32x2 v;
        v[0] = h22u(f16x2{static_cast<f16>(f[0]), static_cast<f16>(f[1])});
        v[1] = h22u(f16x2{static_cast<f16>(f[2]), static_cast<f16>(f[3])});
        st_stream_as(reinterpret_cast<u32x2*>(out + (base + u * 64) * 4), v);
    }
    if (blockIdx.x == 0 && threadIdx.x < total - n4 * 4)
        out[n4 * 4 + threadIdx.x] = static_cast<f16>(x[n4 * 4 + threadIdx.x]);
}

__global__ __launch_bounds__(kBlock) void cast_f32_f16_scalar_kernel(const float* x, f16* out,
                                                                     int64_t total) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride)
        out[i] = static_cast<f16>(x[i]);
}

__global__ __launch_bounds__(kBlock) void tiled_add_kernel(const float* x, const float* table,
                                                           float* out, int64_t total, int64_t block) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride)
        out[i] = x[i] + table[i % block];
}

// Tiled add over a large table in a one-shot 2D grid: workgroup (bx, by)
// takes table vectors [256 bx, 256 bx + 256) (4 floats each, read once per
// thread from the cache) and repetitions [kTileReps by, kTileReps by +
// kTileReps) of them; a thread's kTileReps loads are in flight before its
// first store, and lanes read and write consecutive vectors. No index needs
// a division. Used when the table is a whole number of 16-byte vectors and
// large enough to fill the GPU (a pos-embed table: P x 1024 floats); other
// shapes take the flat kernel.
#ifndef HS_TILE_REPS
#define HS_TILE_REPS 4
#endif
constexpr int kTileReps = HS_TILE_REPS;

__global__ __launch_bounds__(kBlock) void tiled_add_vec_kernel(const float* x,
                                                               const float* __restrict__ table,
                                                               float* out, int64_t reps,
                                                               int64_t block4) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= block4) return;  // no barriers below
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kTileReps;
    const float4 t = ld_f32x4(table + 4 * j);
    const int64_t stride = block4 * 4;
    const float* xp = x + r0 * stride + 4 * j;
    float* op = out + r0 * stride + 4 * j;
    u32x4 v[kTileReps];
#pragma unroll
    for (int r = 0; r < kTileReps; r++)
        if (r0 + r < reps) v[r] = ld_stream(xp + r * stride);
#pragma unroll
    for (int r = 0; r < kTileReps; r++) {
        if (r0 + r >= reps) break;
        u32x4 o;
        o[0] = f2u(u2f(v[r][0]) + t.x), o[1] = f2u(u2f(v[r][1]) + t.y);
        o[2] = f2u(u2f(v[r][2]) + t.z), o[3] = f2u(u2f(v[r][3]) + t.w);
        st_stream(op + r * stride, o);
    }
}

int64_t flat_blocks(int64_t items) {
    const int64_t cap = static_cast<int64_t>(num_cus()) * kBlocksPerCu;
    const int64_t want = ceil_div(items, kBlock);
    return want < 1 ? 1 : (want < cap ? want : cap);
}

template <typename T>
hs_status launch_gelu(hipStream_t st, const void* x, const float* bias, void* out, int64_t rows,
                      int cols) {
    constexpr int V = Vec<T>::N;
    constexpr int U = HS_GELU_U;
    const int64_t total = rows * cols;
    const bool vec_ok = cols % V == 0 && aligned16(x) && aligned16(out) && (!bias || aligned16(bias));
    // HS_GELU_ITERS > 0: a grid in which each thread visits that many rows
    // (the last visit partial), whatever the tensor's size; else a grid of
    // HS_GELU_BPC workgroups per CU.
    const int64_t blocks =
        !vec_ok ? 0
        : HS_GELU_ITERS > 0 ? column_stationary_blocks(total, cols, V, U * HS_GELU_ITERS, 1 << 16)
                            : column_stationary_blocks(total, cols, V, U, HS_GELU_BPC);
    if (blocks > 0) {
        if (bias)
            bias_gelu_kernel<T, true, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
                static_cast<const T*>(x), bias, static_cast<T*>(out), total, cols);
        else
            bias_gelu_kernel<T, false, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
                static_cast<const T*>(x), bias, static_cast<T*>(out), total, cols);
    } else {
        bias_gelu_scalar_kernel<T><<<dim3(static_cast<uint32_t>(flat_blocks(total))), dim3(kBlock), 0, st>>>(
            static_cast<const T*>(x), bias, static_cast<T*>(out), total, cols);
    }
    return check_launch("bias_gelu");
}

template <typename T>
hs_status launch_ls(hipStream_t st, const void* res, const void* x, const float* bias,
                    const float* gamma, void* out, int64_t rows, int cols) {
    constexpr int V = Vec<T>::N;
    constexpr int U = HS_LS_U;
    const int64_t total = rows * cols;
    const bool vec_ok = cols % V == 0 && aligned16(res) && aligned16(x) && aligned16(out) &&
                        aligned16(gamma) && (!bias || aligned16(bias));
    const int iters = HS_LS_ITERS > 0 ? HS_LS_ITERS
                      : HS_LS_BIG_ITERS > 0 && total * static_cast<int64_t>(sizeof(T)) > HS_LS_BIG_BYTES
                          ? HS_LS_BIG_ITERS
                          : 0;
    const int64_t blocks =
        !vec_ok ? 0
        : iters > 0 ? column_stationary_blocks(total, cols, V, U * iters, 1 << 16)
                    : column_stationary_blocks(total, cols, V, U, HS_LS_BPC);
    if (blocks > 0) {
        if (bias)
            bias_ls_kernel<T, true, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
                static_cast<const T*>(res), static_cast<const T*>(x), bias, gamma,
                static_cast<T*>(out), total, cols);
        else
            bias_ls_kernel<T, false, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
                static_cast<const T*>(res), static_cast<const T*>(x), bias, gamma,
                static_cast<T*>(out), total, cols);
    } else {
        bias_ls_scalar_kernel<T><<<dim3(static_cast<uint32_t>(flat_blocks(total))), dim3(kBlock), 0, st>>>(
            static_cast<const T*>(res), static_cast<const T*>(x), bias, gamma,
            static_cast<T*>(out), total, cols);
    }
    return check_launch("bias_ls_residual");
}

// In-place is allowed only as exact aliasing of whole tensors.
bool bad_alias(const void* a, const void* out, int64_t bytes) {
    return a != out && overlaps(a, bytes, out, bytes);
}

}  // namespace
}  // namespace hs

extern "C" {

hs_status hs_bias_gelu(hs_stream_t stream, hs_dtype dt, const void* x, const float* bias,
                       void* out, int64_t rows, int32_t cols) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "bias_gelu: unknown dtype %d", (int)dt);
    if (rows < 0 || cols <= 0)
        return fail(HS_EINVAL, "bias_gelu: rows %lld / cols %d", (long long)rows, cols);
    if (too_large(rows, cols)) return fail(HS_EINVAL, "bias_gelu: tensor too large");
    if (rows == 0) return HS_OK;
    if (!x || !out) return fail(HS_EINVAL, "bias_gelu: null buffer");
    if (bad_alias(x, out, rows * cols * dtype_size(dt)))
        return fail(HS_EINVAL, "bias_gelu: out partially overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16 ? launch_gelu<f16>(st, x, bias, out, rows, cols)
                        : launch_gelu<float>(st, x, bias, out, rows, cols);
}

hs_status hs_gelu(hs_stream_t stream, hs_dtype dt, const void* x, void* out, int64_t total) {
    if (total < 0) return hs::fail(HS_EINVAL, "gelu: negative length %lld", (long long)total);
    if (total == 0) return HS_OK;
    // Without a bias the column split is arbitrary: rows of 8 elements keep
    // the vector path for any length that is a multiple of 8.
    if (total % 8 == 0) return hs_bias_gelu(stream, dt, x, nullptr, out, total / 8, 8);
    return hs_bias_gelu(stream, dt, x, nullptr, out, total, 1);
}

hs_status hs_bias_ls_residual(hs_stream_t stream, hs_dtype dt, const void* res, const void* x,
                              const float* bias, const float* gamma, void* out, int64_t rows,
                              int32_t dim) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "bias_ls_residual: unknown dtype %d", (int)dt);
    if (rows < 0 || dim <= 0)
        return fail(HS_EINVAL, "bias_ls_residual: rows %lld / dim %d", (long long)rows, dim);
    if (too_large(rows, dim)) return fail(HS_EINVAL, "bias_ls_residual: tensor too large");
    if (rows == 0) return HS_OK;
    if (!res || !x || !gamma || !out) return fail(HS_EINVAL, "bias_ls_residual: null buffer");
    const int64_t bytes = rows * dim * dtype_size(dt);
    if (bad_alias(res, out, bytes) || bad_alias(x, out, bytes))
        return fail(HS_EINVAL, "bias_ls_residual: out partially overlaps an input");
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16 ? launch_ls<f16>(st, res, x, bias, gamma, out, rows, dim)
                        : launch_ls<float>(st, res, x, bias, gamma, out, rows, dim);
}

hs_status hs_residual_ls(hs_stream_t stream, hs_dtype dt, const void* res, const void* x,
                         const float* gamma, void* out, int64_t total, int32_t dim) {
    if (total < 0 || dim <= 0)
        return hs::fail(HS_EINVAL, "residual_ls: total %lld / dim %d", (long long)total, dim);
    if (total % dim != 0)
        return hs::fail(HS_EINVAL, "residual_ls: total %lld is not a multiple of dim %d",
                        (long long)total, dim);
    return hs_bias_ls_residual(stream, dt, res, x, nullptr, gamma, out, total / dim, dim);
}

hs_status hs_cast_f32_to_f16(hs_stream_t stream, const float* x, void* out, int64_t total) {
    using namespace hs;
    if (total < 0) return fail(HS_EINVAL, "cast_f32_to_f16: negative length");
    if (total >= kMaxElems) return fail(HS_EINVAL, "cast_f32_to_f16: tensor too large");
    if (total == 0) return HS_OK;
    if (!x || !out) return fail(HS_EINVAL, "cast_f32_to_f16: null buffer");
    if (overlaps(x, total * 4, out, total * 2))
        return fail(HS_EINVAL, "cast_f32_to_f16: out overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    int64_t blocks = ceil_div(ceil_div(total / 4, int64_t{kCastU}), int64_t{kBlock});
    if (blocks < 1) blocks = 1;  // total < 4: workgroup 0 casts the tail
    // the dispatch packet counts work-items in 32 bits
    if (aligned16(x) && aligned16(out) && blocks * kBlock < (int64_t{1} << 32))
        cast_f32_f16_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
            x, static_cast<f16*>(out), total);
    else
        cast_f32_f16_scalar_kernel<<<dim3(static_cast<uint32_t>(flat_blocks(total))), dim3(kBlock), 0, st>>>(
            x, static_cast<f16*>(out), total);
    return check_launch("cast_f32_to_f16");
}

hs_status hs_tiled_add(hs_stream_t stream, const float* x, const float* table, float* out,
                       int64_t total, int64_t block) {
    using namespace hs;
    if (total < 0 || block <= 0) return fail(HS_EINVAL, "tiled_add: total / block");
    if (total >= kMaxElems) return fail(HS_EINVAL, "tiled_add: tensor too large");
    if (total % block != 0)
        return fail(HS_EINVAL, "tiled_add: table of %lld does not tile %lld elements",
                    (long long)block, (long long)total);
    if (total == 0) return HS_OK;
    if (!x || !table || !out) return fail(HS_EINVAL, "tiled_add: null buffer");
    if (bad_alias(x, out, total * 4)) return fail(HS_EINVAL, "tiled_add: out partially overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t rgroups = ceil_div(total / block, int64_t{kTileReps});
    if (block % 4 == 0 && block / 4 >= 65536 && block / 4 < (int64_t{1} << 31) && rgroups < 65536 &&
        aligned16(x) && aligned16(table) && aligned16(out)) {
        const int64_t block4 = block / 4;
        const dim3 grid(static_cast<uint32_t>(ceil_div(block4, int64_t{kBlock})),
                        static_cast<uint32_t>(rgroups));
        tiled_add_vec_kernel<<<grid, dim3(kBlock), 0, st>>>(x, table, out, total / block, block4);
        return check_launch("tiled_add");
    }
    tiled_add_kernel<<<dim3(static_cast<uint32_t>(flat_blocks(total))), dim3(kBlock), 0, st>>>(
        x, table, out, total, block);
    return check_launch("tiled_add");
}

}  // extern "C"
