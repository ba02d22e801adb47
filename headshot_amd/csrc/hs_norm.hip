// Row LayerNorm for gfx950 (replaces shaders/layernorm.wesl, dispatched by
// GpuContext::layernorm, engine/ops.rs:130-153).
//
// Fast path: one wave64 per row with the whole row held in registers — each
// lane loads CHUNKS 16-byte vectors (a 1024-wide f16 row is 2 loads per
// lane, each load instruction a contiguous 1 KiB), mean and variance are
// reduced across the wave with DPP lane permutes (no LDS, no barrier), and
// the row is written back with 16-byte stores. Each wave keeps the weight
// and bias slices it needs in registers and takes U rows, issuing all
// U*CHUNKS loads before it reduces, so every wave has U*2 KiB of HBM reads
// in flight. The grid has one wave per U rows (a grid-stride loop covers
// row counts beyond 2^22 workgroups): measured against persistent grids of
// 2-8 workgroups per CU, which walk several row groups per wave, it is the
// fastest at 44k rows, alone (69.5% of peak against 65.5%) and inside the
// aggregator pass (72.1% against 69.7%).
//
// Narrow path (rows of 8 or 16 vectors, e.g. 64-wide f16 QK-norm rows):
// several rows per wave, each reduced within its group of lanes.
//
// Generic path: any dim, one wave per row, strided over the row three
// times (mean, variance, output) with the second and third reads served by
// the cache.
// LayerNorm keeps cached (temporal) accesses. Alone, non-temporal ones are
// faster (72.7% of peak against 69.5%), but inside the aggregator pass they
// slowed LayerNorm (66.8% against 72.1%) and the LayerScale + residual op
// after it, which reads the same residual rows again (67.7% against 78.5%).
// Per stream, in the S=32 pass: non-temporal stores alone cost LayerNorm
// 29.2 -> 32.0 us, non-temporal loads alone cost the LayerScale after it
// 39.7 -> 45.4 us (the pass 15.07 against 15.30 and 15.67 ms).
#ifndef HS_NT
#define HS_NT 0
#endif
#include "hs_common.hpp"

namespace hs {
namespace {

// Launch shape (overridable at build time for tuning sweeps).
#ifndef HS_LN_U
#define HS_LN_U 2  // rows per wave per iteration
#endif
#ifndef HS_LN_BPC
#define HS_LN_BPC 0  // workgroups per CU of a persistent grid; 0: one wave per U rows
#endif

constexpr int kBlock = 256;  // 4 waves per workgroup
constexpr int kWavesPerBlock = kBlock / 64;
constexpr int kBlocksPerCu = 4;  // generic path

// A row's mean and rsqrt(var + eps) over the f32 values f (lane's values
// at columns c * 64 V + lane * V + k), two-pass, reduced across the wave.
// Shared by every kernel that normalises whole rows per wave, so they agree
// bit for bit on the same row.
template <int CHUNKS, int V>
__device__ __forceinline__ void row_moments(const float (&f)[CHUNKS][V], float eps, float& mean,
                                            float& inv) {
    constexpr int DIM = 64 * V * CHUNKS;
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; c++)
#pragma unroll
        for (int k = 0; k < V; k++) s += f[c][k];
    mean = wave_sum(s) / static_cast<float>(DIM);
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; c++)
#pragma unroll
        for (int k = 0; k < V; k++) {
            const float d = f[c][k] - mean;
            q += d * d;
        }
    const float var = wave_sum(q) / static_cast<float>(DIM);
    inv = rsqrtf(var + eps);
}

// STATS: write each row's (mean, rsqrt(var + eps)) to stats[2 r], [2 r + 1]
// instead of the normalised row (the statistics the row would be normalised
// with, from the same code).
template <typename T, int CHUNKS, int U, bool STATS>
__global__ __launch_bounds__(kBlock) void ln_vec_kernel(const T* x, const float* __restrict__ w,
                                                        const float* __restrict__ b, T* out,
                                                        float* stats, int64_t rows, float eps) {
    constexpr int V = Vec<T>::N;
    constexpr int DIM = 64 * V * CHUNKS;
    const int lane = lane_id();
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;

    float wr[CHUNKS][V], br[CHUNKS][V];
#pragma unroll
    for (int c = 0; c < CHUNKS && !STATS; c++) {
        const int col = c * 64 * V + lane * V;
#pragma unroll
        for (int k = 0; k < V; k += 4) {
            float4 w4 = ld_f32x4(w + col + k), b4 = ld_f32x4(b + col + k);
            wr[c][k] = w4.x, wr[c][k + 1] = w4.y, wr[c][k + 2] = w4.z, wr[c][k + 3] = w4.w;
            br[c][k] = b4.x, br[c][k + 1] = b4.y, br[c][k + 2] = b4.z, br[c][k + 3] = b4.w;
        }
    }

    for (int64_t r0 = wave * U; r0 < rows; r0 += nwaves * U) {
        u32x4 raw[U][CHUNKS];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (r0 + u < rows) {
                const T* xr = x + (r0 + u) * DIM + lane * V;
#pragma unroll
                for (int c = 0; c < CHUNKS; c++) raw[u][c] = ld_stream(xr + c * 64 * V);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (r0 + u >= rows) break;
            float f[CHUNKS][V];
#pragma unroll
            for (int c = 0; c < CHUNKS; c++) unpack(raw[u][c], f[c], T{});
            float mean, inv;
            row_moments(f, eps, mean, inv);
            if constexpr (STATS) {
                if (lane == 0) {
                    f32x2 m2;
                    m2[0] = mean, m2[1] = inv;
                    *reinterpret_cast<f32x2*>(stats + 2 * (r0 + u)) = m2;
                }
                continue;
            }
            T* orow = out + (r0 + u) * DIM + lane * V;
#pragma unroll
            for (int c = 0; c < CHUNKS; c++) {
                float y[V];
#pragma unroll
                for (int k = 0; k < V; k++) y[k] = ln_affine(f[c][k], mean, inv, wr[c][k], br[c][k]);
                st_stream(orow + c * 64 * V, pack(y, T{}));
            }
        }
    }
}

#ifndef HS_LSLN_U
// rows per wave and iteration of the fused LayerScale + LayerNorm kernel:
// at S=32, in the four-op pass, 4 took 58.2 us warm / 60.0 cold (pass
// 14.05 ms) against 61.0 / 62.5 (14.27 ms) for 2 and 72.8 / 73.8 for 1
#define HS_LSLN_U 4
#endif
// Its cache policy per stream (1: non-temporal): res and x loads, out and
// normed stores. In the pass, out (the residual stream) is read again two
// ops later (by LS2, or by the next block's LS1) and res was written so by
// the op before: cached res loads and out stores keep them in the Infinity
// Cache for that reader (S=32 pass 14.51 against 14.83 ms with all four
// streaming, 15.22 ms all cached; the six-op pass took 15.22 ms on the same
// box).
#ifndef HS_LSLN_NT_RES
#define HS_LSLN_NT_RES 0
#endif
#ifndef HS_LSLN_NT_X
#define HS_LSLN_NT_X 1
#endif
#ifndef HS_LSLN_NT_OUT
#define HS_LSLN_NT_OUT 0
#endif
#ifndef HS_LSLN_NT_NORMED
#define HS_LSLN_NT_NORMED 1
#endif
#ifndef HS_LSLN_BPC
#define HS_LSLN_BPC 0  // its workgroups per CU (a persistent grid); 0: one wave per U rows
#endif
// Above this many bytes per stream no reader finds out or res in the 256 MB
// Infinity Cache anyway, and all four streams go non-temporal (S=200,
// 563 MB per stream: 368-390 against 397-411 us in the four-op sequence).
#ifndef HS_LSLN_BIG_BYTES
#define HS_LSLN_BIG_BYTES (int64_t{128} << 20)
#endif

// LayerScale + residual, then the LayerNorm of its output
// (hs_bias_ls_residual_layernorm): the pre-norm block stores x1 = res +
// gamma * dt(x + bias) and the next op normalises x1 (model/block.rs:150-153,
// and a block's output into the next block's LN1, :128). A wave takes U rows
// in the lane layout of ln_vec_kernel; each row's x1 is formed in registers
// exactly as bias_ls_kernel forms it, stored, and normalised from its stored
// (rounded) values by the same moments and affine as ln_vec_kernel, so out
// and normed are bit-identical to hs_bias_ls_residual then hs_layernorm.
// Each row is read once (res and x) and written twice (out and normed).
template <typename T, int CHUNKS, int U, bool BIAS, bool BIG>
__global__ __launch_bounds__(kBlock) void ls_ln_kernel(const T* res, const T* x,
                                                       const float* __restrict__ bias,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ b, T* out,
                                                       T* normed, int64_t rows, float eps) {
    constexpr int V = Vec<T>::N;
    constexpr int DIM = 64 * V * CHUNKS;
    const int lane = lane_id();
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;

    float gr[CHUNKS][V], bsr[CHUNKS][V], wr[CHUNKS][V], br[CHUNKS][V];
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int col = c * 64 * V + lane * V;
#pragma unroll
        for (int k = 0; k < V; k += 4) {
            const float4 g4 = ld_f32x4(gamma + col + k), w4 = ld_f32x4(w + col + k);
            const float4 b4 = ld_f32x4(b + col + k);
            gr[c][k] = g4.x, gr[c][k + 1] = g4.y, gr[c][k + 2] = g4.z, gr[c][k + 3] = g4.w;
            wr[c][k] = w4.x, wr[c][k + 1] = w4.y, wr[c][k + 2] = w4.z, wr[c][k + 3] = w4.w;
            br[c][k] = b4.x, br[c][k + 1] = b4.y, br[c][k + 2] = b4.z, br[c][k + 3] = b4.w;
            if constexpr (BIAS) {
                const float4 s4 = ld_f32x4(bias + col + k);
                bsr[c][k] = s4.x, bsr[c][k + 1] = s4.y, bsr[c][k + 2] = s4.z, bsr[c][k + 3] = s4.w;
            }
        }
    }

    for (int64_t r0 = wave * U; r0 < rows; r0 += nwaves * U) {
        u32x4 rr[U][CHUNKS], xr[U][CHUNKS];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (r0 + u < rows) {
                const int64_t off = (r0 + u) * DIM + lane * V;
#pragma unroll
                for (int c = 0; c < CHUNKS; c++) {
                    rr[u][c] = ld_stream<BIG || HS_LSLN_NT_RES != 0>(res + off + c * 64 * V);
                    xr[u][c] = ld_stream<BIG || HS_LSLN_NT_X != 0>(x + off + c * 64 * V);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (r0 + u >= rows) break;
            const int64_t off = (r0 + u) * DIM + lane * V;
            float f[CHUNKS][V];
#pragma unroll
            for (int c = 0; c < CHUNKS; c++) {
                float fr[V], fx[V];
                unpack(rr[u][c], fr, T{});
                unpack(xr[u][c], fx, T{});
#pragma unroll
                for (int k = 0; k < V; k++) {
                    float v = fx[k];
                    if constexpr (BIAS) v = storage_round(v + bsr[c][k], T{});
                    fr[k] = ls_affine(fr[k], gr[c][k], v);
                }
                const u32x4 o = pack(fr, T{});
                st_stream<BIG || HS_LSLN_NT_OUT != 0>(out + off + c * 64 * V, o);
                unpack(o, f[c], T{});  // the stored value, as hs_layernorm reads it
            }
            float mean, inv;
            row_moments(f, eps, mean, inv);
#pragma unroll
            for (int c = 0; c < CHUNKS; c++) {
                float y[V];
#pragma unroll
                for (int k = 0; k < V; k++) y[k] = ln_affine(f[c][k], mean, inv, wr[c][k], br[c][k]);
                st_stream<BIG || HS_LSLN_NT_NORMED != 0>(normed + off + c * 64 * V, pack(y, T{}));
            }
        }
    }
}

// Narrow rows (dim = G vectors of 16 bytes, G = 8 or 16: a 64-wide f16 row
// such as the reference's QK-norm over head_dim, model/block.rs:136-142):
// a row lives in a group of G lanes, one 16-byte vector per lane, so a wave
// holds 64 / G rows per load instruction and reduces each over its group
// with DPP permutes. Each wave takes U such row groups, all loads issued
// before any row is reduced.
template <typename T, int G, int U, bool STATS = false>
__global__ __launch_bounds__(kBlock) void ln_small_kernel(const T* x, const float* __restrict__ w,
                                                          const float* __restrict__ b, T* out,
                                                          float* stats, int64_t rows, float eps) {
    constexpr int V = Vec<T>::N;
    constexpr int DIM = G * V;
    constexpr int RPW = 64 / G;  // rows per load instruction
    const int lane = lane_id();
    const int piece = lane % G;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
    float wr[V], br[V];
#pragma unroll
    for (int k = 0; k < V && !STATS; k += 4) {
        const float4 w4 = ld_f32x4(w + piece * V + k), b4 = ld_f32x4(b + piece * V + k);
        wr[k] = w4.x, wr[k + 1] = w4.y, wr[k + 2] = w4.z, wr[k + 3] = w4.w;
        br[k] = b4.x, br[k + 1] = b4.y, br[k + 2] = b4.z, br[k + 3] = b4.w;
    }
    for (int64_t r0 = wave * (U * RPW); r0 < rows; r0 += nwaves * (U * RPW)) {
        // every lane of a group shares its row, so the bounds test is uniform
        // across the group that the reductions read
        u32x4 raw[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t row = r0 + u * RPW + lane / G;
            raw[u] = u32x4{0, 0, 0, 0};
            if (row < rows) raw[u] = ld_stream(x + row * DIM + piece * V);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t row = r0 + u * RPW + lane / G;
            float f[V];
            unpack(raw[u], f, T{});
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < V; k++) s += f[k];
            const float mean = group_sum<G>(s) / static_cast<float>(DIM);
            float q = 0.0f;
#pragma unroll
            for (int k = 0; k < V; k++) {
                const float d = f[k] - mean;
                q += d * d;
            }
            const float inv = rsqrtf(group_sum<G>(q) / static_cast<float>(DIM) + eps);
            if constexpr (STATS) {
                if (piece == 0 && row < rows) {
                    f32x2 m2;
                    m2[0] = mean, m2[1] = inv;
                    *reinterpret_cast<f32x2*>(stats + 2 * row) = m2;
                }
                continue;
            }
            float y[V];
#pragma unroll
            for (int k = 0; k < V; k++) y[k] = ln_affine(f[k], mean, inv, wr[k], br[k]);
            if (row < rows) st_stream(out + row * DIM + piece * V, pack(y, T{}));
        }
    }
}

template <typename T, bool STATS>
__global__ __launch_bounds__(kBlock) void ln_generic_kernel(const T* x, const float* __restrict__ w,
                                                            const float* __restrict__ b, T* out,
                                                            float* stats, int64_t rows, int dim,
                                                            float eps) {
    const int lane = lane_id();
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
    for (int64_t row = wave; row < rows; row += nwaves) {
        const T* xr = x + row * dim;
        T* orow = out + row * dim;
        float s = 0.0f;
        for (int j = lane; j < dim; j += 64) s += load_elem(xr + j);
        const float mean = wave_sum(s) / static_cast<float>(dim);
        float q = 0.0f;
        for (int j = lane; j < dim; j += 64) {
            const float d = load_elem(xr + j) - mean;
            q += d * d;
        }
        const float var = wave_sum(q) / static_cast<float>(dim);
        const float inv = rsqrtf(var + eps);
        if constexpr (STATS) {
            if (lane == 0) {
                f32x2 m2;
                m2[0] = mean, m2[1] = inv;
                *reinterpret_cast<f32x2*>(stats + 2 * row) = m2;
            }
            continue;
        }
        for (int j = lane; j < dim; j += 64)
            store_elem(orow + j, ln_affine(load_elem(xr + j), mean, inv, w[j], b[j]));
    }
}

int64_t persistent_blocks(int64_t work_waves) {
    const int64_t cap = static_cast<int64_t>(num_cus()) * kBlocksPerCu;
    int64_t blocks = ceil_div(work_waves, kWavesPerBlock);
    return blocks < cap ? blocks : cap;
}

template <typename T, int CHUNKS, bool STATS = false>
hs_status launch_vec(hipStream_t st, const void* x, const float* w, const float* b, void* out,
                     float* stats, int64_t rows, float eps) {
    constexpr int U = HS_LN_U;
    const int64_t want = ceil_div(ceil_div(rows, U), kWavesPerBlock);
    const int64_t cap = HS_LN_BPC > 0 ? static_cast<int64_t>(num_cus()) * HS_LN_BPC
                                      : int64_t{1} << 22;
    const int64_t blocks = want < cap ? want : cap;
    ln_vec_kernel<T, CHUNKS, U, STATS><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
        static_cast<const T*>(x), w, b, static_cast<T*>(out), stats, rows, eps);
    return check_launch(STATS ? "layernorm_stats" : "layernorm");
}

template <typename T, bool STATS = false>
hs_status launch_small(hipStream_t st, const void* x, const float* w, const float* b, void* out,
                       float* stats, int64_t rows, int dim, float eps) {
    constexpr int V = Vec<T>::N;
    constexpr int U = 2;
    const int64_t want = ceil_div(ceil_div(rows, (dim == 8 * V ? 8 : 4) * U), kWavesPerBlock);
    const int64_t blocks = want < (int64_t{1} << 22) ? want : (int64_t{1} << 22);
    if (dim == 8 * V)
        ln_small_kernel<T, 8, U, STATS><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
            static_cast<const T*>(x), w, b, static_cast<T*>(out), stats, rows, eps);
    else
        ln_small_kernel<T, 16, U, STATS><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
            static_cast<const T*>(x), w, b, static_cast<T*>(out), stats, rows, eps);
    return check_launch(STATS ? "layernorm_stats" : "layernorm");
}

template <typename T>
hs_status launch(hipStream_t st, const void* x, const float* w, const float* b, void* out,
                 int64_t rows, int dim, float eps) {
    constexpr int V = Vec<T>::N;
    const bool vec_ok = aligned16(x) && aligned16(out) && aligned16(w) && aligned16(b) &&
                        dim % (64 * V) == 0;
    if (vec_ok) {
        switch (dim / (64 * V)) {
            case 1: return launch_vec<T, 1>(st, x, w, b, out, nullptr, rows, eps);
            case 2: return launch_vec<T, 2>(st, x, w, b, out, nullptr, rows, eps);
            case 4: return launch_vec<T, 4>(st, x, w, b, out, nullptr, rows, eps);
            default: break;
        }
    }
    const bool small_ok = aligned16(x) && aligned16(out) && aligned16(w) && aligned16(b) &&
                          (dim == 8 * V || dim == 16 * V);
    if (small_ok) return launch_small<T>(st, x, w, b, out, nullptr, rows, dim, eps);
    const int64_t blocks = persistent_blocks(rows);
    ln_generic_kernel<T, false><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
        static_cast<const T*>(x), w, b, static_cast<T*>(out), nullptr, rows, dim, eps);
    return check_launch("layernorm");
}

// The fused LayerScale + residual + LayerNorm launch for row widths of 1,
// 2 or 4 chunks of 64 16-byte vectors with aligned buffers; false if the
// shape needs the two single ops.

template <typename T>
bool launch_ls_ln(hipStream_t st, const void* res, const void* x, const float* bias,
                  const float* gamma, const float* w, const float* b, void* out, void* normed,
                  int64_t rows, int dim, float eps) {
    constexpr int V = Vec<T>::N;
    constexpr int U = HS_LSLN_U;
    if (!(aligned16(res) && aligned16(x) && aligned16(gamma) && aligned16(w) && aligned16(b) &&
          aligned16(out) && aligned16(normed) && (!bias || aligned16(bias)) && dim % (64 * V) == 0))
        return false;
    const int chunks = dim / (64 * V);
    if (chunks != 1 && chunks != 2 && chunks != 4) return false;
    const int64_t want = ceil_div(ceil_div(rows, U), kWavesPerBlock);
    const int64_t cap = HS_LSLN_BPC > 0 ? static_cast<int64_t>(num_cus()) * HS_LSLN_BPC : int64_t{1} << 22;
    const dim3 grid(static_cast<uint32_t>(want < cap ? want : cap));
    const T* R = static_cast<const T*>(res);
    const T* X = static_cast<const T*>(x);
    T* O = static_cast<T*>(out);
    T* N = static_cast<T*>(normed);
    const bool big = rows * dim * static_cast<int64_t>(sizeof(T)) > HS_LSLN_BIG_BYTES;
#define HS_LS_LN(C, G)                                                                            \
    (bias ? (ls_ln_kernel<T, C, U, true, G><<<grid, dim3(kBlock), 0, st>>>(R, X, bias, gamma, w, b, \
                                                                            O, N, rows, eps), 0)  \
          : (ls_ln_kernel<T, C, U, false, G><<<grid, dim3(kBlock), 0, st>>>(R, X, bias, gamma, w, \
                                                                             b, O, N, rows, eps), 0))
    switch (chunks) {
        case 1: big ? HS_LS_LN(1, true) : HS_LS_LN(1, false); break;
        case 2: big ? HS_LS_LN(2, true) : HS_LS_LN(2, false); break;
        default: big ? HS_LS_LN(4, true) : HS_LS_LN(4, false); break;
    }
#undef HS_LS_LN
    return true;
}

// Row statistics only: the kernel (and so the arithmetic) that the
// normalising launch above picks for the same x when the other buffers are
// 16-byte aligned too.
template <typename T>
hs_status launch_stats(hipStream_t st, const void* x, float* stats, int64_t rows, int dim,
                       float eps) {
    constexpr int V = Vec<T>::N;
    if (aligned16(x) && dim % (64 * V) == 0) {
        switch (dim / (64 * V)) {
            case 1: return launch_vec<T, 1, true>(st, x, nullptr, nullptr, nullptr, stats, rows, eps);
            case 2: return launch_vec<T, 2, true>(st, x, nullptr, nullptr, nullptr, stats, rows, eps);
            case 4: return launch_vec<T, 4, true>(st, x, nullptr, nullptr, nullptr, stats, rows, eps);
            default: break;
        }
    }
    if (aligned16(x) && (dim == 8 * V || dim == 16 * V))
        return launch_small<T, true>(st, x, nullptr, nullptr, nullptr, stats, rows, dim, eps);
    const int64_t blocks = persistent_blocks(rows);
    ln_generic_kernel<T, true><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
        static_cast<const T*>(x), nullptr, nullptr, nullptr, stats, rows, dim, eps);
    return check_launch("layernorm_stats");
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_layernorm(hs_stream_t stream, hs_dtype dt, const void* x, const float* w,
                                  const float* b, void* out, int64_t rows, int32_t dim,
                                  float eps) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "layernorm: unknown dtype %d", (int)dt);
    if (rows < 0 || dim <= 0)
        return fail(HS_EINVAL, "layernorm: rows %lld / dim %d", (long long)rows, dim);
    if (too_large(rows, dim)) return fail(HS_EINVAL, "layernorm: tensor too large");
    if (rows == 0) return HS_OK;
    if (!x || !w || !b || !out) return fail(HS_EINVAL, "layernorm: null buffer");
    const int64_t bytes = rows * dim * dtype_size(dt);
    if (x != out && overlaps(x, bytes, out, bytes))
        return fail(HS_EINVAL, "layernorm: out partially overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16 ? launch<f16>(st, x, w, b, out, rows, dim, eps)
                        : launch<float>(st, x, w, b, out, rows, dim, eps);
}

extern "C" hs_status hs_layernorm_stats(hs_stream_t stream, hs_dtype dt, const void* x,
                                        float* stats, int64_t rows, int32_t dim, float eps) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "layernorm_stats: unknown dtype %d", (int)dt);
    if (rows < 0 || dim <= 0)
        return fail(HS_EINVAL, "layernorm_stats: rows %lld / dim %d", (long long)rows, dim);
    if (too_large(rows, dim)) return fail(HS_EINVAL, "layernorm_stats: tensor too large");
    if (rows == 0) return HS_OK;
    if (!x || !stats) return fail(HS_EINVAL, "layernorm_stats: null buffer");
    if (reinterpret_cast<uintptr_t>(stats) % 8 != 0)
        return fail(HS_EINVAL, "layernorm_stats: stats must be 8-byte aligned");
    if (overlaps(x, rows * dim * dtype_size(dt), stats, rows * 8))
        return fail(HS_EINVAL, "layernorm_stats: stats overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16 ? launch_stats<f16>(st, x, stats, rows, dim, eps)
                        : launch_stats<float>(st, x, stats, rows, dim, eps);
}

extern "C" hs_status hs_bias_ls_residual_layernorm(hs_stream_t stream, hs_dtype dt, const void* res,
                                                   const void* x, const float* bias,
                                                   const float* gamma, const float* ln_w,
                                                   const float* ln_b, void* out, void* normed,
                                                   int64_t rows, int32_t dim, float eps) {
    using namespace hs;
    const char* op = "bias_ls_residual_layernorm";
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "%s: unknown dtype %d", op, (int)dt);
    if (rows < 0 || dim <= 0) return fail(HS_EINVAL, "%s: rows %lld / dim %d", op, (long long)rows, dim);
    if (too_large(rows, dim)) return fail(HS_EINVAL, "%s: tensor too large", op);
    if (rows == 0) return HS_OK;
    if (!res || !x || !gamma || !ln_w || !ln_b || !out || !normed)
        return fail(HS_EINVAL, "%s: null buffer", op);
    const int64_t bytes = rows * dim * dtype_size(dt);
    if ((out != res && overlaps(out, bytes, res, bytes)) || (out != x && overlaps(out, bytes, x, bytes)))
        return fail(HS_EINVAL, "%s: out partially overlaps res or x", op);
    if (overlaps(normed, bytes, res, bytes) || overlaps(normed, bytes, x, bytes) ||
        overlaps(normed, bytes, out, bytes))
        return fail(HS_EINVAL, "%s: normed overlaps res, x or out", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool fused = dt == HS_F16 ? launch_ls_ln<f16>(st, res, x, bias, gamma, ln_w, ln_b, out,
                                                       normed, rows, dim, eps)
                                    : launch_ls_ln<float>(st, res, x, bias, gamma, ln_w, ln_b, out,
                                                          normed, rows, dim, eps);
    if (fused) return check_launch(op);
    // other widths and alignments: the two single ops, which the fused
    // kernel reproduces bit for bit
    const hs_status rc = hs_bias_ls_residual(stream, dt, res, x, bias, gamma, out, rows, dim);
    if (rc != HS_OK) return rc;
    return hs_layernorm(stream, dt, out, ln_w, ln_b, normed, rows, dim, eps);
}
