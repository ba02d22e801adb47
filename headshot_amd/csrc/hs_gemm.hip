// Linear layers for gfx950 (replaces GpuContext::linear, engine/ops.rs:81-128,
// shaders/linear_wmma.wgsl and shaders/linear.wesl): out (M, N) = x (M, K)
// @ w (N, K)^T + bias (N, f32), with the epilogues the trunk's blocks apply
// to the result fused into the store (model/block.rs:150-176):
//   EPI_BIAS      out = f16(acc + bias)                       (qkv, linear)
//   EPI_GELU      out = f16(gelu(acc + bias))                 (fc1 + GELU)
//   EPI_LS        out = f16(res + gamma * f16(acc + bias))    (proj/fc2 +
//                                                 LayerScale + residual)
// so the activation between a GEMM and its elementwise op never crosses HBM.
//
// Fast path (f16, N % 128 == 0, K % 32 == 0): matrix-core GEMM. A workgroup
// of 4 waves computes a 256 (rows) x 128 (columns) tile of out, K in steps of
// 32 staged through LDS (double-buffered, the next step prefetched into
// registers while the current one computes). Both operands are K-contiguous
// rows (x rows, w rows), which is exactly the operand layout of
// v_mfma_f32_32x32x16_f16, so both come from LDS with 16-byte reads. Each
// wave owns 128 rows x 64 columns and computes the transposed tile
// out^T = w x^T: its accumulators then hold, per lane, 4 consecutive output
// columns of one output row, so the epilogue reads bias/gamma/residual and
// writes out in 8-byte pieces. Rows past M are clamped on load and masked on
// store.
//
// Generic path (f32, or shapes the fast path does not cover): a tiled
// scalar kernel, f32 accumulation in K order.
#include <math.h>

#include "hs_common.hpp"

namespace hs {
namespace {

typedef f16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum Epi { EPI_BIAS = 0, EPI_GELU = 1, EPI_LS = 2 };

// Exact-erf GELU in the A&S 7.1.26 form used by the elementwise GELU kernel
// (gelu.wesl:18-38 with the 1/sqrt(2) folded into the constants).
__device__ __forceinline__ float gelu_erf(float v) {
    constexpr float kAsP = 0.3275911f * 0.70710678118654752f;
    constexpr float kExpK = 0.84932180028801904f;
    const float h = 0.5f * v;
    const float t = __builtin_amdgcn_rcpf(fmaf(kAsP, fabsf(v), 1.0f));
    float p = fmaf(1.061405429f, t, -1.453152027f);
    p = fmaf(p, t, 1.421413741f);
    p = fmaf(p, t, -0.284496736f);
    p = fmaf(p, t, 0.254829592f);
    p = p * t;
    const float w = v * kExpK;
    const float e = __builtin_amdgcn_exp2f(-(w * w));
    return fmaf(fabsf(h), fmaf(-p, e, 1.0f), h);
}

// ---------------------------------------------------------------------------
// matrix-core path

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 256;  // output rows per workgroup
constexpr int kBN = 128;  // output columns per workgroup
constexpr int kBK = 32;   // K per LDS stage
constexpr int kPitch = kBK + 8;  // halves per LDS row: 80 B, conflict-free 16-byte reads
constexpr int kXChunks = kBM * kBK / 8;  // 16-byte chunks per stage
constexpr int kWChunks = kBN * kBK / 8;
constexpr int kXPer = kXChunks / kThreads;
constexpr int kWPer = kWChunks / kThreads;
static_assert(kXChunks % kThreads == 0 && kWChunks % kThreads == 0, "stage split");

struct GemmSmem {
    f16 x[2][kBM * kPitch];
    f16 w[2][kBN * kPitch];
};

struct StageRegs {
    u32x4 x[kXPer];
    u32x4 w[kWPer];
};

__device__ __forceinline__ h8 as_h8(u32x4 v) { return __builtin_bit_cast(h8, v); }

// 16-byte chunk c of a stage: row c / 4, halves (c % 4) * 8 .. + 8 of the
// 32-wide K slice. x rows past M read row M - 1 (their outputs are masked).
__device__ __forceinline__ void load_stage(StageRegs& r, const f16* x, const f16* w, int64_t m0,
                                           int64_t n0, int M, int K, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < kXPer; i++) {
        const int c = tid + i * kThreads;
        const int64_t row = min(m0 + c / 4, static_cast<int64_t>(M) - 1);
        r.x[i] = ld16(x + row * K + k0 + (c % 4) * 8);
    }
#pragma unroll
    for (int i = 0; i < kWPer; i++) {
        const int c = tid + i * kThreads;
        r.w[i] = ld16(w + (n0 + c / 4) * K + k0 + (c % 4) * 8);
    }
}

__device__ __forceinline__ void store_stage(const StageRegs& r, GemmSmem& sm, int buf, int tid) {
#pragma unroll
    for (int i = 0; i < kXPer; i++) {
        const int c = tid + i * kThreads;
        st16(&sm.x[buf][(c / 4) * kPitch + (c % 4) * 8], r.x[i]);
    }
#pragma unroll
    for (int i = 0; i < kWPer; i++) {
        const int c = tid + i * kThreads;
        st16(&sm.w[buf][(c / 4) * kPitch + (c % 4) * 8], r.w[i]);
    }
}

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
    f16x2 h;
    h.x = static_cast<f16>(a), h.y = static_cast<f16>(b);
    return h22u(h);
}

// Grid: tiles_m * tiles_n workgroups, column tiles fastest, so workgroups
// running together share their x rows.
template <int EPI>
__global__ __launch_bounds__(kThreads) void gemm_f16_kernel(
    const f16* __restrict__ x, const f16* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ gamma, const f16* res, f16* out, int M, int N, int K,
    int tiles_n) {
    __shared__ GemmSmem sm;
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x / tiles_n) * kBM;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x % tiles_n) * kBN;
    const int wm = (wave >> 1) * 128;  // wave's rows within the tile
    const int wn = (wave & 1) * 64;    // wave's columns within the tile

    // acc[a][b]: out^T block of columns wn + 32 a .. + 32 (MFMA rows) and
    // rows wm + 32 b .. + 32 (MFMA columns); register r of lane (l32, hh)
    // is column 8 (r / 4) + 4 hh + r % 4, row l32 of the block.
    f32x16 acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f32x16{};

    const int nsteps = K / kBK;
    StageRegs pre;
    load_stage(pre, x, w, m0, n0, M, K, 0, tid);
    store_stage(pre, sm, 0, tid);
    __syncthreads();
    for (int s = 0; s < nsteps; s++) {
        const int cur = s & 1;
        if (s + 1 < nsteps) load_stage(pre, x, w, m0, n0, M, K, (s + 1) * kBK, tid);
        const f16* wa = &sm.w[cur][(wn + l32) * kPitch + 8 * hh];
        const f16* xb = &sm.x[cur][(wm + l32) * kPitch + 8 * hh];
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ks++) {
            h8 A[2], B[4];
#pragma unroll
            for (int a = 0; a < 2; a++) A[a] = as_h8(ld16(wa + a * 32 * kPitch + 16 * ks));
#pragma unroll
            for (int b = 0; b < 4; b++) B[b] = as_h8(ld16(xb + b * 32 * kPitch + 16 * ks));
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 4; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[a], B[b], acc[a][b], 0, 0, 0);
        }
        if (s + 1 < nsteps) store_stage(pre, sm, cur ^ 1, tid);
        __syncthreads();
    }

    // Epilogue: per (a, b) and r4, lane (l32, hh) owns row m, columns
    // n .. n + 4 of out.
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int64_t m = m0 + wm + 32 * b + l32;
        if (m >= M) continue;
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const int64_t n = n0 + wn + 32 * a + 8 * r4 + 4 * hh;
                float v[4];
                const float4 bv = bias ? ld_f32x4(bias + n) : float4{0.0f, 0.0f, 0.0f, 0.0f};
                v[0] = acc[a][b][4 * r4] + bv.x, v[1] = acc[a][b][4 * r4 + 1] + bv.y;
                v[2] = acc[a][b][4 * r4 + 2] + bv.z, v[3] = acc[a][b][4 * r4 + 3] + bv.w;
                if constexpr (EPI == EPI_GELU) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = gelu_erf(v[e]);
                } else if constexpr (EPI == EPI_LS) {
                    // the GEMM epilogue's f16 store, then res + gamma * x
                    const float4 g = ld_f32x4(gamma + n);
                    const u32x2 rw = *reinterpret_cast<const u32x2*>(res + m * N + n);
                    const f16x2 r01 = u2h2(rw[0]), r23 = u2h2(rw[1]);
                    v[0] = fmaf(g.x, static_cast<float>(static_cast<f16>(v[0])), static_cast<float>(r01.x));
                    v[1] = fmaf(g.y, static_cast<float>(static_cast<f16>(v[1])), static_cast<float>(r01.y));
                    v[2] = fmaf(g.z, static_cast<float>(static_cast<f16>(v[2])), static_cast<float>(r23.x));
                    v[3] = fmaf(g.w, static_cast<float>(static_cast<f16>(v[3])), static_cast<float>(r23.y));
                }
                u32x2 o;
                o[0] = pk_f16(v[0], v[1]), o[1] = pk_f16(v[2], v[3]);
                *reinterpret_cast<u32x2*>(out + m * N + n) = o;
            }
    }
}

// ---------------------------------------------------------------------------
// generic path: 64 x 64 output tile per 256 threads, 4 x 4 per thread,
// K in steps of 16 through LDS; f32 accumulation in K order.

constexpr int kGT = 64, kGK = 16;

template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_generic_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ gamma, const T* res, T* out, int M, int N, int K, int tiles_n) {
    __shared__ float xs[kGK][kGT + 1];
    __shared__ float ws[kGK][kGT + 1];
    const int64_t m0 = static_cast<int64_t>(blockIdx.x / tiles_n) * kGT;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x % tiles_n) * kGT;
    const int tr = threadIdx.x / 16, tc = threadIdx.x % 16;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += kGK) {
        for (int i = threadIdx.x; i < kGK * kGT; i += 256) {
            const int kk = i % kGK, rr = i / kGK;
            const int64_t xm = m0 + rr, wn = n0 + rr;
            const int kidx = k0 + kk;
            xs[kk][rr] = (xm < M && kidx < K) ? static_cast<float>(x[xm * K + kidx]) : 0.0f;
            ws[kk][rr] = (wn < N && kidx < K) ? static_cast<float>(w[wn * K + kidx]) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGK; kk++) {
            float xv[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = xs[kk][tr * 4 + i], wv[i] = ws[kk][tc * 4 + i];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] += xv[i] * wv[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + tr * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t n = n0 + tc * 4 + j;
            if (n >= N) continue;
            float v = acc[i][j] + (bias ? bias[n] : 0.0f);
            if constexpr (EPI == EPI_GELU) v = gelu_erf(v);
            if constexpr (EPI == EPI_LS)
                v = static_cast<float>(res[m * N + n]) + gamma[n] * storage_round(v, T{});
            out[m * N + n] = static_cast<T>(v);
        }
    }
}

template <int EPI>
hs_status launch(hipStream_t st, hs_dtype dt, const void* x, const void* w, const float* bias,
                 const float* gamma, const void* res, void* out, int M, int N, int K,
                 const char* op) {
    const bool fast = dt == HS_F16 && N % kBN == 0 && K % kBK == 0 && aligned16(x) && aligned16(w) &&
                      (!bias || aligned16(bias)) && (!gamma || aligned16(gamma)) &&
                      (reinterpret_cast<uintptr_t>(out) & 7u) == 0 &&
                      (!res || (reinterpret_cast<uintptr_t>(res) & 7u) == 0);
    if (fast) {
        const int tiles_n = N / kBN;
        const int64_t blocks = ceil_div(M, kBM) * tiles_n;
        gemm_f16_kernel<EPI><<<dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, st>>>(
            static_cast<const f16*>(x), static_cast<const f16*>(w), bias, gamma,
            static_cast<const f16*>(res), static_cast<f16*>(out), M, N, K, tiles_n);
        return check_launch(op);
    }
    const int tiles_n = static_cast<int>(ceil_div(N, kGT));
    const int64_t blocks = ceil_div(M, kGT) * tiles_n;
    if (dt == HS_F16)
        gemm_generic_kernel<f16, EPI><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, st>>>(
            static_cast<const f16*>(x), static_cast<const f16*>(w), bias, gamma,
            static_cast<const f16*>(res), static_cast<f16*>(out), M, N, K, tiles_n);
    else
        gemm_generic_kernel<float, EPI><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, st>>>(
            static_cast<const float*>(x), static_cast<const float*>(w), bias, gamma,
            static_cast<const float*>(res), static_cast<float*>(out), M, N, K, tiles_n);
    return check_launch(op);
}

hs_status check(const char* op, hs_dtype dt, const void* x, const void* w, const void* res,
                const void* out, int64_t M, int32_t N, int32_t K, bool needs_res) {
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "%s: unknown dtype", op);
    if (M < 0 || N < 0 || K < 0) return fail(HS_EINVAL, "%s: shape M=%lld N=%d K=%d", op, static_cast<long long>(M), N, K);
    if (M >= (int64_t{1} << 31) || M * N >= (int64_t{1} << 40) || M * K >= (int64_t{1} << 40))
        return fail(HS_EINVAL, "%s: too large", op);
    if (M == 0 || N == 0) return HS_OK;
    if (!x || !w || !out || (needs_res && !res)) return fail(HS_EINVAL, "%s: null buffer", op);
    const int64_t esz = dtype_size(dt);
    const int64_t ob = M * N * esz;
    if (overlaps(out, ob, x, M * K * esz) || overlaps(out, ob, w, int64_t{N} * K * esz))
        return fail(HS_EINVAL, "%s: out overlaps x or w", op);
    if (needs_res && res != out && overlaps(out, ob, res, ob))
        return fail(HS_EINVAL, "%s: out partially overlaps res", op);
    return HS_OK;
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_linear(hs_stream_t stream, hs_dtype dt, const void* x, const void* w,
                               const float* bias, void* out, int64_t m, int32_t n, int32_t k) {
    using namespace hs;
    const hs_status rc = check("linear", dt, x, w, nullptr, out, m, n, k, false);
    if (rc != HS_OK || m == 0 || n == 0) return rc;
    return launch<EPI_BIAS>(static_cast<hipStream_t>(stream), dt, x, w, bias, nullptr, nullptr, out,
                            static_cast<int>(m), n, k, "linear");
}

extern "C" hs_status hs_linear_gelu(hs_stream_t stream, hs_dtype dt, const void* x, const void* w,
                                    const float* bias, void* out, int64_t m, int32_t n, int32_t k) {
    using namespace hs;
    const hs_status rc = check("linear_gelu", dt, x, w, nullptr, out, m, n, k, false);
    if (rc != HS_OK || m == 0 || n == 0) return rc;
    return launch<EPI_GELU>(static_cast<hipStream_t>(stream), dt, x, w, bias, nullptr, nullptr, out,
                            static_cast<int>(m), n, k, "linear_gelu");
}

extern "C" hs_status hs_linear_ls_residual(hs_stream_t stream, hs_dtype dt, const void* x,
                                           const void* w, const float* bias, const float* gamma,
                                           const void* res, void* out, int64_t m, int32_t n,
                                           int32_t k) {
    using namespace hs;
    if (!gamma && m > 0 && n > 0) return fail(HS_EINVAL, "linear_ls_residual: null gamma");
    const hs_status rc = check("linear_ls_residual", dt, x, w, res, out, m, n, k, true);
    if (rc != HS_OK || m == 0 || n == 0) return rc;
    return launch<EPI_LS>(static_cast<hipStream_t>(stream), dt, x, w, bias, gamma, res, out,
                          static_cast<int>(m), n, k, "linear_ls_residual");
}
