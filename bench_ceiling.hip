// Data-movement ceilings for bench.py: each kernel moves the same bytes as
// one of the fused ops, in that op's access pattern, with no arithmetic
// beyond what the byte mix needs. Timed beside the op, the pair says how
// much of the op's distance from the 8 TB/s HBM peak is the memory system's
// own limit for that pattern and how much is the op's.
//
//   copy   1 read : 1 write, contiguous            (layernorm, bias_gelu)
//   add2   2 reads : 1 write, contiguous           (bias_ls_residual)
//   heads  token-major (S*T, 16*64) f16 -> head-major (S, 16, T, 64), two
//          tensors in one launch, 8 heads' 128-byte vectors per store, a
//          wave per two whole rows or per one token's 8-head chunk (chunk
//          by chunk): the fused QK-norm + RoPE pair kernel's two orders
//          (qknorm_rope)
//   cast   f32 rows in, f16 rows out, contiguous   (assembly's byte mix)
//   widen  f16 in, f32 out: 1 read : 2 written     (the cache build's mix)
//   inplace  1 read : 1 write of the same buffer   (rope_apply in place)
//   add2w2 2 reads : 2 writes, contiguous          (bias_ls_residual_layernorm)
//
// Also a shader-clock sampler (hsc_clock) for timing kernels whose speed
// follows the clock the chip's power management sets.
//
// Each kernel runs with non-temporal (streaming) or ordinary cached loads and
// stores, the two policies the library's kernels use, and in two launch
// shapes: four 16-byte vectors per lane (two whole rows per wave for heads)
// or one (one token's 8-head chunk per wave); the bench takes the fastest as
// the ceiling (a
// bare copy is fastest with one vector per lane, 82% of peak against 78%
// with four, while the ops, with their arithmetic, run best with their own
// shapes). Not part of libheadshot_hip: built into bench_ceiling.so next to
// bench.py.
#include "hs_common.hpp"

namespace {

using hs::f16;
using hs::u32x4;

constexpr int kBlock = 256;

template <bool NT, typename V>
__device__ __forceinline__ V ld(const V* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT, typename V>
__device__ __forceinline__ void st(V* p, V v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// Vectors [w * 64 U, (w + 1) * 64 U) for wave w: U wave-contiguous 1 KiB
// pieces per wave.
template <bool NT, int U>
__global__ __launch_bounds__(kBlock) void copy_kernel(const u32x4* __restrict__ a,
                                                      u32x4* __restrict__ o, int64_t n) {
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * U +
                         (threadIdx.x & 63);
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) r[u] = ld<NT>(a + base + u * 64);
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) st<NT>(o + base + u * 64, r[u]);
}

template <bool NT, int U>
__global__ __launch_bounds__(kBlock) void add2_kernel(const u32x4* __restrict__ a,
                                                      const u32x4* __restrict__ b,
                                                      u32x4* __restrict__ o, int64_t n) {
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * U +
                         (threadIdx.x & 63);
    u32x4 ra[U], rb[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) ra[u] = ld<NT>(a + base + u * 64), rb[u] = ld<NT>(b + base + u * 64);
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) st<NT>(o + base + u * 64, ra[u] + rb[u]);
}

// Two tensors, K tokens per wave. Whole rows (SPLIT false): waves [0, W)
// copy the first tensor, [W, 2W) the second, W = ceil(tokens / K), each
// token's two 1 KiB loads (8 heads each). SPLIT: a wave takes one 1 KiB
// chunk (8 heads) of its tokens and the grid runs (chunk, tensor) units
// chunk by chunk, the order the QK-norm pair uses for long sequences. A
// store writes 8 heads' vectors to their head-major rows.
template <bool NT, int K, bool SPLIT>
__global__ __launch_bounds__(kBlock) void heads_kernel(const f16* __restrict__ x0,
                                                       const f16* __restrict__ x1,
                                                       f16* __restrict__ o0, f16* __restrict__ o1,
                                                       int64_t tokens, int seq) {
    constexpr int H = 16, D = 64, NC = SPLIT ? 1 : 2;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + hs::wave_in_block();
    const int64_t per = (tokens + K - 1) / K;
    int which, c0 = 0;
    int64_t u0;
    if constexpr (SPLIT) {
        const int64_t unit = wave / per;
        if (unit > 3) return;
        c0 = static_cast<int>(unit / 2), which = static_cast<int>(unit % 2);
        u0 = (wave - unit * per) * K;
    } else {
        which = wave >= per ? 1 : 0;
        u0 = (wave - which * per) * K;
        if (wave >= 2 * per) return;
    }
    if (u0 >= tokens) return;
    const f16* x = which ? x1 : x0;
    f16* o = which ? o1 : o0;
    const int lane = hs::lane_id(), gsub = lane >> 3, ch = (lane & 7) * 8;
    u32x4 r[K][NC];
#pragma unroll
    for (int k = 0; k < K; k++)
#pragma unroll
        for (int c = 0; c < NC; c++)
            if (u0 + k < tokens) r[k][c] = ld<NT>(reinterpret_cast<const u32x4*>(x + (u0 + k) * (H * D) + ((c0 + c) * 8 + gsub) * D + ch));
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int64_t tok = u0 + k;
        if (tok >= tokens) break;
        const int64_t s = tok / seq, t = tok - s * seq;
#pragma unroll
        for (int c = 0; c < NC; c++)
            st<NT>(reinterpret_cast<u32x4*>(o + ((s * H + (c0 + c) * 8 + gsub) * seq + t) * D + ch), r[k][c]);
    }
}

// n f32 -> f16, four elements (16 bytes in, 8 out) per lane per step.
template <bool NT, int U>
__global__ __launch_bounds__(kBlock) void cast_kernel(const float* __restrict__ a,
                                                      f16* __restrict__ o, int64_t n) {
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * U +
                         (threadIdx.x & 63);
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if ((base + u * 64) * 4 < n) r[u] = ld<NT>(reinterpret_cast<const u32x4*>(a + (base + u * 64) * 4));
#pragma unroll
    for (int u = 0; u < U; u++) {
        if ((base + u * 64) * 4 >= n) continue;
        hs::f16x2 lo, hi;
        lo.x = static_cast<f16>(hs::u2f(r[u][0])), lo.y = static_cast<f16>(hs::u2f(r[u][1]));
        hi.x = static_cast<f16>(hs::u2f(r[u][2])), hi.y = static_cast<f16>(hs::u2f(r[u][3]));
        hs::u32x2 v;
        v[0] = hs::h22u(lo), v[1] = hs::h22u(hi);
        st<NT>(reinterpret_cast<hs::u32x2*>(o + (base + u * 64) * 4), v);
    }
}

// n f16 -> f32, eight elements (16 bytes in, 32 out) per lane per step.
template <bool NT, int U>
__global__ __launch_bounds__(kBlock) void widen_kernel(const u32x4* __restrict__ a,
                                                       u32x4* __restrict__ o, int64_t n) {
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * U +
                         (threadIdx.x & 63);
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) r[u] = ld<NT>(a + base + u * 64);
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (base + u * 64 >= n) continue;
        u32x4 lo, hi;
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const hs::f16x2 p = hs::u2h2(r[u][w]), q = hs::u2h2(r[u][w + 2]);
            lo[2 * w] = hs::f2u(static_cast<float>(p.x)), lo[2 * w + 1] = hs::f2u(static_cast<float>(p.y));
            hi[2 * w] = hs::f2u(static_cast<float>(q.x)), hi[2 * w + 1] = hs::f2u(static_cast<float>(q.y));
        }
        st<NT>(o + 2 * (base + u * 64), lo);
        st<NT>(o + 2 * (base + u * 64) + 1, hi);
    }
}

// o = a + b and o2 = a - b (as 32-bit lanes), n 16-byte vectors each.
template <bool NT, int U>
__global__ __launch_bounds__(kBlock) void add2w2_kernel(const u32x4* __restrict__ a,
                                                        const u32x4* __restrict__ b,
                                                        u32x4* __restrict__ o,
                                                        u32x4* __restrict__ o2, int64_t n) {
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * U +
                         (threadIdx.x & 63);
    u32x4 ra[U], rb[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) ra[u] = ld<NT>(a + base + u * 64), rb[u] = ld<NT>(b + base + u * 64);
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) {
            st<NT>(o + base + u * 64, ra[u] + rb[u]);
            st<NT>(o2 + base + u * 64, ra[u] - rb[u]);
        }
}

// n 16-byte vectors read and written back in place (each lane its own).
template <bool NT, int U>
__global__ __launch_bounds__(kBlock) void inplace_kernel(u32x4* a, int64_t n) {
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~63)) * U +
                         (threadIdx.x & 63);
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) r[u] = ld<NT>(a + base + u * 64);
#pragma unroll
    for (int u = 0; u < U; u++)
        if (base + u * 64 < n) st<NT>(a + base + u * 64, r[u] + u32x4{1, 1, 1, 1});
}

int64_t blocks_for(int64_t lanes_work) { return (lanes_work + kBlock - 1) / kBlock; }

// U: 16-byte vectors per lane (copy, add2, cast) or tokens per wave (heads).
template <bool NT, int U>
int run(int kind, const void* a, const void* b, void* o, void* o2, int64_t n, int32_t s,
        int32_t t, hipStream_t stream) {
    switch (kind) {
        case 0:
        case 1: {
            const int64_t blocks = blocks_for((n + U - 1) / U);
            if (blocks == 0) return 0;
            if (blocks * kBlock >= (int64_t{1} << 32)) return -1;  // 32-bit grid size
            if (kind == 0)
                copy_kernel<NT, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                    static_cast<const u32x4*>(a), static_cast<u32x4*>(o), n);
            else
                add2_kernel<NT, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                    static_cast<const u32x4*>(a), static_cast<const u32x4*>(b),
                    static_cast<u32x4*>(o), n);
            break;
        }
        case 2: {
            // four vectors per lane: two whole rows per wave; one: one token's
            // 1 KiB chunk per wave, chunk by chunk
            constexpr int K = U == 1 ? 1 : 2;
            constexpr bool SPLIT = U == 1;
            const int64_t tokens = static_cast<int64_t>(s) * t;
            const int64_t waves = (SPLIT ? 4 : 2) * ((tokens + K - 1) / K);
            const int64_t blocks = (waves + 3) / 4;
            if (blocks == 0) return 0;
            if (blocks * kBlock >= (int64_t{1} << 32)) return -1;  // 32-bit grid size
            heads_kernel<NT, K, SPLIT><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                static_cast<const f16*>(a), static_cast<const f16*>(b), static_cast<f16*>(o),
                static_cast<f16*>(o2), tokens, t);
            break;
        }
        case 3: {
            if (n % 4 != 0) return -1;
            const int64_t blocks = blocks_for((n / 4 + U - 1) / U);
            if (blocks == 0) return 0;
            if (blocks * kBlock >= (int64_t{1} << 32)) return -1;  // 32-bit grid size
            cast_kernel<NT, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                static_cast<const float*>(a), static_cast<f16*>(o), n);
            break;
        }
        case 6: {
            const int64_t blocks = blocks_for((n + U - 1) / U);
            if (blocks == 0) return 0;
            if (blocks * kBlock >= (int64_t{1} << 32)) return -1;  // 32-bit grid size
            add2w2_kernel<NT, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                static_cast<const u32x4*>(a), static_cast<const u32x4*>(b), static_cast<u32x4*>(o),
                static_cast<u32x4*>(o2), n);
            break;
        }
        case 4:
        case 5: {
            const int64_t blocks = blocks_for((n + U - 1) / U);
            if (blocks == 0) return 0;
            if (blocks * kBlock >= (int64_t{1} << 32)) return -1;  // 32-bit grid size
            if (kind == 4)
                widen_kernel<NT, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                    static_cast<const u32x4*>(a), static_cast<u32x4*>(o), n);
            else
                inplace_kernel<NT, U><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream>>>(
                    static_cast<u32x4*>(o), n);
            break;
        }
        default:
            return -1;
    }
    return static_cast<int>(hipGetLastError());
}

// Shader-clock samples: one wave records (s_memtime, s_memrealtime) n
// times, each once the 100 MHz real-time counter has advanced by `step`
// ticks since the previous sample, with vector stores from lane 0 (every
// wait ends as the counter advances). On a second stream beside the kernels
// under study, the two counters' advance between samples gives the shader
// clock; with n = 1 and step = 0 on the kernels' own stream, one sample
// marks a point of their sequence.
__global__ __launch_bounds__(64) void clock_kernel(unsigned long long* out, int n, int step) {
    for (int i = 0; i < n; i++) {
        const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
        unsigned long long r = r0;
        while (r - r0 < static_cast<unsigned long long>(step)) r = __builtin_amdgcn_s_memrealtime();
        const unsigned long long c = __builtin_amdgcn_s_memtime();
        if (threadIdx.x == 0) {
            out[2 * i] = c;
            out[2 * i + 1] = r;
        }
    }
}

}  // namespace

extern "C" {

// n samples of (shader clock count, 100 MHz real-time count) into out
// (2n 64-bit values), step real-time ticks apart (clock_kernel). Returns 0,
// -1 for an argument the kernel does not take, or the launch's HIP error.
int hsc_clock(unsigned long long* out, int n, int step, hipStream_t stream) {
    if (!out || n < 1 || step < 0) return -1;
    clock_kernel<<<dim3(1), dim3(64), 0, stream>>>(out, n, step);
    return static_cast<int>(hipGetLastError());
}

// kind 0 copy / 1 add2: n 16-byte vectors (a, b -> o). kind 2 heads: s
// frames of t tokens, a and b -> o and o2. kind 3 cast: n f32 elements
// (n % 4 == 0). kind 4 widen: n 16-byte f16 vectors of a -> 2n 16-byte f32
// vectors of o. kind 5 inplace: n 16-byte vectors of o, read and rewritten.
// kind 6 add2w2: n 16-byte vectors, a and b -> o = a + b, o2 = a - b.
// shape 0-7: bit 0 set = cached loads and stores (clear: non-temporal);
// shapes 0-1 four 16-byte vectors per lane (heads: two whole rows per
// wave), 2-3 one (heads: one token's 8-head chunk per wave, chunk by
// chunk), 4-5 two, 6-7 eight (heads: as 0-1). Buffers are 16-byte aligned
// and sized by the caller. Returns 0, or -1 for an argument the kernels do
// not take, or the HIP error code of the launch.
int hsc_run(int kind, int shape, const void* a, const void* b, void* o, void* o2, int64_t n,
            int32_t s, int32_t t, hipStream_t stream) {
    if (n < 0 || s < 0 || t < 0 || shape < 0 || shape > 7) return -1;
    switch (shape) {
        case 0: return run<true, 4>(kind, a, b, o, o2, n, s, t, stream);
        case 1: return run<false, 4>(kind, a, b, o, o2, n, s, t, stream);
        case 2: return run<true, 1>(kind, a, b, o, o2, n, s, t, stream);
        case 3: return run<false, 1>(kind, a, b, o, o2, n, s, t, stream);
        case 4: return run<true, 2>(kind, a, b, o, o2, n, s, t, stream);
        case 5: return run<false, 2>(kind, a, b, o, o2, n, s, t, stream);
        case 6: return run<true, 8>(kind, a, b, o, o2, n, s, t, stream);
        default: return run<false, 8>(kind, a, b, o, o2, n, s, t, stream);
    }
}

}  // extern "C"
