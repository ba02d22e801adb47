// Shared device and host helpers for the gfx950 kernels of libheadshot_hip.
//
// Device side: 16-byte vector loads/stores, f16 <-> f32 conversion (round to
// nearest even), and wave64 reductions built on DPP lane permutes (no LDS).
// Host side: error reporting for the C ABI and launch-shape helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "headshot_hip.h"

namespace hs {

// ---------------------------------------------------------------------------
// host: errors

// Records a message for hs_last_error() and returns `code`.
hs_status fail(hs_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// HS_EHIP with the pending launch error if the last launch failed, else HS_OK.
hs_status check_launch(const char* what);
// Number of compute units of the current device (cached per device).
int num_cus();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// [a, a+na) and [b, b+nb) byte ranges overlap.
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
    auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return na > 0 && nb > 0 && pa < pb + static_cast<uintptr_t>(nb) &&
           pb < pa + static_cast<uintptr_t>(na);
}

inline int64_t dtype_size(hs_dtype dt) { return dt == HS_F16 ? 2 : 4; }

inline bool valid_dtype(hs_dtype dt) { return dt == HS_F32 || dt == HS_F16; }

// Tensors of 2^40 elements or more are refused, so that byte counts and
// offsets stay far inside int64_t (rows and cols non-negative).
constexpr int64_t kMaxElems = int64_t{1} << 40;
inline bool too_large(int64_t rows, int64_t cols) { return cols > 0 && rows >= kMaxElems / cols; }

// ---------------------------------------------------------------------------
// device: storage types and 16-byte vectors

using f16 = _Float16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Elements of T in one 16-byte vector.
template <typename T>
struct Vec {
    static constexpr int N = 16 / sizeof(T);
};

__device__ __forceinline__ u32x4 ld16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Streaming variants for activations, which every op touches exactly once:
// non-temporal loads and stores. On MI355X these sustain ~6.2 TB/s for a
// 1:1 read/write stream against ~4.3-5.0 TB/s for plain accesses in the
// same launch shapes. Parameters (weights, biases, tables) use the cached
// ld16/ld_f32x4 paths because every wave rereads them.
#ifndef HS_NT
#define HS_NT 1
#endif

__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_nt(void* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

template <bool NT = (HS_NT != 0)>
__device__ __forceinline__ u32x4 ld_stream(const void* p) {
    if constexpr (NT) return ld16_nt(p);
    return ld16(p);
}
template <bool NT = (HS_NT != 0)>
__device__ __forceinline__ void st_stream(void* p, u32x4 v) {
    if constexpr (NT)
        st16_nt(p, v);
    else
        st16(p, v);
}

template <typename V>
__device__ __forceinline__ V ld_stream_as(const V* p) {
    if constexpr (HS_NT) return __builtin_nontemporal_load(p);
    return *p;
}
template <typename V>
__device__ __forceinline__ void st_stream_as(V* p, V v) {
    if constexpr (HS_NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

__device__ __forceinline__ float4 ld_f32x4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

// Scalar reinterpretation, always of a value. Bit-casting a vector element
// expression such as v[k] in place reads element 0 with this compiler, so
// elements are passed through these by-value helpers.
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ f16x2 u2h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t h22u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// Unpack a 16-byte vector of T into f32.
__device__ __forceinline__ void unpack(u32x4 v, float (&f)[8], f16) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const f16x2 h = u2h2(v[k]);
        f[2 * k] = static_cast<float>(h.x);
        f[2 * k + 1] = static_cast<float>(h.y);
    }
}
__device__ __forceinline__ void unpack(u32x4 v, float (&f)[4], float) {
#pragma unroll
    for (int k = 0; k < 4; k++) f[k] = u2f(v[k]);
}

// Pack f32 values into a 16-byte vector of T (f16: round to nearest even).
__device__ __forceinline__ u32x4 pack(const float (&f)[8], f16) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        f16x2 h;
        h.x = static_cast<f16>(f[2 * k]);
        h.y = static_cast<f16>(f[2 * k + 1]);
        v[k] = h22u(h);
    }
    return v;
}
__device__ __forceinline__ u32x4 pack(const float (&f)[4], float) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = f2u(f[k]);
    return v;
}

// Exact-erf GELU, gelu.wesl:18-38: 0.5*v*(1 + erf(v/sqrt(2))) with erf by
// Abramowitz & Stegun 7.1.26, erf(z) = sign(z)*(1 - P(t)*t*exp(-z^2)),
// t = 1/(1 + p*|z|). Evaluated in f32 from h = v/2 (exact), with the
// scale folded into the constants (z = v/sqrt(2) is never formed) and the
// sign folded into the final multiply-add, since 0.5*v*sign(v) = |h|:
//   gelu(v) = h + |h| * (1 - P(t)*t*2^(-(h*2k)^2)),
//   t = 1/(1 + (2p/sqrt(2))*|h|),  k = sqrt(log2(e)/2).
// 2p/sqrt(2) * |h| and 2k * h equal p/sqrt(2) * |v| and k * v exactly (the
// factor 2 is exact), so starting from h changes no rounding. 12 VALU
// operations per element from h, including one v_rcp_f32 and one
// v_exp_f32 (both ~1 ulp); the folded constants move the result by a few
// f32 ulps against the shader's operand order, far inside the parity bars.
constexpr float kGeluAsP = 0.3275911f * 0.70710678118654752f;  // p / sqrt(2)
constexpr float kGeluExpK = 0.84932180028801904f;               // sqrt(log2(e) / 2)

__device__ __forceinline__ float gelu_half(float h) {
    const float t = __builtin_amdgcn_rcpf(fmaf(2.0f * kGeluAsP, fabsf(h), 1.0f));
    float p = fmaf(1.061405429f, t, -1.453152027f);
    p = fmaf(p, t, 1.421413741f);
    p = fmaf(p, t, -0.284496736f);
    p = fmaf(p, t, 0.254829592f);
    p = p * t;
    const float w = h * (2.0f * kGeluExpK);
    const float e = __builtin_amdgcn_exp2f(-(w * w));  // exp(-v^2/2)
    return fmaf(fabsf(h), fmaf(-p, e, 1.0f), h);
}
__device__ __forceinline__ float gelu_f(float v) { return gelu_half(0.5f * v); }

// v as a materialised f32 value. The reference computes in f32 and then
// stores its storage type: two roundings. Left alone, the compiler may fold
// a multiply-add and the following f16 conversion into one v_fma_mix_f16
// (one rounding, from the exact result), which differs exactly at f16 ties,
// and it makes that choice differently in different kernels.
__device__ __forceinline__ float as_f32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// The value a later dispatch would read back after storing v as T: the
// reference rounds to its storage type after every dispatch, and the fused
// kernels reproduce those rounding points in registers.
__device__ __forceinline__ float storage_round(float v, f16) {
    return static_cast<float>(static_cast<f16>(as_f32(v)));
}
__device__ __forceinline__ float storage_round(float v, float) { return v; }

// One LayerScale + residual output value before its storage rounding
// (residual_ls.wesl:28, res + gamma * x): the multiply-add as fmaf, the f32
// result materialised, so every kernel that applies it rounds the same way.
__device__ __forceinline__ float ls_affine(float res, float gamma, float x) {
    return as_f32(fmaf(gamma, x, res));
}

// One LayerNorm output value before its storage rounding: (x - mean) * inv *
// w + b, the multiply-add spelled as fmaf and the f32 result materialised.
// Every kernel that normalises a row (the LayerNorm kernels and the linear
// layers' LayerNorm prologue) computes it through this helper, so a row
// normalised inside a product is bit-identical to the row hs_layernorm
// stores.
__device__ __forceinline__ float ln_affine(float x, float mean, float inv, float w, float b) {
    return as_f32(fmaf((x - mean) * inv, w, b));
}

template <typename T>
__device__ __forceinline__ float load_elem(const T* p) {
    return static_cast<float>(*p);
}
template <typename T>
__device__ __forceinline__ void store_elem(T* p, float v) {
    *p = static_cast<T>(v);
}

// ---------------------------------------------------------------------------
// device: wave64 lane permutes (DPP) and reductions

// dpp_ctrl encodings (GFX9 DPP).
constexpr int kQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <- lane 7-i within each 8 lanes
constexpr int kRowMirror = 0x140;      // lane i <- lane 15-i within each 16 lanes
constexpr int kRowBcast15 = 0x142;     // lane 15 of each row -> next row
constexpr int kRowBcast31 = 0x143;     // lane 31 -> rows 2 and 3

template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                           BANK_MASK, false));
}

// Sum over each aligned group of 8 lanes; every lane receives its group's sum.
__device__ __forceinline__ float sum8(float v) {
    v += dpp<kQuadXor1>(v);
    v += dpp<kQuadXor2>(v);
    v += dpp<kRowHalfMirror>(v);
    return v;
}

// Sum over each aligned group of 16 lanes; every lane receives the sum.
__device__ __forceinline__ float sum16(float v) {
    v = sum8(v);
    v += dpp<kRowMirror>(v);
    return v;
}

// Sum over the whole wave64, returned wave-uniform (scalar register).
__device__ __forceinline__ float wave_sum(float v) {
    v = sum16(v);
    v += dpp<kRowBcast15, 0xA>(v);
    v += dpp<kRowBcast31, 0xC>(v);
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over lane groups of G (8, 16 or 64) lanes.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 8 || G == 16 || G == 64, "group of 8, 16 or 64 lanes");
    if constexpr (G == 8) return sum8(v);
    if constexpr (G == 16) return sum16(v);
    if constexpr (G == 64) return wave_sum(v);
}

// Value held by the mirror-partner lane within a group of G lanes
// (lane i <-> G-1-i).
template <int G>
__device__ __forceinline__ float group_mirror(float v) {
    static_assert(G == 8 || G == 16, "mirror within 8 or 16 lanes");
    if constexpr (G == 8) return dpp<kRowHalfMirror>(v);
    if constexpr (G == 16) return dpp<kRowMirror>(v);
}

// QK-norm and rotate-half RoPE of one 64-wide head vector spread over a
// group of G lanes, V = 64 / G values per lane. The lane of piece p < G / 2
// holds channels [p V, p V + V), the lane of piece p >= G / 2 the matching
// upper channels [32 + (G - 1 - p) V, + V), so a channel's RoPE partner sits
// in the mirror lane. LayerNorm over the 64 channels with f32 statistics
// (eps, weight wr, bias br of the lane's channels), the storage rounding the
// reference applies between its layernorm and rope_apply dispatches, then,
// when rot, the rotation with cs = cos and sn = -sin (lower lanes) or +sin
// (upper lanes) of the lane's channels. Every lane of a group must take the
// same branches (the reductions and the mirror read across the group). The
// results are f32 values the caller rounds to T once more on store, as the
// reference's rope_apply output is.
template <typename T, int G, bool NORM, int V>
__device__ __forceinline__ void qk_norm_rope_vec(float (&f)[V], const float (&wr)[V],
                                                 const float (&br)[V], float eps, bool rot,
                                                 const float (&cs)[V], const float (&sn)[V]) {
    static_assert(G * V == 64, "one 64-wide head vector per group");
    if constexpr (NORM) {
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < V; k++) sum += f[k];
        const float mean = group_sum<G>(sum) / 64.0f;
        // the multiply-adds are spelled out as fmaf so that every kernel
        // sharing this code rounds them the same way
        float q = 0.0f;
#pragma unroll
        for (int k = 0; k < V; k++) {
            const float d = f[k] - mean;
            q = fmaf(d, d, q);
        }
        const float var = group_sum<G>(q) / 64.0f;
        const float inv = rsqrtf(var + eps);
#pragma unroll
        for (int k = 0; k < V; k++) f[k] = storage_round(fmaf((f[k] - mean) * inv, wr[k], br[k]), T{});
    }
    if (rot) {
#pragma unroll
        for (int k = 0; k < V; k++) f[k] = as_f32(fmaf(f[k], cs[k], group_mirror<G>(f[k]) * sn[k]));
    }
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Index of the calling wave within its workgroup, as a wave-uniform (scalar)
// value: the compiler cannot prove threadIdx.x >> 6 uniform by itself, and
// without this it keeps every index derived from it, and the integer
// divisions on it, in vector registers and vector instructions.
__device__ __forceinline__ int wave_in_block() {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

}  // namespace hs
