// Non-causal attention for gfx950 (replaces the reference's attention.wesl
// and attn_merge.wesl, dispatched by engine/ops.rs:228-267 and called by
// model/block.rs:148-149): softmax(q k^T / sqrt(d)) v per (frame, head) over
// head-major (S, H, T, D) tensors, with the softmax statistics and the
// accumulation in f32, plus the (S, H, T, D) -> (S*T, H*D) head merge.
//
// Fast path (f16, D = 64): flash attention on the matrix cores. A wave owns
// 32 queries; a workgroup of kWaves waves shares 64-key K/V tiles staged in
// LDS (double-buffered, the next tile prefetched into registers while the
// current one computes). The wave computes the transposed score block
// S^T = K Q^T with v_mfma_f32_32x32x16_f16, so each lane holds one query's
// column (16 keys per 32-key block, lanes l and l+32 splitting the keys):
// the online-softmax max needs one cross-half exchange per tile and the row
// sums none until the end. P^T is rounded to f16 in registers and fed
// straight back as the B operand of O^T += V^T P^T; the V^T operand comes
// from row-major V in LDS through the gfx950 transposing read
// ds_read_b64_tr_b16, with the key order matching the order in which the
// score accumulator holds P^T. The running max is lazy: after the first
// tile a query keeps its reference max m and a tile's weights are computed
// against it without the tile max; only when a lane's row sum over the tile
// exceeds 2^15 (a weight might then overflow f16) does the tile take the
// max path, which moves m if the tile's scores exceed it by more than 2^8
// and rescales the output. When many sequences have a partial last query
// tile (the frame blocks), those tiles run as a second launch in which the
// waves whose queries all lie past T skip the arithmetic. Workgroups
// are ordered XCD-aware: all query tiles of one (frame, head) run on one
// XCD, so its K/V stream through that XCD's L2.
//
// f32, D = 64 (16-byte aligned buffers): the same transposed flash scheme
// on v_mfma_f32_32x32x2_f32 (flash_f32_kernel).
//
// Generic path (D = 128, or unaligned buffers): one thread per query over
// LDS-staged f32 K/V tiles, the reference's per-key online softmax in its
// operand order.
#include <math.h>

#include "hs_common.hpp"

namespace hs {
namespace {

typedef f16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kXcds = 8;

// ---------------------------------------------------------------------------
// flash attention, f16, D = 64

#ifndef HS_ATT_WAVES
#define HS_ATT_WAVES 8  // waves (32 queries each) per workgroup
#endif
constexpr int kD = 64;
constexpr int kWaves = HS_ATT_WAVES;
constexpr int kThreads = 64 * kWaves;
#ifndef HS_ATT_QB
#define HS_ATT_QB 1  // 32-query blocks per wave
#endif
constexpr int kQB = HS_ATT_QB;
constexpr int kBM = 32 * kQB * kWaves;  // queries per workgroup
#ifndef HS_ATT_BN
#define HS_ATT_BN 64  // keys per tile (a multiple of 32)
#endif
constexpr int kBN = HS_ATT_BN;    // keys per tile
#ifndef HS_ATT_LAZY
#define HS_ATT_LAZY 8.0f  // running-max slack before a rescale (log2 units)
#endif
constexpr float kLazyMax = HS_ATT_LAZY;
constexpr int kKB = kBN / 32;     // 32-key blocks per tile
// LDS row pitches (halves) of the K and V tiles, multiples of 8 so rows
// stay 16-byte aligned. The LDS has 64 4-byte banks and serves a 16-byte
// read 16 lanes at a time, an 8-byte read 32 lanes at a time. K (144 B
// rows): the 16 rows of one 16-byte read start 36 banks apart, covering
// all 64 banks once. V (192 B rows): the transposing read's 32 lanes cover
// 4 rows x 64 bytes, and rows 48 banks apart put the four 16-bank spans on
// disjoint banks. Both are conflict-free (a common 160 B pitch makes every
// K read and V read two-way conflicted).
#ifndef HS_ATT_KPAD
#define HS_ATT_KPAD 8
#endif
#ifndef HS_ATT_VPAD
#define HS_ATT_VPAD 32
#endif
constexpr int kKPitch = kD + HS_ATT_KPAD;
constexpr int kVPitch = kD + HS_ATT_VPAD;
static_assert(HS_ATT_KPAD % 8 == 0 && HS_ATT_VPAD % 8 == 0, "rows must stay 16-byte aligned");
constexpr int kChunks = kBN * kD / 8;  // 16-byte chunks per K (or V) tile
constexpr int kPer = (kChunks + kThreads - 1) / kThreads;
static_assert(kChunks % kThreads == 0 || kThreads % kChunks == 0, "tile split");

struct FlashSmem {
    f16 k[2][kBN * kKPitch];
    f16 v[2][kBN * kVPitch];
};

__device__ __forceinline__ h8 as_h8(u32x4 v) { return __builtin_bit_cast(h8, v); }

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
    f16x2 h;
    h.x = static_cast<f16>(a), h.y = static_cast<f16>(b);
    return h22u(h);
}

// One thread's share of a 64-row K or V tile: 16-byte chunk c = tid + i *
// kThreads is row c / 8, channels (c % 8) * 8 .. + 8.
struct TileChunks {
    u32x4 c[kPer];
};

// Loads rows [key0, key0 + 64) of one (frame, head); rows past the
// sequence end are clamped to the last row (their scores are masked).
__device__ __forceinline__ void load_rows(TileChunks& r, const f16* src, int key0, int t, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = tid + i * kThreads;
        if (kChunks % kThreads != 0 && c >= kChunks) break;
        const int row = min(key0 + c / 8, t - 1);
        r.c[i] = ld16(src + static_cast<int64_t>(row) * kD + (c % 8) * 8);
    }
}

// Row-major into LDS with a padded pitch.
template <int kPitch>
__device__ __forceinline__ void store_rows(const TileChunks& r, f16* buf, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = tid + i * kThreads;
        if (kChunks % kThreads != 0 && c >= kChunks) break;
        st16(&buf[(c / 8) * kPitch + (c % 8) * 8], r.c[i]);
    }
}

// S^T (keys x queries) of one tile for the wave's query blocks: s[b][kb]
// holds keys [32 kb, 32 kb + 32) of the tile; register r of lane (n, hh) is
// key 8 (r / 4) + 4 hh + r % 4 of its block, query n of query block b.
// Each K operand read from LDS feeds the MFMAs of every query block.
__device__ __forceinline__ void qk_scores(f32x16 (&s)[kQB][kKB], const f16* kbuf,
                                          const h8 (&qa)[kQB][4], int n, int hh) {
    const f16* a0 = kbuf + n * kKPitch + 8 * hh;
    const f32x16 z = {};
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
#pragma unroll
        for (int kb = 0; kb < kKB; kb++) {
            const h8 kv = as_h8(ld16(a0 + 32 * kb * kKPitch + 16 * ks));
#pragma unroll
            for (int b = 0; b < kQB; b++)
                s[b][kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kv, qa[b][ks], ks ? s[b][kb] : z, 0, 0, 0);
        }
    }
}

// Keys at or past t score -inf (the partial last tile).
// The two halves of the wave (lanes l and l ^ 32) exchanged with the gfx950
// v_permlane32_swap: applied to two copies of v it leaves lane l holding
// (v[l], v[l + 32]) for l < 32 and (v[l - 32], v[l]) above, so the pair's
// max or sum needs no select and no LDS round trip (ds_bpermute). Both
// halves get the same bits.
__device__ __forceinline__ float halves_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                    __builtin_bit_cast(uint32_t, v), false, false);
    return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
                 __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
}
__device__ __forceinline__ float halves_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                    __builtin_bit_cast(uint32_t, v), false, false);
    return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
           __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

__device__ __forceinline__ void mask_tail(f32x16 (&s)[kKB], int key0, int t, int hh) {
#pragma unroll
    for (int kb = 0; kb < kKB; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int kr = key0 + 32 * kb + 8 * (r / 4) + 4 * hh + (r % 4);
            if (kr >= t) s[kb][r] = -INFINITY;
        }
}

// The tile's weights against reference m: P^T as f16 B operands
// (registers 8 kk .. 8 kk + 7 of s[kb] in p[kb][kk]) and their row sum over
// this lane's keys, which adds the f16 weights the P.V product uses: two
// levels of packed f16 additions (partial sums of four weights, each
// addition rounded to f16, at most 2^-11 relative) and four v_dot2 into
// f32. Beside MFMAs a v_dot2 costs ~6 cycles that do not overlap them (an
// issue-rate probe), so the packed additions replace twelve of the sixteen
// (global calls 3% faster, frame calls 2%). Masked keys weigh exp2(-inf) = 0; a weight or partial sum past
// f16's range gives an infinite sum, which takes the max path.
__device__ __forceinline__ float weights_tile(const f32x16 (&s)[kKB], float c, float m,
                                              u32x4 (&p)[kKB][2]) {
    f16x2 w2[kKB * 8];
#pragma unroll
    for (int kk = 0; kk < 2; kk++)
#pragma unroll
        for (int w = 0; w < 4; w++)
#pragma unroll
            for (int kb = 0; kb < kKB; kb++) {
                const int r = 8 * kk + 2 * w;
                p[kb][kk][w] = pk_f16(__builtin_amdgcn_exp2f(fmaf(s[kb][r], c, -m)),
                                      __builtin_amdgcn_exp2f(fmaf(s[kb][r + 1], c, -m)));
                w2[(kk * 4 + w) * kKB + kb] = u2h2(p[kb][kk][w]);
            }
    constexpr int kHalf = kKB * 4, kQuarter = kKB * 2;
#pragma unroll
    for (int i = 0; i < kHalf; i++) w2[i] = w2[i] + w2[i + kHalf];
#pragma unroll
    for (int i = 0; i < kQuarter; i++) w2[i] = w2[i] + w2[i + kQuarter];
    const f16x2 one2 = {static_cast<f16>(1.0f), static_cast<f16>(1.0f)};
    float ps = 0.0f;
#pragma unroll
    for (int i = 0; i < kQuarter; i++) ps = __builtin_amdgcn_fdot2(w2[i], one2, ps, false);
    return ps;
}

// A lane's row sum over one tile above which its weights take the max path:
// every weight is then at most 2^15, inside f16's range.
constexpr float kRowSumMax = 32768.0f;

// Online-softmax update for one tile's scores (already masked) through the
// tile max: returns the weights in p and the factor the running output must
// be scaled by.
__device__ __forceinline__ float softmax_tile(const f32x16 (&s)[kKB], float c, float& m, float& l,
                                              u32x4 (&p)[kKB][2]) {
    // a sequential chain, which the compiler turns into v_max3_f32
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < kKB; kb++)
#pragma unroll
        for (int r = (kb == 0 ? 1 : 0); r < 16; r += 2)
            mx = r + 1 < 16 ? fmaxf(fmaxf(mx, s[kb][r]), s[kb][r + 1]) : fmaxf(mx, s[kb][r]);
    mx = halves_max(mx);
    // The reference moves only when the tile's scores exceed it by more than
    // kLazyMax (log2 units): the weights exp2(s c - m) then stay below
    // 2^kLazyMax, exact in f16 to its usual relative precision, and the
    // final O / l is unchanged mathematically (both use the same m).
    const float m_cand = fmaxf(m, mx * c);
    const float m_new = m_cand > m + kLazyMax ? m_cand : m;
    const float corr = __builtin_amdgcn_exp2f(m - m_new);
    const float ps = weights_tile(s, c, m_new, p);
    l = fmaf(l, corr, ps);
    m = m_new;
    return corr;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// O^T (channels x queries) += V^T P^T; o0 channels [0, 32), o1 [32, 64).
// The A operand (V^T rows = channels) comes from row-major V through
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element j
// from the (i % 4)-th half of lane 4 j + i / 4's 8-byte read. Lane 4 j' + q
// of the group therefore reads V[key j'][c0 + 4 q .. + 4), and lane i gets
// channel c0 + i of 4 keys; two such reads give the 8 keys of one operand,
// in the order the score accumulator holds P^T (keys 16 kk + 4 hh + j and
// 16 kk + 8 + 4 hh + j of a 32-key block).
__device__ __forceinline__ void pv_update(f32x16 (&o)[kQB][2], const f16* vbuf,
                                          const u32x4 (&p)[kQB][kKB][2], int n, int hh) {
    const int lane16 = n & 15;  // lane within its 16-lane group
    const int c0 = n & 16;      // channel base of the group within a 32-channel block
    const f16* base = vbuf + (4 * hh + lane16 / 4) * kVPitch + c0 + 4 * (lane16 % 4);
#pragma unroll
    for (int kb2 = 0; kb2 < kKB; kb2++)
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const f16* r0 = base + (32 * kb2 + 16 * kk) * kVPitch;
            h8 a[2];
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(r0 + 32 * mb));
                const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(r0 + 8 * kVPitch + 32 * mb));
                const u32x2 wl = __builtin_bit_cast(u32x2, lo), wh = __builtin_bit_cast(u32x2, hi);
                u32x4 w;
                w[0] = wl[0], w[1] = wl[1], w[2] = wh[0], w[3] = wh[1];
                a[mb] = as_h8(w);
            }
#pragma unroll
            for (int b = 0; b < kQB; b++) {
                o[b][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], as_h8(p[b][kb2][kk]), o[b][0], 0, 0, 0);
                o[b][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1], as_h8(p[b][kb2][kk]), o[b][1], 0, 0, 0);
            }
        }
}

__device__ __forceinline__ void rescale(f32x16& o0, f32x16& o1, float corr) {
    if (__any(corr != 1.0f)) {
#pragma unroll
        for (int r = 0; r < 16; r++) o0[r] *= corr, o1[r] *= corr;
    }
}

// Normalises and stores the wave's 32 output rows; register r of o_mb is
// channel 32 mb + 8 (r / 4) + 4 hh + r % 4 of query n.
__device__ __forceinline__ void store_out(const f32x16& o0, const f32x16& o1, float l, f16* orow,
                                          int hh) {
    const float inv = 1.0f / halves_sum(l);
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
        const int d0 = 8 * r4 + 4 * hh;
        u32x2 w0, w1;
        w0[0] = pk_f16(o0[4 * r4] * inv, o0[4 * r4 + 1] * inv);
        w0[1] = pk_f16(o0[4 * r4 + 2] * inv, o0[4 * r4 + 3] * inv);
        w1[0] = pk_f16(o1[4 * r4] * inv, o1[4 * r4 + 1] * inv);
        w1[1] = pk_f16(o1[4 * r4 + 2] * inv, o1[4 * r4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d0) = w0;
        *reinterpret_cast<u32x2*>(orow + 32 + d0) = w1;
    }
}

// grid.x = kXcds * ceil(SH / kXcds) * QT workgroups; workgroup b runs on XCD
// b % kXcds and takes (frame*head) index sh = (b / kXcds / QT) * kXcds +
// b % kXcds, query tile qt0 + (b / kXcds) % QT.
// TAIL: the launch of the partial last query tiles (qt0 = their index),
// whose waves with every query past T only stage K and V.
template <bool TAIL>
__global__ __launch_bounds__(kThreads) void flash_f16_kernel(
    const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
    f16* __restrict__ out, int sh_count, int heads, int t, int qtiles, float c,
    int token_major, int qt0) {
    __shared__ FlashSmem sm;
    const int b = blockIdx.x;
    const int slot = b / kXcds;
    const int sh = (slot / qtiles) * kXcds + b % kXcds;
    if (sh >= sh_count) return;  // workgroup-uniform, before any barrier
    const int qt = qt0 + slot % qtiles;
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int n = lane & 31, hh = lane >> 5;
    const int64_t base = static_cast<int64_t>(sh) * t * kD;
    const f16* qb = q + base;
    const f16* kb = k + base;
    const f16* vb = v + base;

    // Q^T as the B operand: lane (n, hh) of block b holds
    // q[qi_b][16 ks + 8 hh .. + 8), qi_b = query n of the wave's block b.
    int qi[kQB];
    h8 qa[kQB][4];
#pragma unroll
    for (int b = 0; b < kQB; b++) {
        qi[b] = qt * kBM + (wave * kQB + b) * 32 + n;
        const int qc = min(qi[b], t - 1);
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
            qa[b][ks] = as_h8(ld16(qb + static_cast<int64_t>(qc) * kD + 16 * ks + 8 * hh));
    }
    // Q must have arrived before the tile loop: otherwise the compiler sinks
    // these loads into the loop's preheader and, unable to tell them from
    // the prefetch loads issued inside the loop, waits for the prefetch at
    // every tile's first MFMA.
#pragma unroll
    for (int b = 0; b < kQB; b++)
#pragma unroll
        for (int ks = 0; ks < 4; ks++) asm volatile("" ::"v"(qa[b][ks]));

    f32x16 o[kQB][2];
    float m[kQB], l[kQB];
#pragma unroll
    for (int b = 0; b < kQB; b++) {
        o[b][0] = f32x16{}, o[b][1] = f32x16{};
        m[b] = -INFINITY, l[b] = 0.0f;
    }
    const int ntiles = static_cast<int>(ceil_div(t, kBN));

    // Double-buffered tiles: tile j + 1 is loaded into registers while tile
    // j computes from LDS, then written to the other buffer (last read in
    // iteration j - 1, which the barrier at its end closed).
    TileChunks pk, pv;
    load_rows(pk, kb, 0, t, tid);
    load_rows(pv, vb, 0, t, tid);
    store_rows<kKPitch>(pk, sm.k[0], tid);
    store_rows<kVPitch>(pv, sm.v[0], tid);
    __syncthreads();
    for (int j = 0; j < ntiles; j++) {
        const int cur = j & 1;
        if (j + 1 < ntiles) {
            load_rows(pk, kb, (j + 1) * kBN, t, tid);
            load_rows(pv, vb, (j + 1) * kBN, t, tid);
        }
        if (!TAIL || qt * kBM + wave * kQB * 32 < t) {
        f32x16 sc[kQB][kKB];
        qk_scores(sc, sm.k[cur], qa, n, hh);
        u32x4 p[kQB][kKB][2];
#pragma unroll
        for (int b = 0; b < kQB; b++) {
            if ((j + 1) * kBN > t) mask_tail(sc[b], j * kBN, t, hh);
            // After the first tile, weights against the kept reference; the
            // max path only when some lane's sum says a weight may exceed
            // 2^15 (a row sum above 2^15 means a weight above 2^10, more
            // than kLazyMax over m, so that path then moves m).
            bool max_path = j == 0;
            if (!max_path) {
                const float ps = weights_tile(sc[b], c, m[b], p[b]);
                max_path = __any(!(ps <= kRowSumMax));
                if (!max_path) l[b] += ps;
            }
            if (max_path) {
                const float corr = softmax_tile(sc[b], c, m[b], l[b], p[b]);
                rescale(o[b][0], o[b][1], corr);
            }
        }
        pv_update(o, sm.v[cur], p, n, hh);
        }
        if (j + 1 < ntiles) {
            store_rows<kKPitch>(pk, sm.k[cur ^ 1], tid);
            store_rows<kVPitch>(pv, sm.v[cur ^ 1], tid);
        }
        __syncthreads();
    }

#pragma unroll
    for (int b = 0; b < kQB; b++) {
        if (qi[b] >= t) continue;
        f16* orow;
        if (token_major) {
            const int s = sh / heads, h = sh - s * heads;
            orow = out + ((static_cast<int64_t>(s) * t + qi[b]) * heads + h) * kD;
        } else {
            orow = out + base + static_cast<int64_t>(qi[b]) * kD;
        }
        store_out(o[b][0], o[b][1], l[b], orow, hh);
    }
}

// ---------------------------------------------------------------------------
// generic attention: one thread per query, f32 math in the reference's order

constexpr int kGThreads = 256;
constexpr int kGKeys = 32;  // keys per LDS tile

template <typename T, int D>
__global__ __launch_bounds__(kGThreads) void attention_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ out,
    int heads, int t, float scale, int token_major) {
    __shared__ float ks[kGKeys][D];
    __shared__ float vs[kGKeys][D];
    const int sh = blockIdx.y;
    const int64_t base = static_cast<int64_t>(sh) * t * D;
    const int qi = blockIdx.x * kGThreads + threadIdx.x;
    const int qc = min(qi, t - 1);
    float qv[D], acc[D];
#pragma unroll
    for (int d = 0; d < D; d++) {
        qv[d] = static_cast<float>(q[base + static_cast<int64_t>(qc) * D + d]);
        acc[d] = 0.0f;
    }
    float m = -3.4e38f, l = 0.0f;
    for (int k0 = 0; k0 < t; k0 += kGKeys) {
        const int nk = min(kGKeys, t - k0);
        __syncthreads();
        for (int i = threadIdx.x; i < kGKeys * D; i += kGThreads) {
            const int r = i / D, d = i % D;
            const int row = min(k0 + r, t - 1);
            ks[r][d] = static_cast<float>(k[base + static_cast<int64_t>(row) * D + d]);
            vs[r][d] = static_cast<float>(v[base + static_cast<int64_t>(row) * D + d]);
        }
        __syncthreads();
        for (int kk = 0; kk < nk; kk++) {
            // vec4 partial sums, then their horizontal sum (attention.wesl:65-70)
            float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int d = 0; d < D; d += 4)
#pragma unroll
                for (int e = 0; e < 4; e++) s4[e] += qv[d + e] * ks[kk][d + e];
            const float score = (s4[0] + s4[1] + s4[2] + s4[3]) * scale;
            const float m_new = fmaxf(m, score);
            const float corr = expf(m - m_new);
            const float e = expf(score - m_new);
            l = l * corr + e;
#pragma unroll
            for (int d = 0; d < D; d++) acc[d] = acc[d] * corr + e * vs[kk][d];
            m = m_new;
        }
    }
    if (qi >= t) return;
    const float inv = 1.0f / l;
    T* orow;
    if (token_major) {
        const int s = sh / heads, h = sh - s * heads;
        orow = out + ((static_cast<int64_t>(s) * t + qi) * heads + h) * D;
    } else {
        orow = out + base + static_cast<int64_t>(qi) * D;
    }
#pragma unroll
    for (int d = 0; d < D; d++) orow[d] = static_cast<T>(acc[d] * inv);
}

// ---------------------------------------------------------------------------
// head merge: (S, H, T, D) -> (S*T, H*D), 16-byte vectors when D allows

template <typename T>
__global__ __launch_bounds__(256) void merge_vec_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                        int64_t nvec, int heads, int t, int d) {
    constexpr int V = Vec<T>::N;
    const int dv = d / V;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < nvec; i += stride) {
        // i enumerates output vectors: token row r = s*T + ti, head h, chunk c
        const int c = static_cast<int>(i % dv);
        const int64_t rh = i / dv;
        const int h = static_cast<int>(rh % heads);
        const int64_t r = rh / heads;
        const int64_t s = r / t;
        const int ti = static_cast<int>(r - s * t);
        const int64_t src = ((s * heads + h) * t + ti) * d + static_cast<int64_t>(c) * V;
        st_stream(out + i * V, ld_stream(x + src));
    }
}

// One wave per kMergeTok consecutive tokens: a token's output row is H*D
// contiguous elements, NV 16-byte vectors per lane (lane l holds vectors l,
// l + 64, ...: head j / dv, chunk j % dv of vector j). The token's frame
// and position are wave-uniform; the per-lane head and chunk offsets are
// computed once. All kMergeTok * NV loads are in flight before the first
// store, and every store instruction writes 1 KiB contiguous.
constexpr int kMergeTok = 2;

template <typename T, int NV>
__global__ __launch_bounds__(256) void merge_tok_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                        int rows, int heads, int t, int d) {
    constexpr int V = Vec<T>::N;
    const int lane = lane_id();
    const int dv = d / V;
    const int hv = heads * dv;  // = 64 * NV
    const int r0 = (static_cast<int>(blockIdx.x) * 4 + wave_in_block()) * kMergeTok;
    if (r0 >= rows) return;  // wave-uniform; no barriers
    int64_t off[NV];  // per-lane element offset within a frame for token 0
#pragma unroll
    for (int n = 0; n < NV; n++) {
        const int j = lane + 64 * n;
        const int h = j / dv;
        off[n] = static_cast<int64_t>(h) * t * d + static_cast<int64_t>(j - h * dv) * V;
    }
    u32x4 v[kMergeTok][NV];
#pragma unroll
    for (int k = 0; k < kMergeTok; k++) {
        const int r = r0 + k;
        if (r >= rows) break;
        const int s = r / t, ti = r - s * t;
        const T* src = x + (static_cast<int64_t>(s) * heads * t + ti) * d;
#pragma unroll
        for (int n = 0; n < NV; n++) v[k][n] = ld_stream(src + off[n]);
    }
#pragma unroll
    for (int k = 0; k < kMergeTok; k++) {
        const int r = r0 + k;
        if (r >= rows) break;
        T* dst = out + static_cast<int64_t>(r) * hv * V;
#pragma unroll
        for (int n = 0; n < NV; n++) st_stream(dst + (lane + 64 * n) * V, v[k][n]);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void merge_scalar_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                           int64_t total, int heads, int t, int d) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
        const int dd = static_cast<int>(i % d);
        const int64_t rh = i / d;
        const int h = static_cast<int>(rh % heads);
        const int64_t r = rh / heads;
        const int64_t s = r / t;
        const int ti = static_cast<int>(r - s * t);
        out[i] = x[((s * heads + h) * t + ti) * d + dd];
    }
}

// ---------------------------------------------------------------------------
// f32 flash attention, head_dim 64, on v_mfma_f32_32x32x2_f32. A workgroup
// of kF32Waves waves takes kF32Q queries of one (frame, head), a wave 32 of
// them; keys stream through LDS in tiles of kF32Keys: K row-major [key][dim]
// and V transposed [dim][key], rows padded to kF32Pitch floats, written
// from a register prefetch of the next tile issued while the current one
// computes. Per tile and wave, in transposed form so that a lane's column is
// its own query (its softmax statistics need only the lane pair's
// exchange):
//   S^T (keys x queries) = K Q^T: MFMA j of dim group g takes element j of
//     lane (n, hh)'s 16-byte chunk 8 g + 4 hh of its K row and of query n
//     (held in registers), i.e. sums dims 8 g + j and 8 g + 4 + j; register
//     r of lane (n, hh) is then key 8 (r / 4) + 4 hh + r % 4 of the 32-key
//     block, query n.
//   online softmax in log2 units, as the f16 kernel: m = the running max of
//     s c, weights exp2(s c - m), c = scale / ln 2.
//   O^T (dims x queries) += V^T P^T: MFMA j = 4 qd + e takes, from lane (n,
//     hh), element e of V^T row (dim) n's chunk at key 8 qd + 4 hh and the
//     weight in score register j, which is that same key: the scores are
//     the B operand as they stand.
// The output (O / l) leaves from the accumulators: register quad r4 of lane
// (n, hh) is dims 32 db + 8 r4 + 4 hh .. + 4 of query n, one 16-byte store.
constexpr int kF32Waves = 4;
constexpr int kF32Threads = 64 * kF32Waves;
constexpr int kF32Q = 32 * kF32Waves;  // queries per workgroup
constexpr int kF32Keys = 64;           // keys per LDS tile
constexpr int kF32Pitch = 68;          // floats per LDS row (16-byte aligned, 4 banks apart)
constexpr int kF32Loads = kF32Keys * kD / 4 / kF32Threads;  // 16-byte loads per thread, K or V
static_assert(kF32Loads * kF32Threads * 4 == kF32Keys * kD, "tile split");

struct alignas(16) F32FlashSmem {
    float k[kF32Keys * kF32Pitch];  // [key][dim]
    float vt[kD * kF32Pitch];       // [dim][key]
};

__global__ __launch_bounds__(kF32Threads, 2) void flash_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, int sh_count, int heads, int t, int qtiles, float c, int token_major) {
    __shared__ F32FlashSmem sm;
    // the f16 kernel's XCD-aware order: the query tiles of one (frame,
    // head) run on one XCD and share its L2 copy of K and V
    const int b = blockIdx.x;
    const int slot = b / kXcds;
    const int sh = (slot / qtiles) * kXcds + b % kXcds;
    if (sh >= sh_count) return;  // workgroup-uniform, before any barrier
    const int qt = slot % qtiles;
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int n = lane & 31, hh = lane >> 5;
    const int64_t base = static_cast<int64_t>(sh) * t * kD;
    const float* kb = k + base;
    const float* vb = v + base;

    // query n of the wave (queries past T read row T - 1; not stored)
    const int qi = qt * kF32Q + wave * 32 + n;
    const float* qrow = q + base + static_cast<int64_t>(min(qi, t - 1)) * kD;
    float4 qv[8];
#pragma unroll
    for (int g = 0; g < 8; g++) qv[g] = ld_f32x4(qrow + 8 * g + 4 * hh);

    f32x16 o[2] = {f32x16{}, f32x16{}};
    float m = -3.0e38f, l = 0.0f;

    // staging: load i of thread tid is float4 f = tid + kF32Threads i of the
    // tile, key f / 16, dims 4 (f % 16) .. + 4 (16 lanes per 256-byte row)
    float4 kr[kF32Loads], vr[kF32Loads];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kF32Loads; i++) {
            const int f = tid + kF32Threads * i;
            const int64_t row = min(k0 + f / 16, t - 1);  // keys past T: masked below
            kr[i] = ld_f32x4(kb + row * kD + 4 * (f % 16));
            vr[i] = ld_f32x4(vb + row * kD + 4 * (f % 16));
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kF32Loads; i++) {
            const int f = tid + kF32Threads * i;
            const int key = f / 16, d0 = 4 * (f % 16);
            *reinterpret_cast<float4*>(sm.k + key * kF32Pitch + d0) = kr[i];
            sm.vt[(d0 + 0) * kF32Pitch + key] = vr[i].x;
            sm.vt[(d0 + 1) * kF32Pitch + key] = vr[i].y;
            sm.vt[(d0 + 2) * kF32Pitch + key] = vr[i].z;
            sm.vt[(d0 + 3) * kF32Pitch + key] = vr[i].w;
        }
    };
    load(0);
    for (int k0 = 0; k0 < t; k0 += kF32Keys) {
        __syncthreads();  // every wave's reads of the previous tile are done
        stage();
        __syncthreads();
        if (k0 + kF32Keys < t) load(k0 + kF32Keys);

        f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const float4 a =
                    *reinterpret_cast<const float4*>(sm.k + (32 * kb2 + n) * kF32Pitch + 8 * g + 4 * hh);
                s[kb2] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qv[g].x, s[kb2], 0, 0, 0);
                s[kb2] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qv[g].y, s[kb2], 0, 0, 0);
                s[kb2] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qv[g].z, s[kb2], 0, 0, 0);
                s[kb2] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qv[g].w, s[kb2], 0, 0, 0);
            }
        if (k0 + kF32Keys > t) {
#pragma unroll
            for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (k0 + 32 * kb2 + 8 * (r / 4) + 4 * hh + r % 4 >= t) s[kb2][r] = -INFINITY;
        }
        float mx = s[0][0];
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[kb2][r]);
        // every tile holds a key below T, so the pair's max is finite
        const float m_new = fmaxf(m, halves_max(mx) * c);
        const float corr = __builtin_amdgcn_exp2f(m - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[kb2][r], c, -m_new));
                s[kb2][r] = p;
                sum += p;
            }
        l = l * corr + halves_sum(sum);
        m = m_new;
        o[0] *= corr;
        o[1] *= corr;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
                for (int qd = 0; qd < 4; qd++) {
                    const float4 a = *reinterpret_cast<const float4*>(
                        sm.vt + (32 * db + n) * kF32Pitch + 32 * kb2 + 8 * qd + 4 * hh);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, s[kb2][4 * qd + 0], o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, s[kb2][4 * qd + 1], o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, s[kb2][4 * qd + 2], o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, s[kb2][4 * qd + 3], o[db], 0, 0, 0);
                }
    }
    if (qi >= t) return;  // after the last barrier
    float* orow = token_major
                      ? out + ((static_cast<int64_t>(sh / heads) * t + qi) * heads + sh % heads) * kD
                      : out + base + static_cast<int64_t>(qi) * kD;
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = f2u(o[db][4 * r4 + e] / l);
            st16(orow + 32 * db + 8 * r4 + 4 * hh, w);
        }
}

int64_t grid_blocks(int64_t items) {
    const int64_t cap = static_cast<int64_t>(num_cus()) * 8;
    const int64_t blocks = ceil_div(items, 256);
    return blocks < 1 ? 1 : (blocks < cap ? blocks : cap);
}

hs_status check_attention(const char* op, hs_dtype dt, const void* q, const void* k,
                          const void* v, const void* out, int32_t s, int32_t h, int32_t t,
                          int32_t d) {
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "%s: unknown dtype", op);
    if (s < 0 || h < 0 || t < 0 || d <= 0)
        return fail(HS_EINVAL, "%s: shape (%d, %d, %d, %d)", op, s, h, t, d);
    const int64_t n = static_cast<int64_t>(s) * h * t * d;
    if (static_cast<int64_t>(s) * h * t >= (int64_t{1} << 31) || n >= (int64_t{1} << 40))
        return fail(HS_EINVAL, "%s: S*H*T must be below 2^31", op);
    if (n == 0) return HS_OK;
    if (!q || !k || !v || !out) return fail(HS_EINVAL, "%s: null buffer", op);
    const int64_t bytes = n * dtype_size(dt);
    if (overlaps(out, bytes, q, bytes) || overlaps(out, bytes, k, bytes) ||
        overlaps(out, bytes, v, bytes))
        return fail(HS_EINVAL, "%s: out overlaps an input", op);
    return HS_OK;
}

hs_status launch_attention(hipStream_t st, hs_dtype dt, const void* q, const void* k,
                           const void* v, void* out, int s, int h, int t, int d, int token_major) {
    const int sh = s * h;
    const float scale = 1.0f / sqrtf(static_cast<float>(d));
    const bool flash_ok = dt == HS_F16 && d == kD && aligned16(q) && aligned16(k) && aligned16(v) &&
                          (reinterpret_cast<uintptr_t>(out) & 7u) == 0;
    if (flash_ok) {
        const int qtiles = static_cast<int>(ceil_div(t, kBM));
        const int64_t blocks = static_cast<int64_t>(kXcds) * ceil_div(sh, kXcds) * qtiles;
        if (blocks < (int64_t{1} << 31) / kThreads) {
            const float c = scale * 1.4426950408889634f;  // scores enter exp2
            // A partial last query tile runs as a launch of its own when
            // there are enough of them to fill the chip (two workgroups per
            // CU, e.g. 32 frames x 16 heads of 1374 tokens): its waves past
            // T then leave their SIMDs to the live ones. With fewer (one
            // long sequence) they stay in the main launch, where they
            // overlap the other tiles.
            const bool split = t % kBM != 0 && qtiles > 1 && sh >= 2 * num_cus();
            const int main_tiles = split ? qtiles - 1 : qtiles;
            const int64_t mblocks = static_cast<int64_t>(kXcds) * ceil_div(sh, kXcds) * main_tiles;
            flash_f16_kernel<false><<<dim3(static_cast<uint32_t>(mblocks)), dim3(kThreads), 0, st>>>(
                static_cast<const f16*>(q), static_cast<const f16*>(k), static_cast<const f16*>(v),
                static_cast<f16*>(out), sh, h, t, main_tiles, c, token_major, 0);
            if (split) {
                const int64_t tblocks = static_cast<int64_t>(kXcds) * ceil_div(sh, kXcds);
                flash_f16_kernel<true><<<dim3(static_cast<uint32_t>(tblocks)), dim3(kThreads), 0, st>>>(
                    static_cast<const f16*>(q), static_cast<const f16*>(k), static_cast<const f16*>(v),
                    static_cast<f16*>(out), sh, h, t, 1, c, token_major, qtiles - 1);
            }
            return check_launch("attention");
        }
    }
    if (dt == HS_F32 && d == kD && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out)) {
        const int qtiles = static_cast<int>(ceil_div(t, kF32Q));
        const int64_t blocks = static_cast<int64_t>(kXcds) * ceil_div(sh, kXcds) * qtiles;
        if (blocks < (int64_t{1} << 31) / kF32Threads) {
            flash_f32_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(kF32Threads), 0, st>>>(
                static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
                static_cast<float*>(out), sh, h, t, qtiles, scale * 1.4426950408889634f, token_major);
            return check_launch("attention");
        }
    }
    if (sh > 65535) return fail(HS_EUNSUPPORTED, "attention: S*H above 65535 on the generic path");
    const dim3 grid(static_cast<uint32_t>(ceil_div(t, kGThreads)), static_cast<uint32_t>(sh));
    if (d == 64 && dt == HS_F16)
        attention_generic_kernel<f16, 64><<<grid, dim3(kGThreads), 0, st>>>(
            static_cast<const f16*>(q), static_cast<const f16*>(k), static_cast<const f16*>(v),
            static_cast<f16*>(out), h, t, scale, token_major);
    else if (d == 64)
        attention_generic_kernel<float, 64><<<grid, dim3(kGThreads), 0, st>>>(
            static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
            static_cast<float*>(out), h, t, scale, token_major);
    else
        attention_generic_kernel<float, 128><<<grid, dim3(kGThreads), 0, st>>>(
            static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
            static_cast<float*>(out), h, t, scale, token_major);
    return check_launch("attention");
}

hs_status attention_entry(const char* op, hs_stream_t stream, hs_dtype dt, const void* q,
                          const void* k, const void* v, void* out, int32_t s, int32_t h,
                          int32_t t, int32_t d, int token_major) {
    const hs_status rc = check_attention(op, dt, q, k, v, out, s, h, t, d);
    if (rc != HS_OK || static_cast<int64_t>(s) * h * t == 0) return rc;
    // head_dim 64 (f32 and f16) or 128 (f32 only), as engine/ops.rs:233-238
    if (!(d == 64 || (d == 128 && dt == HS_F32)))
        return fail(HS_EUNSUPPORTED, "%s: unsupported head_dim %d for this dtype", op, d);
    return launch_attention(static_cast<hipStream_t>(stream), dt, q, k, v, out, s, h, t, d,
                            token_major);
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_attention(hs_stream_t stream, hs_dtype dt, const void* q, const void* k,
                                  const void* v, void* out, int32_t s, int32_t h, int32_t t,
                                  int32_t d) {
    return hs::attention_entry("attention", stream, dt, q, k, v, out, s, h, t, d, 0);
}

extern "C" hs_status hs_attention_merged(hs_stream_t stream, hs_dtype dt, const void* q,
                                         const void* k, const void* v, void* out, int32_t s,
                                         int32_t h, int32_t t, int32_t d) {
    return hs::attention_entry("attention_merged", stream, dt, q, k, v, out, s, h, t, d, 1);
}

extern "C" hs_status hs_attn_merge(hs_stream_t stream, hs_dtype dt, const void* x, void* out,
                                   int32_t s, int32_t h, int32_t t, int32_t d) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "attn_merge: unknown dtype");
    if (s < 0 || h < 0 || t < 0 || d < 0)
        return fail(HS_EINVAL, "attn_merge: shape (%d, %d, %d, %d)", s, h, t, d);
    const int64_t total = static_cast<int64_t>(s) * h * t * d;
    if (total >= (int64_t{1} << 40)) return fail(HS_EINVAL, "attn_merge: tensor too large");
    if (total == 0) return HS_OK;
    if (!x || !out) return fail(HS_EINVAL, "attn_merge: null buffer");
    const int64_t bytes = total * dtype_size(dt);
    if (overlaps(out, bytes, x, bytes)) return fail(HS_EINVAL, "attn_merge: out overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int per = dt == HS_F16 ? 8 : 4;
    const int64_t rows = static_cast<int64_t>(s) * t;
    const int64_t hv = d % per == 0 ? static_cast<int64_t>(h) * (d / per) : 0;
    if (aligned16(x) && aligned16(out) && rows < (int64_t{1} << 30) &&
        (hv == 64 || hv == 128 || hv == 256)) {
        const int64_t waves = ceil_div(rows, int64_t{kMergeTok});
        const dim3 grid(static_cast<uint32_t>(ceil_div(waves, int64_t{4})));
        const int r = static_cast<int>(rows);
#define HS_MERGE_LAUNCH(NV)                                                                        \
    if (dt == HS_F16)                                                                              \
        merge_tok_kernel<f16, NV><<<grid, dim3(256), 0, st>>>(static_cast<const f16*>(x),          \
                                                             static_cast<f16*>(out), r, h, t, d);  \
    else                                                                                           \
        merge_tok_kernel<float, NV><<<grid, dim3(256), 0, st>>>(static_cast<const float*>(x),      \
                                                               static_cast<float*>(out), r, h, t, d)
        if (hv == 64) {
            HS_MERGE_LAUNCH(1);
        } else if (hv == 128) {
            HS_MERGE_LAUNCH(2);
        } else {
            HS_MERGE_LAUNCH(4);
        }
#undef HS_MERGE_LAUNCH
        return check_launch("attn_merge");
    }
    if (d % per == 0 && aligned16(x) && aligned16(out)) {
        const int64_t nvec = total / per;
        const dim3 grid(static_cast<uint32_t>(grid_blocks(nvec)));
        if (dt == HS_F16)
            merge_vec_kernel<f16><<<grid, dim3(256), 0, st>>>(static_cast<const f16*>(x), static_cast<f16*>(out), nvec, h, t, d);
        else
            merge_vec_kernel<float><<<grid, dim3(256), 0, st>>>(static_cast<const float*>(x), static_cast<float*>(out), nvec, h, t, d);
        return check_launch("attn_merge");
    }
    const dim3 grid(static_cast<uint32_t>(grid_blocks(total)));
    if (dt == HS_F16)
        merge_scalar_kernel<f16><<<grid, dim3(256), 0, st>>>(static_cast<const f16*>(x), static_cast<f16*>(out), total, h, t, d);
    else
        merge_scalar_kernel<float><<<grid, dim3(256), 0, st>>>(static_cast<const float*>(x), static_cast<float*>(out), total, h, t, d);
    return check_launch("attn_merge");
}
