// split_heads + QK-norm + 2D RoPE for gfx950 (replaces the reference's
// split_heads.wesl, layernorm.wesl at dim 64 and rope_apply.wesl, dispatched
// in sequence by model/block.rs:130-146), plus the stand-alone split_heads
// and in-place rope_apply surface ops.
//
// Fast path (head_dim 64): a wave owns one token row of the token-major
// projection (S*T, H*64) at a time, all H heads. A 64-wide head vector is
// spread over a group of G lanes (8 for f16, 16 for f32), each lane holding
// one 16-byte vector, so one load instruction covers 64/G heads and LN(64)
// is a G-lane DPP reduction with no LDS. Rotate-half RoPE pairs channel i
// with i+32; the lane holding channels [i, i+V) sits opposite the lane
// holding [32+i, 32+i+V) under the DPP row mirror (lane j <-> G-1-j), so
// each lane gets its partner's values with one permute per element. Norm,
// rotation and the reference's intermediate storage rounding stay in
// registers; each element crosses HBM once each way.
//
// Memory pattern: the row's loads are contiguous 1 KiB pieces (f16) issued
// together, and a wave pipelines K consecutive rows so the next row's loads
// are in flight while the current one is computed and stored. Each store
// writes 64/G heads' 128-byte vectors of one token into the head-major
// (S, H, T, 64) output that attention consumes. (A pure copy with exactly
// this addressing runs as fast as a contiguous copy of the same bytes when
// T is a frame's 1374 tokens.) For long sequences (T >= kSplitSeq, the
// global blocks' 43,968 tokens) the output's head regions lie megabytes
// apart and writing all of them at once costs: there a wave takes one
// 1 KiB load chunk (64/G heads) of each row and the grid runs chunk by
// chunk, so half as many regions receive writes at a time (S=32 global
// layout, q and k: 61.5 us against 66.0; a pure copy in that order 75% of
// the HBM peak against 67%; in the frame layout the split is slower, 66 us
// against 59).
//
// RoPE tables: all 64/G head groups of a wave need the same cos/sin values
// for a token, so per-lane table loads would fetch each row 64/G times (as
// many bytes as the activations themselves, through the same load path;
// measured 7% of the kernel's time at S=32). Each wave instead stages its
// K tokens' cos and sin rows in a 1 KiB LDS slice with one 16-byte load per
// lane (K = 2), and the lanes read their channels from there.
//
// hs_qknorm_rope_pair runs q and k in one launch (the first half of the grid
// takes q with its norm, the second half k): each launch pays ~4 us of
// fill and drain at S=32, so one launch for both halves that cost.
//
// rope_apply on head-major tensors with head_dim 64 runs the same lane
// layout in place (rope_vec_kernel: a wave takes a few tokens of one frame
// across a group of heads, so each token's table row is read once per
// group).
//
// Generic path (any head_dim, either input layout): one wave per head vector,
// lanes strided over the vector; used for shapes the fast paths do not
// cover.
#include "hs_common.hpp"

namespace hs {
namespace {

// Launch shape (overridable at build time for tuning sweeps).
#ifndef HS_QK_K
#define HS_QK_K 2  // work units per wave (software-pipelined)
#endif
#ifndef HS_QK_BPC
#define HS_QK_BPC 8  // resident workgroups per CU (generic path)
#endif
#ifndef HS_ROPE_HB
// heads per wave of the in-place rope_apply kernel, all loaded together:
// at S=32 (16 heads) 8 took 30.5 us warm / 33.2 cold against 31.9 / 35.1
// for 16 (one wave per token tile), 31.6 / 33.2 for 4 and 34.2 / 36.1 for 2
#define HS_ROPE_HB 8
#endif
// Sequence length from which a wave takes one load chunk of each row
// instead of the whole row (see above).
constexpr int kSplitSeq = 8192;

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / 64;
constexpr int kBlocksPerCu = HS_QK_BPC;

int64_t persistent_blocks(int64_t work_waves) {
    const int64_t cap = static_cast<int64_t>(num_cus()) * kBlocksPerCu;
    const int64_t blocks = ceil_div(work_waves, kWavesPerBlock);
    return blocks < cap ? blocks : cap;
}

// Row mapping: a work unit is one token row (all H heads). A load
// instruction covers HPI = 64/G heads, so the row is CH contiguous 1 KiB
// loads; the token index, its frame and the RoPE decision are wave-uniform
// (scalar divide, uniform branch), and each store writes HPI heads' vectors
// of one token (HPI separate 128-byte pieces of the head-major output).
template <typename T, int H, bool NORM, bool ROPE, bool SPLIT>
struct QknRow {
    static constexpr int D = 64;
    static constexpr int V = Vec<T>::N;
    static constexpr int G = D / V;
    static constexpr int HPI = 64 / G;
    static constexpr int CH = H / HPI;
    static_assert(H % HPI == 0, "whole load instructions per row");
    static constexpr int NCH = SPLIT ? 1 : CH;  // load chunks per wave and row
    static constexpr int HB = NCH;              // loads per unit (buffer size)

    const T* __restrict__ x;
    const float* __restrict__ sin_tab;
    const float* __restrict__ cos_tab;
    T* __restrict__ out;
    int seq, prefix, ch, gsub;
    bool upper;
    const float* tab;      // this wave's LDS slice: per token, cos row then sin row
    int64_t tab_tok0;      // token of the slice's first row
    float eps;
    float wr[V], br[V];
    int c0;                // first load chunk of the row this wave takes

    __device__ __forceinline__ void load(u32x4 (&raw)[HB], int64_t tok) const {
        const T* xr = x + tok * (H * D) + gsub * D + ch;
#pragma unroll
        for (int c = 0; c < NCH; c++) raw[c] = ld_stream(xr + (c0 + c) * HPI * D);
    }

    __device__ __forceinline__ void process(const u32x4 (&raw)[HB], int64_t tok) const {
        // tokens < 2^31 (checked on the host): wave-uniform 32-bit divide
        const uint32_t s = static_cast<uint32_t>(tok) / static_cast<uint32_t>(seq);
        const int t = static_cast<int>(static_cast<uint32_t>(tok) - s * static_cast<uint32_t>(seq));
        T* obase = out + (static_cast<int64_t>(s) * H + gsub) * seq * D +
                   static_cast<int64_t>(t) * D + ch;
        float cs[V], sn[V];
        // Two copies of the row code, chosen by a wave-uniform branch, so
        // the rotated and the unrotated results never meet in one register.
        if (ROPE && t >= prefix) {
            const float* trow = tab + (tok - tab_tok0) * 2 * D + ch;
            const float sg = upper ? 1.0f : -1.0f;
#pragma unroll
            for (int k = 0; k < V; k += 4) {
                const float4 c4 = *reinterpret_cast<const float4*>(trow + k);
                const float4 s4 = *reinterpret_cast<const float4*>(trow + D + k);
                cs[k] = c4.x, cs[k + 1] = c4.y, cs[k + 2] = c4.z, cs[k + 3] = c4.w;
                sn[k] = sg * s4.x, sn[k + 1] = sg * s4.y, sn[k + 2] = sg * s4.z,
                sn[k + 3] = sg * s4.w;
            }
            emit<true>(raw, obase, cs, sn);
        } else {
#pragma unroll
            for (int k = 0; k < V; k++) cs[k] = sn[k] = 0.0f;
            emit<false>(raw, obase, cs, sn);
        }
    }

    template <bool ROT>
    __device__ __forceinline__ void emit(const u32x4 (&raw)[HB], T* obase, const float (&cs)[V],
                                         const float (&sn)[V]) const {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            float f[V];
            unpack(raw[c], f, T{});
            qk_norm_rope_vec<T, G, NORM>(f, wr, br, eps, ROT, cs, sn);
            st_stream(obase + static_cast<int64_t>(c0 + c) * HPI * seq * D, pack(f, T{}));
        }
    }
};

// One or two tensors of the same shape that share the RoPE tables and one
// launch (q and k of a block): waves [0, W) take the first, [W, 2W) the
// second, W = ceil(tokens / K); with SPLIT the units (chunk, tensor) run
// chunk-major, W waves each.
template <typename T>
struct QknTensors {
    const T* x[2];
    const float* nw[2];
    const float* nb[2];
    T* out[2];
    int n;
};

// Each wave runs K consecutive units with a two-buffer software pipeline:
// the loads of unit i+1 are in flight while unit i is normalised, rotated
// and stored, so waves overlap memory with arithmetic instead of alternating
// between them in lockstep.
template <typename T, int H, bool NORM, bool ROPE, int K, bool SPLIT>
__global__ __launch_bounds__(kBlock) void qkn_row_kernel(
    QknTensors<T> ts, const float* __restrict__ sin_tab, const float* __restrict__ cos_tab,
    int64_t tokens, int seq, int prefix, float eps) {
    using Row = QknRow<T, H, NORM, ROPE, SPLIT>;
    constexpr int G = Row::G, V = Row::V, HB = Row::HB;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t per_tensor = ceil_div(tokens, int64_t{K});
    int which, chunk = 0;
    int64_t u0;
    if constexpr (SPLIT) {
        const int64_t unit = wave / per_tensor;
        chunk = static_cast<int>(unit / ts.n), which = static_cast<int>(unit % ts.n);
        if (chunk >= Row::CH) return;  // wave-uniform: the kernel has no barriers
        u0 = (wave - unit * per_tensor) * K;
    } else {
        which = wave >= per_tensor ? 1 : 0;
        if (which >= ts.n) return;  // wave-uniform: the kernel has no barriers
        u0 = (wave - which * per_tensor) * K;
    }
    if (u0 >= tokens) return;  // the grid's last workgroup may run past the second tensor
    const int64_t u_end = u0 + K < tokens ? u0 + K : tokens;
    const int lane = lane_id();
    const int piece = lane % G;
    Row tl;
    tl.c0 = chunk;
    tl.x = ts.x[which], tl.out = ts.out[which];
    tl.sin_tab = sin_tab, tl.cos_tab = cos_tab;
    tl.seq = seq, tl.prefix = prefix, tl.eps = eps;
    tl.gsub = lane / G;
    // Channels held by this lane: lower-half pieces hold [piece*V, +V), the
    // mirrored upper-half pieces hold the matching [32 + (G-1-piece)*V, +V).
    tl.upper = piece >= G / 2;
    tl.ch = tl.upper ? 32 + (G - 1 - piece) * V : piece * V;
    if constexpr (NORM) {
        const float* nw = ts.nw[which];
        const float* nb = ts.nb[which];
#pragma unroll
        for (int k = 0; k < V; k += 4) {
            float4 w4 = ld_f32x4(nw + tl.ch + k), b4 = ld_f32x4(nb + tl.ch + k);
            tl.wr[k] = w4.x, tl.wr[k + 1] = w4.y, tl.wr[k + 2] = w4.z, tl.wr[k + 3] = w4.w;
            tl.br[k] = b4.x, tl.br[k + 1] = b4.y, tl.br[k + 2] = b4.z, tl.br[k + 3] = b4.w;
        }
    }

    // RoPE table rows of the wave's K tokens, staged through LDS: one 16-byte
    // load per lane covers two tokens' cos and sin rows (1 KiB), instead of
    // every lane reading its own 64 bytes of both rows per token.
    __shared__ float4 tab_lds[kWavesPerBlock][K * 2 * 64 / 4];
    if constexpr (ROPE) {
        float4* slice = tab_lds[wave_in_block()];
#pragma unroll
        for (int i0 = 0; i0 < K * 2 * 64 / 4; i0 += 64) {
            const int i = i0 + lane;
            const int k = i / 32, which_tab = (i / 16) & 1, off = (i & 15) * 4;
            const int64_t tok = u0 + k;
            if (tok < u_end) {
                const int t = static_cast<int>(static_cast<uint32_t>(tok) % static_cast<uint32_t>(seq));
                if (t >= prefix) {
                    const float* src = which_tab ? sin_tab : cos_tab;
                    slice[i] = ld_f32x4(src + static_cast<int64_t>(t - prefix) * 64 + off);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        tl.tab = reinterpret_cast<const float*>(slice);
        tl.tab_tok0 = u0;
    }
    u32x4 a[HB], b[HB];
    tl.load(a, u0);
#pragma unroll 1
    for (int64_t u = u0; u < u_end; u += 2) {
        if (u + 1 < u_end) tl.load(b, u + 1);
        tl.process(a, u);
        if (u + 1 >= u_end) break;
        if (u + 2 < u_end) tl.load(a, u + 2);
        tl.process(b, u + 1);
    }
}

// In-place rotate-half RoPE on head-major (S, H, T, 64) vectors (the
// rope_apply surface op), in the row kernel's lane layout: a vector in a
// group of G lanes, each channel's RoPE partner in the mirror lane. A wave
// takes TG = 64 / G consecutive tokens of one frame in a group of HB heads,
// all HB loads in flight together: each load instruction covers one head's
// TG vectors (contiguous in head-major order), and each lane reads its
// token's sin/cos row once for the group. Prefix tokens are neither read
// nor written.
template <typename T, int HB>
__global__ __launch_bounds__(kBlock) void rope_vec_kernel(T* x, const float* __restrict__ sin_tab,
                                                          const float* __restrict__ cos_tab,
                                                          int nseq, int heads, int seq,
                                                          int prefix) {
    constexpr int D = 64, V = Vec<T>::N, G = D / V, TG = 64 / G;
    const int lane = lane_id();
    const int piece = lane % G;
    const bool upper = piece >= G / 2;
    const int ch = upper ? 32 + (G - 1 - piece) * V : piece * V;
    const float none[V] = {};
    const int tiles = static_cast<int>(ceil_div(seq, TG));
    // unit = (frame, head group of HB, token tile), token tiles fastest
    const int groups = static_cast<int>(ceil_div(heads, HB));
    const int64_t per_frame = static_cast<int64_t>(groups) * tiles;
    const int64_t unit = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    if (unit >= static_cast<int64_t>(nseq) * per_frame) return;  // wave-uniform; no barriers
    const int s = static_cast<int>(unit / per_frame);
    const int rem = static_cast<int>(unit - static_cast<int64_t>(s) * per_frame);
    const int grp = rem / tiles;
    const int t = (rem - grp * tiles) * TG + lane / G;
    const int hend = grp * HB + HB < heads ? grp * HB + HB : heads;
    // a group's lanes share their token, so `live` is uniform across the
    // group that the mirror permute reads
    const bool live = t < seq && t >= prefix;
    float cs[V], sn[V];
#pragma unroll
    for (int k = 0; k < V; k++) cs[k] = sn[k] = 0.0f;
    if (live) {
        const int64_t row = static_cast<int64_t>(t - prefix) * D + ch;
        const float sg = upper ? 1.0f : -1.0f;
#pragma unroll
        for (int k = 0; k < V; k += 4) {
            const float4 c4 = ld_f32x4(cos_tab + row + k), s4 = ld_f32x4(sin_tab + row + k);
            cs[k] = c4.x, cs[k + 1] = c4.y, cs[k + 2] = c4.z, cs[k + 3] = c4.w;
            sn[k] = sg * s4.x, sn[k + 1] = sg * s4.y, sn[k + 2] = sg * s4.z, sn[k + 3] = sg * s4.w;
        }
    }
    T* base = x + (static_cast<int64_t>(s) * heads * seq + t) * D + ch;
    const int64_t hstride = static_cast<int64_t>(seq) * D;
    {
        const int h0 = grp * HB;
        u32x4 raw[HB];
#pragma unroll
        for (int j = 0; j < HB; j++) {
            raw[j] = u32x4{0, 0, 0, 0};
            if (live && h0 + j < hend) raw[j] = ld_stream(base + (h0 + j) * hstride);
        }
        if (!live) return;
#pragma unroll
        for (int j = 0; j < HB; j++) {
            if (h0 + j >= hend) break;  // wave-uniform
            float f[V];
            unpack(raw[j], f, T{});
            qk_norm_rope_vec<T, G, false>(f, none, none, 0.0f, true, cs, sn);
            st_stream(base + (h0 + j) * hstride, pack(f, T{}));
        }
    }
}

// One wave per head vector. in_head_major selects the input layout:
// false = token-major (S*T, H*D), true = head-major (S, H, T, D). The output
// is head-major and may equal the input when the input is head-major.
template <typename T>
__global__ __launch_bounds__(kBlock) void qkn_generic_kernel(
    const T* x, bool in_head_major, const float* __restrict__ nw, const float* __restrict__ nb,
    const float* __restrict__ sin_tab, const float* __restrict__ cos_tab, T* out, int nseq,
    int seq, int heads, int d, int prefix, float eps) {
    const int lane = lane_id();
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
    const int64_t nvec = static_cast<int64_t>(nseq) * seq * heads;
    const bool norm = nw != nullptr;
    const int half = d / 2;
    for (int64_t v = wave; v < nvec; v += nwaves) {
        int64_t s, h, t;
        if (in_head_major) {
            t = v % seq;
            const int64_t sh = v / seq;
            h = sh % heads;
            s = sh / heads;
        } else {
            h = v % heads;
            const int64_t tok = v / heads;
            t = tok % seq;
            s = tok / seq;
        }
        const T* xin = in_head_major ? x + v * d : x + (s * seq + t) * heads * d + h * d;
        T* o = out + ((s * heads + h) * seq + t) * d;
        float mean = 0.0f, inv = 1.0f;
        if (norm) {
            float sum = 0.0f;
            for (int j = lane; j < d; j += 64) sum += load_elem(xin + j);
            mean = wave_sum(sum) / static_cast<float>(d);
            float q = 0.0f;
            for (int j = lane; j < d; j += 64) {
                const float dd = load_elem(xin + j) - mean;
                q += dd * dd;
            }
            inv = rsqrtf(wave_sum(q) / static_cast<float>(d) + eps);
        }
        const bool rot = sin_tab != nullptr && t >= prefix;
        if (rot) {
            const int64_t row = (t - prefix) * d;
            for (int dp = lane; dp < half; dp += 64) {
                float lo = load_elem(xin + dp), hi = load_elem(xin + dp + half);
                if (norm) {
                    lo = storage_round((lo - mean) * inv * nw[dp] + nb[dp], T{});
                    hi = storage_round((hi - mean) * inv * nw[dp + half] + nb[dp + half], T{});
                }
                store_elem(o + dp, lo * cos_tab[row + dp] - hi * sin_tab[row + dp]);
                store_elem(o + dp + half,
                           hi * cos_tab[row + half + dp] + lo * sin_tab[row + half + dp]);
            }
        } else {
            for (int j = lane; j < d; j += 64) {
                float val = load_elem(xin + j);
                if (norm) val = (val - mean) * inv * nw[j] + nb[j];
                store_elem(o + j, val);
            }
        }
    }
}

// Row waves of a launch: K tokens per wave and tensor, times the load
// chunks of a row when each wave takes one.
template <typename T>
int64_t row_waves(int64_t tokens, int n, int h, int seq) {
    const int64_t parts = seq >= kSplitSeq ? h / Vec<T>::N : 1;
    return ceil_div(tokens, int64_t{HS_QK_K}) * n * parts;
}

template <typename T, int H, bool NORM, bool ROPE>
hs_status launch_rows(hipStream_t st, const QknTensors<T>& ts, const float* sn, const float* cs,
                      int64_t tokens, int seq, int prefix, float eps) {
    constexpr int K = HS_QK_K;
    const int64_t blocks = ceil_div(row_waves<T>(tokens, ts.n, H, seq), int64_t{kWavesPerBlock});
    if (seq >= kSplitSeq)
        qkn_row_kernel<T, H, NORM, ROPE, K, true>
            <<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(ts, sn, cs, tokens, seq,
                                                                          prefix, eps);
    else
        qkn_row_kernel<T, H, NORM, ROPE, K, false>
            <<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(ts, sn, cs, tokens, seq,
                                                                          prefix, eps);
    return check_launch("qknorm_rope");
}

template <typename T, int H>
hs_status launch_rows_flags(hipStream_t st, const QknTensors<T>& ts, const float* sn,
                            const float* cs, int64_t tokens, int seq, int prefix, float eps) {
    const bool norm = ts.nw[0] != nullptr, rope = sn != nullptr && prefix < seq;
    if (norm && rope) return launch_rows<T, H, true, true>(st, ts, sn, cs, tokens, seq, prefix, eps);
    if (norm) return launch_rows<T, H, true, false>(st, ts, sn, cs, tokens, seq, prefix, eps);
    if (rope) return launch_rows<T, H, false, true>(st, ts, sn, cs, tokens, seq, prefix, eps);
    return launch_rows<T, H, false, false>(st, ts, sn, cs, tokens, seq, prefix, eps);
}

template <typename T>
hs_status launch_generic(hipStream_t st, const void* x, bool in_head_major, const float* nw,
                         const float* nb, const float* sn, const float* cs, void* out, int s,
                         int t, int h, int d, int prefix, float eps) {
    const int64_t nvec = static_cast<int64_t>(s) * t * h;
    const int64_t blocks = persistent_blocks(nvec);
    qkn_generic_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
        static_cast<const T*>(x), in_head_major, nw, nb, sn, cs, static_cast<T*>(out), s, t, h, d,
        prefix, eps);
    return check_launch("qknorm_rope");
}

// Token-major input, one or two tensors: the row path when head_dim is 64,
// H is one of the instantiated head counts and every pointer is 16-byte
// aligned; otherwise the generic kernel, one launch per tensor.
template <typename T>
hs_status dispatch_tok(hipStream_t st, const QknTensors<T>& ts, const float* sn, const float* cs,
                       int s, int t, int h, int d, int prefix, float eps) {
    bool ptrs_ok = !sn || (aligned16(sn) && aligned16(cs));
    for (int i = 0; i < ts.n; i++)
        ptrs_ok = ptrs_ok && aligned16(ts.x[i]) && aligned16(ts.out[i]) &&
                  (!ts.nw[i] || (aligned16(ts.nw[i]) && aligned16(ts.nb[i])));
    const int64_t tokens = static_cast<int64_t>(s) * t;
    // The dispatch packet counts work-items in 32 bits: the row grid has one
    // wave per K tokens per tensor; beyond that the persistent generic
    // kernel runs.
    const int64_t row_blocks = ceil_div(row_waves<T>(tokens, ts.n, h, t), int64_t{kWavesPerBlock});
    const bool grid_ok = row_blocks * kBlock < (int64_t{1} << 32);
    if (d == 64 && ptrs_ok && grid_ok) {
        switch (h) {
            case 8: return launch_rows_flags<T, 8>(st, ts, sn, cs, tokens, t, prefix, eps);
            case 16: return launch_rows_flags<T, 16>(st, ts, sn, cs, tokens, t, prefix, eps);
            case 32: return launch_rows_flags<T, 32>(st, ts, sn, cs, tokens, t, prefix, eps);
            default: break;
        }
    }
    for (int i = 0; i < ts.n; i++)
        if (hs_status e = launch_generic<T>(st, ts.x[i], false, ts.nw[i], ts.nb[i], sn, cs,
                                            ts.out[i], s, t, h, d, prefix, eps))
            return e;
    return HS_OK;
}

template <typename T>
hs_status dispatch_tok(hipStream_t st, const void* x, const float* nw, const float* nb,
                       const float* sn, const float* cs, void* out, int s, int t, int h, int d,
                       int prefix, float eps) {
    QknTensors<T> ts{};
    ts.x[0] = static_cast<const T*>(x), ts.nw[0] = nw, ts.nb[0] = nb;
    ts.out[0] = static_cast<T*>(out), ts.n = 1;
    return dispatch_tok<T>(st, ts, sn, cs, s, t, h, d, prefix, eps);
}

hs_status check_shape(const char* op, int32_t s, int32_t t, int32_t h, int32_t d) {
    if (s < 0 || t < 0 || h < 0 || d < 0)
        return fail(HS_EINVAL, "%s: negative shape (%d, %d, %d, %d)", op, s, t, h, d);
    const int64_t n = static_cast<int64_t>(s) * t * h * d;
    if (n > (int64_t{1} << 40)) return fail(HS_EINVAL, "%s: tensor too large", op);
    if (static_cast<int64_t>(s) * t * h >= (int64_t{1} << 31))
        return fail(HS_EINVAL, "%s: S*T*H must be below 2^31", op);
    return HS_OK;
}

}  // namespace
}  // namespace hs

extern "C" {

hs_status hs_qknorm_rope(hs_stream_t stream, hs_dtype dt, const void* x_tok, const float* nw,
                         const float* nb, const float* sin_tab, const float* cos_tab,
                         void* out_head, int32_t s, int32_t t, int32_t h, int32_t d,
                         int32_t prefix, float eps) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "qknorm_rope: unknown dtype %d", (int)dt);
    if (hs_status e = check_shape("qknorm_rope", s, t, h, d)) return e;
    if ((nw == nullptr) != (nb == nullptr))
        return fail(HS_EINVAL, "qknorm_rope: norm weight and bias must both be given or both NULL");
    if ((sin_tab == nullptr) != (cos_tab == nullptr))
        return fail(HS_EINVAL, "qknorm_rope: sin and cos tables must both be given or both NULL");
    if (sin_tab && (prefix < 0 || prefix > t))
        return fail(HS_EINVAL, "qknorm_rope: prefix %d outside [0, T=%d]", prefix, t);
    if (sin_tab && d % 2 != 0) return fail(HS_EINVAL, "qknorm_rope: RoPE needs an even head_dim");
    const int64_t n = static_cast<int64_t>(s) * t * h * d;
    if (n == 0) return HS_OK;
    if (!x_tok || !out_head) return fail(HS_EINVAL, "qknorm_rope: null buffer");
    const int64_t bytes = n * dtype_size(dt);
    if (overlaps(x_tok, bytes, out_head, bytes))
        return fail(HS_EINVAL, "qknorm_rope: out_head overlaps x_tok");
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16
               ? dispatch_tok<f16>(st, x_tok, nw, nb, sin_tab, cos_tab, out_head, s, t, h, d, prefix, eps)
               : dispatch_tok<float>(st, x_tok, nw, nb, sin_tab, cos_tab, out_head, s, t, h, d, prefix, eps);
}

hs_status hs_qknorm_rope_pair(hs_stream_t stream, hs_dtype dt, const void* q_tok,
                              const void* k_tok, const float* qn_w, const float* qn_b,
                              const float* kn_w, const float* kn_b, const float* sin_tab,
                              const float* cos_tab, void* q_head, void* k_head, int32_t s,
                              int32_t t, int32_t h, int32_t d, int32_t prefix, float eps) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "qknorm_rope_pair: unknown dtype %d", (int)dt);
    if (hs_status e = check_shape("qknorm_rope_pair", s, t, h, d)) return e;
    if ((qn_w == nullptr) != (qn_b == nullptr) || (kn_w == nullptr) != (kn_b == nullptr))
        return fail(HS_EINVAL,
                    "qknorm_rope_pair: each norm's weight and bias must both be given or both NULL");
    if ((qn_w == nullptr) != (kn_w == nullptr))
        return fail(HS_EINVAL, "qknorm_rope_pair: QK-norm must be given for both q and k or for neither");
    if ((sin_tab == nullptr) != (cos_tab == nullptr))
        return fail(HS_EINVAL, "qknorm_rope_pair: sin and cos tables must both be given or both NULL");
    if (sin_tab && (prefix < 0 || prefix > t))
        return fail(HS_EINVAL, "qknorm_rope_pair: prefix %d outside [0, T=%d]", prefix, t);
    if (sin_tab && d % 2 != 0)
        return fail(HS_EINVAL, "qknorm_rope_pair: RoPE needs an even head_dim");
    const int64_t n = static_cast<int64_t>(s) * t * h * d;
    if (n == 0) return HS_OK;
    if (!q_tok || !k_tok || !q_head || !k_head)
        return fail(HS_EINVAL, "qknorm_rope_pair: null buffer");
    const int64_t bytes = n * dtype_size(dt);
    const void* outs[2] = {q_head, k_head};
    for (const void* o : outs)
        if (overlaps(q_tok, bytes, o, bytes) || overlaps(k_tok, bytes, o, bytes))
            return fail(HS_EINVAL, "qknorm_rope_pair: an output overlaps an input");
    if (overlaps(q_head, bytes, k_head, bytes))
        return fail(HS_EINVAL, "qknorm_rope_pair: q_head overlaps k_head");
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto run = [&](auto tag) {
        using T = decltype(tag);
        QknTensors<T> ts{};
        ts.x[0] = static_cast<const T*>(q_tok), ts.x[1] = static_cast<const T*>(k_tok);
        ts.nw[0] = qn_w, ts.nb[0] = qn_b, ts.nw[1] = kn_w, ts.nb[1] = kn_b;
        ts.out[0] = static_cast<T*>(q_head), ts.out[1] = static_cast<T*>(k_head);
        ts.n = 2;
        return dispatch_tok<T>(st, ts, sin_tab, cos_tab, s, t, h, d, prefix, eps);
    };
    return dt == HS_F16 ? run(f16{}) : run(float{});
}

hs_status hs_split_heads(hs_stream_t stream, hs_dtype dt, const void* x, void* out, int32_t s,
                         int32_t t, int32_t h, int32_t d) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "split_heads: unknown dtype %d", (int)dt);
    if (hs_status e = check_shape("split_heads", s, t, h, d)) return e;
    const int64_t n = static_cast<int64_t>(s) * t * h * d;
    if (n == 0) return HS_OK;
    if (!x || !out) return fail(HS_EINVAL, "split_heads: null buffer");
    const int64_t bytes = n * dtype_size(dt);
    if (overlaps(x, bytes, out, bytes)) return fail(HS_EINVAL, "split_heads: out overlaps x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dt == HS_F16
               ? dispatch_tok<f16>(st, x, nullptr, nullptr, nullptr, nullptr, out, s, t, h, d, 0, 0.0f)
               : dispatch_tok<float>(st, x, nullptr, nullptr, nullptr, nullptr, out, s, t, h, d, 0, 0.0f);
}

hs_status hs_rope_apply(hs_stream_t stream, hs_dtype dt, void* x, const float* sin_tab,
                        const float* cos_tab, int32_t s, int32_t h, int32_t t, int32_t d,
                        int32_t prefix) {
    using namespace hs;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "rope_apply: unknown dtype %d", (int)dt);
    if (hs_status e = check_shape("rope_apply", s, t, h, d)) return e;
    if (prefix < 0 || prefix > t)
        return fail(HS_EINVAL, "rope_apply: prefix %d outside [0, T=%d]", prefix, t);
    if (d % 2 != 0) return fail(HS_EINVAL, "rope_apply: head_dim %d is odd", d);
    const int64_t n = static_cast<int64_t>(s) * t * h * d;
    if (n == 0 || prefix == t) return HS_OK;
    if (!x || !sin_tab || !cos_tab) return fail(HS_EINVAL, "rope_apply: null buffer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int tg = dt == HS_F16 ? 8 : 4;  // tokens per load instruction
    constexpr int HB = HS_ROPE_HB;
    const int64_t units = static_cast<int64_t>(s) * ceil_div(h, HB) * ceil_div(t, tg);
    const int64_t blocks = ceil_div(units, int64_t{kWavesPerBlock});
    if (d == 64 && aligned16(x) && aligned16(sin_tab) && aligned16(cos_tab) &&
        blocks * kBlock < (int64_t{1} << 32)) {
        if (dt == HS_F16)
            rope_vec_kernel<f16, HB><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
                static_cast<f16*>(x), sin_tab, cos_tab, s, h, t, prefix);
        else
            rope_vec_kernel<float, HB><<<dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, st>>>(
                static_cast<float*>(x), sin_tab, cos_tab, s, h, t, prefix);
        return check_launch("rope_apply");
    }
    return dt == HS_F16
               ? launch_generic<f16>(st, x, true, nullptr, nullptr, sin_tab, cos_tab, x, s, t, h, d, prefix, 0.0f)
               : launch_generic<float>(st, x, true, nullptr, nullptr, sin_tab, cos_tab, x, s, t, h, d, prefix, 0.0f);
}

}  // extern "C"
