// Linear layers for gfx950 (replaces GpuContext::linear, engine/ops.rs:81-128,
// shaders/linear_wmma.wgsl and shaders/linear.wesl): out (M, N) = x (M, K)
// @ w (N, K)^T + bias (N, f32), with the epilogues the trunk's blocks apply
// to the result fused into the store (model/block.rs:150-176):
//   EPI_BIAS      out = f16(acc + bias)                       (qkv, linear)
//   EPI_GELU      out = f16(gelu(acc + bias))                 (fc1 + GELU)
//   EPI_LS        out = f16(res + gamma * f16(acc + bias))    (proj/fc2 +
//                                                 LayerScale + residual)
//   EPI_QKV       the fused q|k|v projection: f16(acc + bias), split into
//                 heads and written head-major, with QK-norm and RoPE
//                 applied to q and k (model/block.rs:128-146)
// so the activation between a GEMM and its elementwise op never crosses HBM.
//
// Fast path (f16, N % kBN == 0, K % kBK == 0): matrix-core GEMM. A workgroup
// of kWaves waves computes a 256 (rows) x kBN (columns) tile of out, K in
// steps of kBK staged through LDS (double-buffered; the next step's tiles go straight
// from global memory into LDS with buffer_load_dwordx4 ... lds while the
// current one computes, with no registers in between). Both operands are K-contiguous
// rows (x rows, w rows), which is exactly the operand layout of
// v_mfma_f32_32x32x16_f16, so both come from LDS with 16-byte reads. Each
// wave owns 128 rows x 64 columns and computes the transposed tile
// out^T = w x^T: its accumulators then hold, per lane, 4 consecutive output
// columns of one output row. The epilogue adds the bias (and applies GELU)
// there, stages the f16 results through LDS, and then streams whole rows:
// 16-byte reads of the residual and 16-byte writes of out. Rows past M are
// clamped on load and masked on store. The writes are non-temporal: every
// workgroup of a round stores its tile at about the same time, and streaming
// stores drain that burst faster than write-allocating ones (fc1 + GELU at
// S=32: 494 us against 523).
//
// f32 (N % 128 == 0, K % 32 == 0; every epilogue but the q|k|v split, with
// or without the LayerNorm prologue): the same arrangement on the f32
// matrix cores in 128 x 128 tiles, the epilogue stored straight from the
// accumulators.
//
// Generic path (the shapes neither covers): a tiled scalar kernel, f32
// accumulation in K order.
#include <math.h>

#include <initializer_list>
#include <mutex>
#include <type_traits>

#include "hs_common.hpp"

namespace hs {
namespace {

typedef f16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum Epi { EPI_BIAS = 0, EPI_GELU = 1, EPI_LS = 2, EPI_QKV = 3 };

// The q|k|v epilogue's outputs and parameters: out[0..2] head-major (S, H,
// T, 64) q, k, v; QK-norm weight / bias per q and k (null: none); RoPE
// tables (T - prefix, 64) (null: none).
struct QkvArgs {
    void* out[3];  // f16 or f32, as the product
    const float* nw[2];
    const float* nb[2];
    const float* sin_tab;
    const float* cos_tab;
    int seq, heads, prefix;
    float eps;
};

// The LayerNorm prologue (hs_linear_ln*): stats holds each x row's (mean,
// rsqrt(var + eps)) from hs_layernorm_stats, ln_w / ln_b the LayerNorm's
// affine parameters over the K input columns. The product reads each x
// element as hs_layernorm would have stored it.
struct LnArgs {
    const float* stats;
    const float* ln_w;
    const float* ln_b;
};

// ---------------------------------------------------------------------------
// matrix-core path

#ifndef HS_GEMM_WAVES
#define HS_GEMM_WAVES 8  // waves per workgroup: 2 row groups x (waves / 2) column groups
#endif
#ifndef HS_GEMM_BK
#define HS_GEMM_BK 64  // K per LDS stage
#endif
#ifndef HS_GEMM_XCD
#define HS_GEMM_XCD 1  // XCD-aware tile order
#endif
constexpr int kWaves = HS_GEMM_WAVES;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 256;               // output rows per workgroup (2 x 128)
constexpr int kBN = 64 * (kWaves / 2);  // output columns per workgroup
constexpr int kBK = HS_GEMM_BK;
constexpr int kRowChunks = kBK / 8;      // 16-byte chunks per LDS row
constexpr int kRowsPerInstr = 64 / kRowChunks;
constexpr int kRowsPer256B = 128 / kBK;  // LDS rows per 64-bank period
// Stages are filled by buffer_load_dwordx4 ... lds (LDS-DMA): one wave
// instruction puts its 64 lanes' 16-byte chunks into 1 KiB of LDS in lane
// order, i.e. kRowsPerInstr unpadded rows. Lane L of instruction j supplies
// row kRowsPerInstr * j + L / kRowChunks at physical chunk L % kRowChunks,
// which holds logical chunk (L % kRowChunks) ^ swz(row), swz(row) = (row /
// kRowsPer256B) % kRowChunks: with that XOR swizzle the operand reads (16
// consecutive rows, one logical chunk) hit 16 distinct 16-byte bank groups.
// The buffer form (a descriptor in scalar registers, a per-lane offset fixed
// for the tile, the stage's column in the scalar offset) costs no vector
// instruction per load, and unlike the global (FLAT-encoded) form it lets
// the compiler wait for the operand reads of one k-slice with lgkmcnt(n)
// while the next slice's reads are in flight.
constexpr int kXInstr = kBM * kBK / 8 / 64;  // wave instructions per x stage
constexpr int kWInstr = kBN * kBK / 8 / 64;  // per w stage
constexpr int kLoads = kXInstr / kWaves + kWInstr / kWaves;  // per wave and stage
static_assert(kXInstr % kWaves == 0 && kWInstr % kWaves == 0, "stage split");
static_assert((kBK / 16) % 2 == 0, "operand register sets alternate within a stage");

struct GemmSmem {
    f16 x[2][kBM * kBK];
    f16 w[2][kBN * kBK];
};
// With the LayerNorm prologue, x stages land in `raw` one stage ahead of
// their use and are normalised from there into x[]: raw follows GemmSmem.
constexpr size_t kRawBytes = size_t{2} * kBM * kBK;
// Epilogue staging: each wave's 128 x 64 output block as f16 rows of
// kEpiPitch halves (144 B: 16-byte aligned rows, spread over the banks).
constexpr int kEpiPitch = 64 + 8;
constexpr int kEpiWave = 128 * kEpiPitch;  // halves per wave
constexpr size_t smem_bytes(bool ln) {
    const size_t loop = sizeof(GemmSmem) + (ln ? kRawBytes : 0);
    const size_t epi = size_t{2} * kWaves * kEpiWave;
    return loop > epi ? loop : epi;
}
static_assert(smem_bytes(true) <= 160 * 1024, "gfx950 has 160 KiB of LDS per workgroup");

__device__ __forceinline__ h8 as_h8(u32x4 v) { return __builtin_bit_cast(h8, v); }

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int row) { return (row / kRowsPer256B) % kRowChunks; }

// Per-lane byte offsets of this wave's stage loads within the tile's x and
// w row blocks; x rows past M read row M - 1 (their outputs are masked).
struct StageOffsets {
    uint32_t x[kXInstr / kWaves];
    uint32_t w[kWInstr / kWaves];
};

__device__ __forceinline__ StageOffsets stage_offsets(int64_t m0, int M, int K, int wave,
                                                     int lane) {
    StageOffsets o;
    const int prow = lane / kRowChunks, pc = lane % kRowChunks;
#pragma unroll
    for (int i = 0; i < kXInstr / kWaves; i++) {
        const int row = kRowsPerInstr * (wave + kWaves * i) + prow;
        const int lrow = static_cast<int>(min(m0 + row, static_cast<int64_t>(M) - 1) - m0);
        o.x[i] = static_cast<uint32_t>(lrow * K * 2 + 16 * (pc ^ swz(row)));
    }
#pragma unroll
    for (int i = 0; i < kWInstr / kWaves; i++) {
        const int row = kRowsPerInstr * (wave + kWaves * i) + prow;
        o.w[i] = static_cast<uint32_t>(row * K * 2 + 16 * (pc ^ swz(row)));
    }
    return o;
}

// Issue this wave's LDS-DMA loads of one stage's x (or w) rows from the
// buffer resource covering the tile's rows into dst; koff = the stage's
// first column, in bytes.
__device__ __forceinline__ void issue_x(f16* dst, __amdgpu_buffer_rsrc_t xr, int koff,
                                        const StageOffsets& o, int wave) {
#pragma unroll
    for (int i = 0; i < kXInstr / kWaves; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (lds_void*)(dst + (wave + kWaves * i) * 512), 16, o.x[i], koff, 0, 0);
}
__device__ __forceinline__ void issue_w(f16* dst, __amdgpu_buffer_rsrc_t wr, int koff,
                                        const StageOffsets& o, int wave) {
#pragma unroll
    for (int i = 0; i < kWInstr / kWaves; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wr, (lds_void*)(dst + (wave + kWaves * i) * 512), 16, o.w[i], koff, 0, 0);
}
__device__ __forceinline__ void issue_stage(GemmSmem& sm, int buf, __amdgpu_buffer_rsrc_t xr,
                                            __amdgpu_buffer_rsrc_t wr, int koff,
                                            const StageOffsets& o, int wave) {
    issue_x(sm.x[buf], xr, koff, o, wave);
    issue_w(sm.w[buf], wr, koff, o, wave);
}

// The LayerNorm prologue. Lane L of a wave normalises exactly the 16-byte
// pieces that its own x loads put into LDS: instruction i's piece, at
// halves (wave + kWaves i) * 512 + 8 L, is row kRowsPerInstr (wave + kWaves
// i) + L / kRowChunks of the tile, logical chunk lc = (L % kRowChunks) ^
// swz(row), and swz(row) does not depend on i. So a lane needs only its own
// loads to have landed (vmcnt, no barrier), its rows' statistics stay in
// registers for the whole product, and each stage's parameters are the 8
// columns 8 lc of that stage.
constexpr int kLnRows = kXInstr / kWaves;  // x pieces per lane and stage
static_assert((kRowsPerInstr * kWaves / kRowsPer256B) % kRowChunks == 0,
              "a lane's x pieces share one logical chunk");
constexpr int kLnParamLoads = 4;            // 16-byte loads of ln_w / ln_b per stage
#ifndef HS_GEMM_LN_SLICES
#define HS_GEMM_LN_SLICES 2  // k slices of a step over which the next stage is normalised
#endif
#ifndef HS_GEMM_LN_VALU
#define HS_GEMM_LN_VALU 8  // vector instructions scheduled after each of those slices' MFMAs
#endif
#ifndef HS_GEMM_LN_FIRST
#define HS_GEMM_LN_FIRST 1  // the first of those slices (the pieces are read at slice 0)
#endif
#ifndef HS_GEMM_LN_HINTS
#define HS_GEMM_LN_HINTS 1  // interleave by scheduling groups (0: the compiler's order)
#endif
constexpr int kLnSlices = HS_GEMM_LN_SLICES;
constexpr int kLnFirst = HS_GEMM_LN_FIRST;
constexpr bool kLnHints = HS_GEMM_LN_HINTS != 0;
constexpr int kLnValuPerMfma = HS_GEMM_LN_VALU;
static_assert(kLnRows % kLnSlices == 0 && kLnFirst >= 0 && kLnFirst + kLnSlices < kBK / 16,
              "LayerNorm slices: the next stage's parameters load in a later slice");

struct LnLane {
    f32x2 st[kLnRows];  // (mean, rstd) of the lane's rows
    int col;            // first column of the lane's chunk within a stage
};

__device__ __forceinline__ LnLane ln_lane(const LnArgs& la, int64_t m0, int M, int wave, int lane) {
    LnLane ll;
#pragma unroll
    for (int i = 0; i < kLnRows; i++) {
        const int row = kRowsPerInstr * (wave + kWaves * i) + lane / kRowChunks;
        // rows past M were loaded from row M - 1 and are normalised with its
        // statistics (their products are masked)
        const int64_t r = min(m0 + row, static_cast<int64_t>(M) - 1);
        ll.st[i] = *reinterpret_cast<const f32x2*>(la.stats + 2 * r);
    }
    ll.col = 8 * ((lane % kRowChunks) ^ swz(kRowsPerInstr * wave + lane / kRowChunks));
    return ll;
}

// The LayerNorm parameters of the lane's 8 columns of the stage at column k0.
__device__ __forceinline__ void ln_params(const LnArgs& la, const LnLane& ll, int k0,
                                          float4 (&gb)[kLnParamLoads]) {
    const int c = k0 + ll.col;
    gb[0] = ld_f32x4(la.ln_w + c), gb[1] = ld_f32x4(la.ln_w + c + 4);
    gb[2] = ld_f32x4(la.ln_b + c), gb[3] = ld_f32x4(la.ln_b + c + 4);
}

// Halves offset of the lane's piece i within an x stage.
__device__ __forceinline__ int ln_off(int i, int wave, int lane) {
    return (wave + kWaves * i) * 512 + 8 * lane;
}

// One normalised piece: the 8 f16 values of v, with the row's (mean, rstd)
// and the lane's column parameters gb (ln_w then ln_b), rounded to f16 as
// hs_layernorm stores them.
__device__ __forceinline__ u32x4 ln_piece(u32x4 v, f32x2 st, const float4 (&gb)[kLnParamLoads]) {
    const float g[8] = {gb[0].x, gb[0].y, gb[0].z, gb[0].w, gb[1].x, gb[1].y, gb[1].z, gb[1].w};
    const float b[8] = {gb[2].x, gb[2].y, gb[2].z, gb[2].w, gb[3].x, gb[3].y, gb[3].z, gb[3].w};
    float f[8];
    unpack(v, f, f16{});
#pragma unroll
    for (int j = 0; j < 8; j++) f[j] = ln_affine(f[j], st[0], st[1], g[j], b[j]);
    return pack(f, f16{});
}

// Normalises all of the lane's pieces of the stage in `raw` into `dst`.
__device__ __forceinline__ void ln_stage(const f16* raw, f16* dst, const LnLane& ll,
                                         const float4 (&gb)[kLnParamLoads], int wave, int lane) {
#pragma unroll
    for (int i = 0; i < kLnRows; i++)
        st16(dst + ln_off(i, wave, lane), ln_piece(ld16(raw + ln_off(i, wave, lane)), ll.st[i], gb));
}

// Buffer descriptor word 3 for raw (unstructured, stride 0) buffers on gfx950.
constexpr int kRawBufferFlags = 0x00020000;

// Operand read: logical chunk k of LDS row `row` (rows of kBK halves).
__device__ __forceinline__ h8 ld_op(const f16* buf, int row, int k) {
    return as_h8(ld16(buf + row * kBK + 8 * (k ^ swz(row))));
}

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
    f16x2 h;
    h.x = static_cast<f16>(a), h.y = static_cast<f16>(b);
    return h22u(h);
}

// Phase 2 of the q|k|v epilogue: the wave's staged block is 128 token rows
// of one head of q, k or v (its 64 columns). 8 lanes per row hold the head
// vector in the lane layout of qk_norm_rope_vec (the QK-norm / RoPE fused
// op's), so each head vector is normalised, rotated and rounded by the same
// code as there; each row's 128 bytes go to (frame, head, token) of the
// head-major output.
__device__ __forceinline__ void qkv_heads_out(const f16* stage, const QkvArgs& qa, int64_t row0,
                                              int M, int64_t col, int lane) {
    const int hd = qa.heads * 64;
    const int which = static_cast<int>(col / hd);            // 0 q, 1 k, 2 v: wave-uniform
    const int head = static_cast<int>(col - int64_t{which} * hd) / 64;
    const int piece = lane & 7;
    const bool upper = piece >= 4;
    const int ch = upper ? 32 + (7 - piece) * 8 : piece * 8;
    const float* nw = which < 2 ? qa.nw[which] : nullptr;
    const float* nb = which < 2 ? qa.nb[which] : nullptr;
    const bool norm = nw != nullptr;
    const bool rope = which < 2 && qa.sin_tab != nullptr;
    float wr[8], br[8];
    if (norm) {
        const float4 w0 = ld_f32x4(nw + ch), w1 = ld_f32x4(nw + ch + 4);
        const float4 b0 = ld_f32x4(nb + ch), b1 = ld_f32x4(nb + ch + 4);
        wr[0] = w0.x, wr[1] = w0.y, wr[2] = w0.z, wr[3] = w0.w;
        wr[4] = w1.x, wr[5] = w1.y, wr[6] = w1.z, wr[7] = w1.w;
        br[0] = b0.x, br[1] = b0.y, br[2] = b0.z, br[3] = b0.w;
        br[4] = b1.x, br[5] = b1.y, br[6] = b1.z, br[7] = b1.w;
    }
    f16* obase = static_cast<f16*>(qa.out[which]) + static_cast<int64_t>(head) * qa.seq * 64 + ch;
    const float sg = upper ? 1.0f : -1.0f;
    // this lane's row: token m = s * seq + t (m < 2^31), advanced by 8 rows
    // per step
    int64_t m = row0 + (lane >> 3);
    uint32_t s = static_cast<uint32_t>(m) / static_cast<uint32_t>(qa.seq);
    int t = static_cast<int>(static_cast<uint32_t>(m) - s * static_cast<uint32_t>(qa.seq));
    for (int rr = 0; rr < 128; rr += 8) {
        if (m >= M) break;  // rows grow with rr: the rest are past M too
        float f[8];
        unpack(ld16(stage + (rr + (lane >> 3)) * kEpiPitch + ch), f, f16{});
        const bool rot = rope && t >= qa.prefix;  // the same for the row's 8 lanes
        float cs[8], sn[8];
        if (rot) {
            const int64_t trow = static_cast<int64_t>(t - qa.prefix) * 64 + ch;
            const float4 c0 = ld_f32x4(qa.cos_tab + trow), c1 = ld_f32x4(qa.cos_tab + trow + 4);
            const float4 s0 = ld_f32x4(qa.sin_tab + trow), s1 = ld_f32x4(qa.sin_tab + trow + 4);
            cs[0] = c0.x, cs[1] = c0.y, cs[2] = c0.z, cs[3] = c0.w;
            cs[4] = c1.x, cs[5] = c1.y, cs[6] = c1.z, cs[7] = c1.w;
            sn[0] = sg * s0.x, sn[1] = sg * s0.y, sn[2] = sg * s0.z, sn[3] = sg * s0.w;
            sn[4] = sg * s1.x, sn[5] = sg * s1.y, sn[6] = sg * s1.z, sn[7] = sg * s1.w;
        }
        if (norm)
            qk_norm_rope_vec<f16, 8, true>(f, wr, br, qa.eps, rot, cs, sn);
        else
            qk_norm_rope_vec<f16, 8, false>(f, wr, br, qa.eps, rot, cs, sn);
        st16_nt(obase + (static_cast<int64_t>(s) * qa.heads * qa.seq + t) * 64, pack(f, f16{}));
        m += 8;
        t += 8;
        while (t >= qa.seq) t -= qa.seq, s++;
    }
}

// Grid: tiles_m * tiles_n workgroups, column tiles fastest, so workgroups
// running together share their x rows.
template <int EPI, bool LN>
__global__ __launch_bounds__(kThreads, 8 / kWaves) void gemm_f16_kernel(
    const f16* __restrict__ x, const f16* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ gamma, const f16* res, f16* out, int M, int N, int K,
    int tiles_n, int ntiles, QkvArgs qa, LnArgs la) {
    __shared__ __align__(16) unsigned char smem_raw[smem_bytes(LN)];
    GemmSmem& sm = *reinterpret_cast<GemmSmem*>(smem_raw);
    f16* const raw = reinterpret_cast<f16*>(smem_raw + sizeof(GemmSmem));  // LN only
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
#if HS_GEMM_XCD
    // Workgroup b runs on XCD b % 8; XCD x takes the contiguous tile range
    // [x * per, (x + 1) * per), so the column tiles of one row tile (which
    // share its x rows) run on one XCD and its L2. The grid is padded to a
    // multiple of 8 workgroups.
    const int per = static_cast<int>(gridDim.x / 8);
    const int tile = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (tile >= ntiles) return;  // padding, before any barrier
#else
    const int tile = static_cast<int>(blockIdx.x);
#endif
    const int64_t m0 = static_cast<int64_t>(tile / tiles_n) * kBM;
    const int64_t n0 = static_cast<int64_t>(tile % tiles_n) * kBN;
    const int wm = (wave / (kWaves / 2)) * 128;  // wave's rows within the tile
    const int wn = (wave % (kWaves / 2)) * 64;   // wave's columns within the tile

    // acc[a][b]: out^T block of columns wn + 32 a .. + 32 (MFMA rows) and
    // rows wm + 32 b .. + 32 (MFMA columns); register r of lane (l32, hh)
    // is column 8 (r / 4) + 4 hh + r % 4, row l32 of the block.
    f32x16 acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f32x16{};

    const int nsteps = K / kBK;
    const int wv = wave_in_block();
    const StageOffsets so = stage_offsets(m0, M, K, wv, lane);
    const int xrows = static_cast<int>(min(static_cast<int64_t>(kBM), M - m0));
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(x + m0 * K), 0, xrows * K * 2, kRawBufferFlags);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(w + n0 * K), 0, kBN * K * 2, kRawBufferFlags);
    // Both buffers start filled (stages 0 and 1). The waits below are
    // explicit: vmcnt counts this wave's loads, which complete in order, and
    // the barrier then covers every wave's.
    //
    // With the LayerNorm prologue, stage s's x lands in raw during step s - 2
    // (its parameters loaded just before it) and is normalised into x[s & 1]
    // by its own lanes during step s - 1, beside that step's multiplies; w
    // keeps the schedule above. Per wave, in issue order: params(s + 2),
    // x(s + 2) in the middle of step s, w(s + 2) after its closing barrier.
    constexpr int kXL = kXInstr / kWaves, kWL = kWInstr / kWaves;
    LnLane ll;
    float4 gb[kLnParamLoads];
    if constexpr (LN) {
        ll = ln_lane(la, m0, M, wv, lane);
        ln_params(la, ll, 0, gb);
        issue_x(raw, xr, 0, so, wv);
        issue_w(sm.w[0], wr, 0, so, wv);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kWL) : "memory");  // params(0), x(0)
        ln_stage(raw, sm.x[0], ll, gb, wv, lane);
        if (nsteps > 1) {
            ln_params(la, ll, kBK, gb);
            issue_x(raw, xr, 2 * kBK, so, wv);
            issue_w(sm.w[1], wr, 2 * kBK, so, wv);
            // w(0) landed; x[0]'s normalised pieces written
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kLnParamLoads + kXL + kWL)
                         : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
    } else {
        issue_stage(sm, 0, xr, wr, 0, so, wv);
        if (nsteps > 1) {
            issue_stage(sm, 1, xr, wr, 2 * kBK, so, wv);
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kLoads) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        }
    }
    // Operand registers in two sets: the next 16-wide k slice is read from
    // LDS while the current one multiplies, across stage boundaries too.
    h8 A[2][2], B[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++) A[0][a] = ld_op(sm.w[0], wn + 32 * a + l32, hh);
#pragma unroll
    for (int b = 0; b < 4; b++) B[0][b] = ld_op(sm.x[0], wm + 32 * b + l32, hh);
    if constexpr (LN) {
        // One step of the product with the prologue: the multiplies of stage
        // s and, beside them, NORM: stage s + 1's LayerNorm from raw into
        // x[cur ^ 1] (last read in step s - 1, before the barrier that
        // closed it), ISSUE: the loads of stage s + 2. The flags are
        // compile-time, so each step is one basic block in which the
        // scheduler can place the LayerNorm's vector work between the
        // multiplies. The lane's kLnRows pieces are read at slice 0 and
        // normalised over the first kLnSlices slices; raw is refilled at
        // slice 1, once the pieces are in registers, and the next stage's
        // parameters load at slice kLnSlices, once these are used.
        auto step = [&](int s, auto norm_c, auto issue_c) {
            constexpr bool NORM = decltype(norm_c)::value, ISSUE = decltype(issue_c)::value;
            const int cur = s & 1;
            u32x4 rw[kLnRows];
#pragma unroll
            for (int ks = 0; ks < kBK / 16; ks++) {
                const int p = ks & 1;  // kBK / 16 is even: set 0 holds slice 0 of every stage
                if constexpr (ISSUE) {
                    if (ks == 1) {
                        // the lane's raw pieces (read at slice 0) are in
                        // registers: refill raw with x(s + 2)
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        issue_x(raw, xr, 2 * (s + 2) * kBK, so, wv);
                    }
                }
                if (ks + 1 < kBK / 16) {
                    const int kc = 2 * (ks + 1) + hh;
#pragma unroll
                    for (int a = 0; a < 2; a++) A[p ^ 1][a] = ld_op(sm.w[cur], wn + 32 * a + l32, kc);
#pragma unroll
                    for (int b = 0; b < 4; b++) B[p ^ 1][b] = ld_op(sm.x[cur], wm + 32 * b + l32, kc);
                }
                if constexpr (NORM) {
                    if (ks == 0) {
                        // params(s + 1), x(s + 1) landed; w(s + 1) may be in flight
                        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kWL) : "memory");
#pragma unroll
                        for (int i = 0; i < kLnRows; i++) rw[i] = ld16(raw + ln_off(i, wv, lane));
                    }
                    if (ks >= kLnFirst && ks < kLnFirst + kLnSlices) {
                        constexpr int per = kLnRows / kLnSlices;
#pragma unroll
                        for (int i = (ks - kLnFirst) * per; i < (ks - kLnFirst + 1) * per; i++)
                            st16(sm.x[cur ^ 1] + ln_off(i, wv, lane), ln_piece(rw[i], ll.st[i], gb));
                    }
                    if constexpr (ISSUE) {
                        if (ks == kLnFirst + kLnSlices) ln_params(la, ll, (s + 2) * kBK, gb);
                    }
                }
                if (ks + 1 == kBK / 16) {
                    // every wave's reads of stage s are done; w(s + 1) and
                    // the normalised x(s + 1) have landed (params(s + 2) and
                    // x(s + 2) may be in flight)
                    if constexpr (ISSUE)
                        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kLnParamLoads + kXL)
                                     : "memory");
                    else
                        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    // w[cur] is free: refill it with stage s + 2
                    if constexpr (ISSUE) issue_w(sm.w[cur], wr, 2 * (s + 2) * kBK, so, wv);
                    if constexpr (NORM) {
#pragma unroll
                        for (int a = 0; a < 2; a++) A[p ^ 1][a] = ld_op(sm.w[cur ^ 1], wn + 32 * a + l32, hh);
#pragma unroll
                        for (int b = 0; b < 4; b++) B[p ^ 1][b] = ld_op(sm.x[cur ^ 1], wm + 32 * b + l32, hh);
                    }
                }
#pragma unroll
                for (int a = 0; a < 2; a++)
#pragma unroll
                    for (int b = 0; b < 4; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[p][a], B[p][b], acc[a][b], 0, 0, 0);
                if (NORM && !kLnHints) {
                    // the scheduler's own order
                } else if (NORM && ks == 0 && kLnFirst > 0) {
                    // the operand and raw reads ahead of the multiplies
                    __builtin_amdgcn_sched_group_barrier(0x100, 6 + kLnRows, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
                } else if (NORM && ks >= kLnFirst && ks < kLnFirst + kLnSlices) {
                    // the LayerNorm's vector work between the multiplies
                    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // an MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, kLnValuPerMfma, 0);  // VALU
                    }
                } else {
                    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // LDS reads
                    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // MFMAs
                }
            }
        };
        int s = 0;
        for (; s + 2 < nsteps; s++) step(s, std::true_type{}, std::true_type{});
        if (s + 1 < nsteps) step(s++, std::true_type{}, std::false_type{});
        step(s, std::false_type{}, std::false_type{});
    } else {
    for (int s = 0; s < nsteps; s++) {
        const int cur = s & 1;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ks++) {
            const int p = ks & 1;  // kBK / 16 is even: set 0 holds slice 0 of every stage
            if (ks + 1 < kBK / 16) {
                const int kc = 2 * (ks + 1) + hh;
#pragma unroll
                for (int a = 0; a < 2; a++) A[p ^ 1][a] = ld_op(sm.w[cur], wn + 32 * a + l32, kc);
#pragma unroll
                for (int b = 0; b < 4; b++) B[p ^ 1][b] = ld_op(sm.x[cur], wm + 32 * b + l32, kc);
            } else {
                // every wave's reads of stage s are done and stage s + 1
                // (the only load in flight) has landed
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                // buffer cur is free: refill it with stage s + 2
                if (s + 2 < nsteps) issue_stage(sm, cur, xr, wr, 2 * (s + 2) * kBK, so, wv);
                if (s + 1 < nsteps) {
#pragma unroll
                    for (int a = 0; a < 2; a++) A[p ^ 1][a] = ld_op(sm.w[cur ^ 1], wn + 32 * a + l32, hh);
#pragma unroll
                    for (int b = 0; b < 4; b++) B[p ^ 1][b] = ld_op(sm.x[cur ^ 1], wm + 32 * b + l32, hh);
                }
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 4; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[p][a], B[p][b], acc[a][b], 0, 0, 0);
            // keep the reads above ahead of these multiplies
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // MFMAs
        }
    }
    }

    // Epilogue, in two phases so that global memory sees whole rows.
    // 1. Each lane turns its accumulators (row l32 of block b, columns
    //    32 a + 8 r4 + 4 hh .. + 4) into the linear's stored value,
    //    f16(acc + bias) (for GELU: f16(gelu(acc + bias))), and writes it
    //    to the wave's staging block in LDS (free once every wave has left
    //    the main loop).
    f16* stage = reinterpret_cast<f16*>(smem_raw) + wave * kEpiWave;
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
            const int cl = 32 * a + 8 * r4 + 4 * hh;  // column within the wave's block
            const float4 bv = bias ? ld_f32x4(bias + n0 + wn + cl) : float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < 4; b++) {
                float v[4];
                v[0] = acc[a][b][4 * r4] + bv.x, v[1] = acc[a][b][4 * r4 + 1] + bv.y;
                v[2] = acc[a][b][4 * r4 + 2] + bv.z, v[3] = acc[a][b][4 * r4 + 3] + bv.w;
                if constexpr (EPI == EPI_GELU) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = gelu_f(v[e]);
                }
                u32x2 o;
                o[0] = pk_f16(v[0], v[1]), o[1] = pk_f16(v[2], v[3]);
                *reinterpret_cast<u32x2*>(stage + (32 * b + l32) * kEpiPitch + cl) = o;
            }
        }
    // only this wave reads its block back: a wave-level fence suffices
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (EPI == EPI_QKV) {
        qkv_heads_out(stage, qa, m0 + wm, M, n0 + wn, lane);
        return;
    }
    // 2. 8 lanes per 128-byte row piece, 8 rows per instruction: 16-byte
    //    loads of the staged values (and of res), 16-byte stores of out.
    const int c8 = 8 * (lane & 7);
    const int64_t n = n0 + wn + c8;
    float4 g0 = {0.0f, 0.0f, 0.0f, 0.0f}, g1 = g0;
    if constexpr (EPI == EPI_LS) g0 = ld_f32x4(gamma + n), g1 = ld_f32x4(gamma + n + 4);
#pragma unroll 4
    for (int rr = 0; rr < 128; rr += 8) {
        const int rl = rr + (lane >> 3);
        const int64_t m = m0 + wm + rl;
        if (m >= M) break;  // rows grow with rr: the rest are past M too
        u32x4 v = ld16(stage + rl * kEpiPitch + c8);
        if constexpr (EPI == EPI_LS) {
            // res + gamma * x, x the linear's stored (f16) value
            const u32x4 r = ld16(res + m * N + n);
            const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f16x2 xv = u2h2(v[q]), rv = u2h2(r[q]);
                v[q] = pk_f16(fmaf(gg[2 * q], static_cast<float>(xv.x), static_cast<float>(rv.x)),
                              fmaf(gg[2 * q + 1], static_cast<float>(xv.y), static_cast<float>(rv.y)));
            }
        }
        st16_nt(out + m * N + n, v);
    }
}

// ---------------------------------------------------------------------------
// f32 matrix-core path (f32, N % 128 == 0, K % 32 == 0): v_mfma_f32_32x32x2_f32
// in the f16 kernel's arrangement. A workgroup of WAVES waves in 2 row
// groups computes a (2 WROWS) x (32 WAVES) tile, each wave WROWS rows x 64
// columns as out^T blocks of 32 x 32; K in stages of 32 floats through LDS,
// double-buffered and filled by LDS-DMA. A stage row is 128 bytes (8
// chunks of 4 floats) with the f16 kernel's swizzle: logical chunk c of row
// r sits at physical chunk c ^ ((r / 2) % 8). In slice ks of a stage lane
// (l32, hh) reads logical chunk 2 ks + hh (floats 8 ks + 4 hh .. + 4) of its
// rows, and MFMA j of the slice takes element j of both operands: it sums
// k = 8 ks + j (lanes hh = 0) and 8 ks + 4 + j (hh = 1), so the four MFMAs
// of a slice cover its 8 k. The epilogue stores from the accumulators:
// register quad r4 of lane (l32, hh) is 4 consecutive columns of one row
// (16 bytes; the lane pair's quads are 32 contiguous bytes, and the wave's
// four r4 complete the row's 128 bytes of the block).
//
// Shapes: F32Shape, 4 waves, 128 x 128 tiles, 64 KiB of LDS, two
// workgroups per CU. It beats 8 waves in 256 x 256 tiles (128 KiB, one per
// CU) at every trunk shape, by 6-9% at S=32 (43968 x 4096 x 1024: 2716 us
// against 2873) and by 3x where 256 x 256 tiles are too few to fill the
// chip (2748 x 1024 x 4096, 44 of them: 286 us against 925). Below 512
// tiles of 128 x 128 (the chip's slots at two per CU) F32Narrow, 4 waves
// of 32 x 64 in 64 x 128 tiles (48 KiB, three per CU), doubles the tile
// count: 6-23% faster there (2748 x 1024 x 1024: 74 us against 82; 5496 x
// 1024 x 4096: 434 against 515), within 5% either way above.
template <int WAVES, int WROWS>
struct F32Tile {
    static constexpr int kWaves = WAVES, kThreads = 64 * WAVES;
    static constexpr int kBM = 2 * WROWS, kBN = 32 * WAVES;
    static constexpr int kBK = 32;                      // floats per stage row
    static constexpr int kXI = kBM * 8 / 64 / WAVES;    // LDS-DMA instructions per wave, x stage
    static constexpr int kWI = kBN * 8 / 64 / WAVES;    // w stage
    static constexpr int kRB = WROWS / 32;              // 32-row blocks per wave
    static constexpr int kWavesPerEu = 8 / WAVES;
    static_assert(kXI * 64 * WAVES == kBM * 8 && kWI * 64 * WAVES == kBN * 8, "stage split");
};
using F32Shape = F32Tile<4, 64>;
using F32Narrow = F32Tile<4, 32>;

template <typename P>
struct F32Smem {
    float x[2][P::kBM * P::kBK];
    float w[2][P::kBN * P::kBK];
};
static_assert(2 * sizeof(F32Smem<F32Shape>) <= 160 * 1024 && 3 * sizeof(F32Smem<F32Narrow>) <= 160 * 1024,
              "workgroups per CU");

// Per-lane byte offsets of a wave's stage loads (4 instructions each for
// x and w): instruction i of wave wv brings rows
// 8 (wv + waves i) .. + 8, lane L row + L / 8 at physical chunk L % 8; x
// rows past M read row M - 1 (their outputs are masked).
struct F32Offsets {
    uint32_t x[4];
    uint32_t w[4];
};
static_assert(F32Shape::kXI <= 4 && F32Shape::kWI <= 4 && F32Narrow::kXI <= 4 && F32Narrow::kWI <= 4,
              "at most four stage loads per wave and operand");

// xi / wi: the loads per wave of an x / w stage (compile-time after inlining)
__device__ __forceinline__ F32Offsets f32_offsets(int64_t m0, int M, int K, int waves, int wv,
                                                  int lane, int xi, int wi) {
    F32Offsets o;
    const int prow = lane / 8, pc = lane % 8;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = 8 * (wv + waves * i) + prow;
        const int lrow = static_cast<int>(min(m0 + row, static_cast<int64_t>(M) - 1) - m0);
        o.x[i] = i < xi ? static_cast<uint32_t>(lrow * K * 4 + 16 * (pc ^ swz(row))) : 0u;
        o.w[i] = i < wi ? static_cast<uint32_t>(row * K * 4 + 16 * (pc ^ swz(row))) : 0u;
    }
    return o;
}

// This wave's LDS-DMA loads of one stage into xdst / wdst (1 KiB, i.e. 8
// rows of 32 floats, per instruction); koff = the stage's first column in
// bytes.
__device__ __forceinline__ void f32_issue(float* xdst, float* wdst, __amdgpu_buffer_rsrc_t xr,
                                          __amdgpu_buffer_rsrc_t wr, int koff, const F32Offsets& o,
                                          int waves, int wv, int xi, int wi) {
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (i < xi)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(xdst + (wv + waves * i) * 256), 16,
                                                     o.x[i], koff, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (i < wi)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(wdst + (wv + waves * i) * 256), 16,
                                                     o.w[i], koff, 0, 0);
}

// Operand chunk c (4 floats) of LDS row `row` (rows of 32 floats).
__device__ __forceinline__ u32x4 f32_op(const float* buf, int row, int c) {
    return ld16(buf + row * 32 + 4 * (c ^ swz(row)));
}

// The f32 q|k|v epilogue's staging: each wave's block (32 kRB token rows x
// one head's 64 columns, acc + bias) in rows of kQkvPitch floats (16-byte
// aligned, 4 banks apart), in the LDS the stages used.
constexpr int kQkvPitch = 68;
template <typename P>
constexpr size_t f32_smem_bytes(int epi) {
    const size_t loop = sizeof(F32Smem<P>);
    const size_t qkv = epi == EPI_QKV ? size_t{4} * P::kWaves * 32 * P::kRB * kQkvPitch : 0;
    return loop > qkv ? loop : qkv;
}
static_assert(2 * f32_smem_bytes<F32Shape>(EPI_QKV) <= 160 * 1024 &&
                  3 * f32_smem_bytes<F32Narrow>(EPI_QKV) <= 160 * 1024,
              "workgroups per CU with the q|k|v staging");

// The f32 q|k|v epilogue's second phase: the wave's staged block is `rows`
// token rows of one head of q, k or v. 16 lanes per row hold the head
// vector in the lane layout of the standalone f32 QK-norm / RoPE op (piece
// p < 8: channels 4 p .. + 4; p >= 8: 32 + 4 (15 - p) .. + 4), so each head
// vector is normalised and rotated by the same code as there, and each
// row's 256 bytes go to (frame, head, token) of the head-major output.
__device__ __forceinline__ void qkv_heads_out_f32(const float* stage, const QkvArgs& qa, int64_t row0,
                                                  int M, int64_t col, int lane, int rows) {
    const int hd = qa.heads * 64;
    const int which = static_cast<int>(col / hd);  // 0 q, 1 k, 2 v: wave-uniform
    const int head = static_cast<int>(col - int64_t{which} * hd) / 64;
    const int piece = lane & 15;
    const bool upper = piece >= 8;
    const int ch = upper ? 32 + (15 - piece) * 4 : piece * 4;
    const float* nw = which < 2 ? qa.nw[which] : nullptr;
    const float* nb = which < 2 ? qa.nb[which] : nullptr;
    const bool norm = nw != nullptr;
    const bool rope = which < 2 && qa.sin_tab != nullptr;
    float wr[4] = {0.0f, 0.0f, 0.0f, 0.0f}, br[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (norm) {
        const float4 w0 = ld_f32x4(nw + ch), b0 = ld_f32x4(nb + ch);
        wr[0] = w0.x, wr[1] = w0.y, wr[2] = w0.z, wr[3] = w0.w;
        br[0] = b0.x, br[1] = b0.y, br[2] = b0.z, br[3] = b0.w;
    }
    float* obase = static_cast<float*>(qa.out[which]) + static_cast<int64_t>(head) * qa.seq * 64 + ch;
    const float sg = upper ? 1.0f : -1.0f;
    // this lane's row: token m = s * seq + t (m < 2^31), advanced by 4 rows
    // per step
    int64_t m = row0 + (lane >> 4);
    uint32_t s = static_cast<uint32_t>(m) / static_cast<uint32_t>(qa.seq);
    int t = static_cast<int>(static_cast<uint32_t>(m) - s * static_cast<uint32_t>(qa.seq));
    for (int rr = 0; rr < rows; rr += 4) {
        if (m >= M) break;  // rows grow with rr: the rest are past M too
        const u32x4 v = ld16(stage + (rr + (lane >> 4)) * kQkvPitch + ch);
        float f[4] = {u2f(v[0]), u2f(v[1]), u2f(v[2]), u2f(v[3])};
        const bool rot = rope && t >= qa.prefix;  // the same for the row's 16 lanes
        float cs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, sn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (rot) {
            const int64_t trow = static_cast<int64_t>(t - qa.prefix) * 64 + ch;
            const float4 c4 = ld_f32x4(qa.cos_tab + trow), s4 = ld_f32x4(qa.sin_tab + trow);
            cs[0] = c4.x, cs[1] = c4.y, cs[2] = c4.z, cs[3] = c4.w;
            sn[0] = sg * s4.x, sn[1] = sg * s4.y, sn[2] = sg * s4.z, sn[3] = sg * s4.w;
        }
        if (norm)
            qk_norm_rope_vec<float, 16, true>(f, wr, br, qa.eps, rot, cs, sn);
        else
            qk_norm_rope_vec<float, 16, false>(f, wr, br, qa.eps, rot, cs, sn);
        u32x4 o;
        o[0] = f2u(f[0]), o[1] = f2u(f[1]), o[2] = f2u(f[2]), o[3] = f2u(f[3]);
        st16(obase + (static_cast<int64_t>(s) * qa.heads * qa.seq + t) * 64, o);
        m += 4;
        t += 4;
        while (t >= qa.seq) t -= qa.seq, s++;
    }
}

template <int EPI, typename P, bool LN>
__global__ __launch_bounds__(P::kThreads, P::kWavesPerEu) void gemm_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ gamma, const float* res, float* out, int M, int N, int K,
    int tiles_n, int ntiles, LnArgs la, QkvArgs qa) {
    constexpr int kRB = P::kRB;
    __shared__ __align__(16) unsigned char smem_raw[f32_smem_bytes<P>(EPI)];
    F32Smem<P>& sm = *reinterpret_cast<F32Smem<P>*>(smem_raw);
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
#if HS_GEMM_XCD
    // the f16 kernel's XCD-aware tile order
    const int per = static_cast<int>(gridDim.x / 8);
    const int tile = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (tile >= ntiles) return;  // padding, before any barrier
#else
    const int tile = static_cast<int>(blockIdx.x);
#endif
    const int64_t m0 = static_cast<int64_t>(tile / tiles_n) * P::kBM;
    const int64_t n0 = static_cast<int64_t>(tile % tiles_n) * P::kBN;
    const int wm = (wave / (P::kWaves / 2)) * (32 * kRB);
    const int wn = (wave % (P::kWaves / 2)) * 64;

    // acc[a][b]: register r of lane (l32, hh) is column wn + 32 a + 8 (r / 4)
    // + 4 hh + r % 4, row wm + 32 b + l32 of the tile
    f32x16 acc[2][kRB];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < kRB; b++) acc[a][b] = f32x16{};

    const int nsteps = K / P::kBK;
    const int wv = wave_in_block();
    const F32Offsets so = f32_offsets(m0, M, K, P::kWaves, wv, lane, P::kXI, P::kWI);
    const int xrows = static_cast<int>(min(static_cast<int64_t>(P::kBM), M - m0));
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + m0 * K), 0, xrows * K * 4, kRawBufferFlags);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(w + n0 * K), 0, P::kBN * K * 4, kRawBufferFlags);
    constexpr int kStageFloats = P::kBK, kStageBytes = P::kBK * 4;
    auto issue = [&](int buf, int koff) {
        f32_issue(sm.x[buf], sm.w[buf], xr, wr, koff, so, P::kWaves, wv, P::kXI, P::kWI);
    };
    // The LayerNorm prologue (hs_linear_ln*): each lane normalises, in
    // place, the x pieces that its own stage loads brought (instruction i:
    // floats (wv + WAVES i) * 256 + 4 lane .. + 4 of the stage), once they
    // have landed (vmcnt, no barrier) and before the barrier that opens the
    // stage to every wave. The pieces' rows are fixed for the kernel, so
    // their (mean, rstd) stay in registers; their logical chunk (lane % 8) ^
    // swz(row) does not depend on i, so a stage needs 4 columns of ln_w and
    // ln_b per lane, loaded one stage ahead. Each element becomes what
    // hs_layernorm stores for it.
    static_assert(P::kWaves % 2 == 0, "a lane's x pieces share one logical chunk");
    f32x2 lst[4];
    int lcol = 0;
    float4 lw = {0.0f, 0.0f, 0.0f, 0.0f}, lb = lw;
    if constexpr (LN) {
#pragma unroll
        for (int i = 0; i < P::kXI; i++) {
            const int row = 8 * (wv + P::kWaves * i) + lane / 8;
            // rows past M hold row M - 1 and take its statistics
            const int64_t r = min(m0 + row, static_cast<int64_t>(M) - 1);
            lst[i] = *reinterpret_cast<const f32x2*>(la.stats + 2 * r);
        }
        lcol = 4 * ((lane % 8) ^ swz(8 * wv + lane / 8));
        lw = ld_f32x4(la.ln_w + lcol), lb = ld_f32x4(la.ln_b + lcol);
    }
    auto normalise = [&](int buf) {  // with the stage's parameters in lw, lb
#pragma unroll
        for (int i = 0; i < P::kXI; i++) {
            float* piece = sm.x[buf] + (wv + P::kWaves * i) * 256 + 4 * lane;
            const u32x4 v = ld16(piece);
            u32x4 o;
            o[0] = f2u(ln_affine(u2f(v[0]), lst[i][0], lst[i][1], lw.x, lb.x));
            o[1] = f2u(ln_affine(u2f(v[1]), lst[i][0], lst[i][1], lw.y, lb.y));
            o[2] = f2u(ln_affine(u2f(v[2]), lst[i][0], lst[i][1], lw.z, lb.z));
            o[3] = f2u(ln_affine(u2f(v[3]), lst[i][0], lst[i][1], lw.w, lb.w));
            st16(piece, o);
        }
    };
    issue(0, 0);
    if (nsteps > 1) issue(1, kStageBytes);
    if constexpr (LN) {
        // stage 0 landed (stage 1's loads, the last issued, may be in flight)
        if (nsteps > 1)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(P::kXI + P::kWI) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        normalise(0);
        if (nsteps > 1) lw = ld_f32x4(la.ln_w + kStageFloats + lcol), lb = ld_f32x4(la.ln_b + kStageFloats + lcol);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        if (nsteps > 1)
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(P::kXI + P::kWI) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    }
    // operand registers in two sets: the next slice is read from LDS while
    // the current one multiplies, across stage boundaries too
    u32x4 A[2][2], B[2][kRB];
#pragma unroll
    for (int a = 0; a < 2; a++) A[0][a] = f32_op(sm.w[0], wn + 32 * a + l32, hh);
#pragma unroll
    for (int b = 0; b < kRB; b++) B[0][b] = f32_op(sm.x[0], wm + 32 * b + l32, hh);
    for (int s = 0; s < nsteps; s++) {
        const int cur = s & 1;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int p = ks & 1;
            if (ks + 1 < 4) {
                const int kc = 2 * (ks + 1) + hh;
#pragma unroll
                for (int a = 0; a < 2; a++) A[p ^ 1][a] = f32_op(sm.w[cur], wn + 32 * a + l32, kc);
#pragma unroll
                for (int b = 0; b < kRB; b++) B[p ^ 1][b] = f32_op(sm.x[cur], wm + 32 * b + l32, kc);
            } else {
                // every wave's reads of stage s are done and stage s + 1 has
                // landed (and, with the prologue, is normalised); buffer cur
                // is refilled with stage s + 2
                if constexpr (LN) {
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    if (s + 1 < nsteps) {
                        normalise(cur ^ 1);
                        if (s + 2 < nsteps) {
                            const int c = (s + 2) * kStageFloats + lcol;
                            lw = ld_f32x4(la.ln_w + c), lb = ld_f32x4(la.ln_b + c);
                        }
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                } else {
                    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                }
                if (s + 2 < nsteps) issue(cur, (s + 2) * kStageBytes);
                if (s + 1 < nsteps) {
#pragma unroll
                    for (int a = 0; a < 2; a++) A[p ^ 1][a] = f32_op(sm.w[cur ^ 1], wn + 32 * a + l32, hh);
#pragma unroll
                    for (int b = 0; b < kRB; b++) B[p ^ 1][b] = f32_op(sm.x[cur ^ 1], wm + 32 * b + l32, hh);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int a = 0; a < 2; a++)
#pragma unroll
                    for (int b = 0; b < kRB; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(u2f(A[p][a][j]), u2f(B[p][b][j]),
                                                                         acc[a][b], 0, 0, 0);
        }
    }

    if constexpr (EPI == EPI_QKV) {
        // every wave has left the main loop: the stages' LDS takes the
        // waves' blocks
        __syncthreads();
        float* stage = reinterpret_cast<float*>(smem_raw) + wave * (32 * kRB * kQkvPitch);
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const int cl = 32 * a + 8 * r4 + 4 * hh;
                const float4 bv = bias ? ld_f32x4(bias + n0 + wn + cl) : float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int b = 0; b < kRB; b++) {
                    u32x4 o;
                    o[0] = f2u(acc[a][b][4 * r4] + bv.x), o[1] = f2u(acc[a][b][4 * r4 + 1] + bv.y);
                    o[2] = f2u(acc[a][b][4 * r4 + 2] + bv.z), o[3] = f2u(acc[a][b][4 * r4 + 3] + bv.w);
                    st16(stage + (32 * b + l32) * kQkvPitch + cl, o);
                }
            }
        // only this wave reads its block back: a wave-level fence suffices
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        qkv_heads_out_f32(stage, qa, m0 + wm, M, n0 + wn, lane, 32 * kRB);
        return;
    }
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
            const int64_t n = n0 + wn + 32 * a + 8 * r4 + 4 * hh;
            const float4 bv = bias ? ld_f32x4(bias + n) : float4{0.0f, 0.0f, 0.0f, 0.0f};
            float4 gv = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (EPI == EPI_LS) gv = ld_f32x4(gamma + n);
#pragma unroll
            for (int b = 0; b < kRB; b++) {
                const int64_t m = m0 + wm + 32 * b + l32;
                if (m >= M) continue;
                float v[4] = {acc[a][b][4 * r4] + bv.x, acc[a][b][4 * r4 + 1] + bv.y,
                              acc[a][b][4 * r4 + 2] + bv.z, acc[a][b][4 * r4 + 3] + bv.w};
                if constexpr (EPI == EPI_GELU) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = gelu_f(v[e]);
                }
                if constexpr (EPI == EPI_LS) {
                    // res + gamma * x, read and written by this lane only
                    // (res may be out)
                    const float4 rv = ld_f32x4(res + m * N + n);
                    v[0] = rv.x + gv.x * v[0], v[1] = rv.y + gv.y * v[1];
                    v[2] = rv.z + gv.z * v[2], v[3] = rv.w + gv.w * v[3];
                }
                u32x4 o;
                o[0] = f2u(v[0]), o[1] = f2u(v[1]), o[2] = f2u(v[2]), o[3] = f2u(v[3]);
                st16_nt(out + m * N + n, o);
            }
        }
}

// ---------------------------------------------------------------------------
// generic path: 64 x 64 output tile per 256 threads, 4 x 4 per thread,
// K in steps of 16 through LDS; f32 accumulation in K order.

constexpr int kGT = 64, kGK = 16;

template <typename T, int EPI, bool LN>
__global__ __launch_bounds__(256) void gemm_generic_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ gamma, const T* res, T* out, int M, int N, int K, int tiles_n,
    LnArgs la) {
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
            float xv = (xm < M && kidx < K) ? static_cast<float>(x[xm * K + kidx]) : 0.0f;
            if constexpr (LN) {
                // the element as hs_layernorm stores it
                if (xm < M && kidx < K)
                    xv = storage_round(ln_affine(xv, la.stats[2 * xm], la.stats[2 * xm + 1],
                                                 la.ln_w[kidx], la.ln_b[kidx]),
                                       T{});
            }
            xs[kk][rr] = xv;
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
            if constexpr (EPI == EPI_GELU) v = gelu_f(v);
            if constexpr (EPI == EPI_LS)
                v = static_cast<float>(res[m * N + n]) + gamma[n] * storage_round(v, T{});
            out[m * N + n] = static_cast<T>(v);
        }
    }
}

bool fast_shape(hs_dtype dt, int N, int K, const void* x, const void* w, const float* bias,
                const float* gamma, const void* out, const void* res) {
    // K == 0 takes the generic kernel (out = bias): the fast path's first
    // stage would read K-tiles that do not exist
    // K <= 2^20 keeps a tile's byte offsets (256 rows x K x 2) in 32 bits
    return dt == HS_F16 && N % kBN == 0 && K > 0 && K % kBK == 0 && K <= (1 << 20) && aligned16(x) && aligned16(w) &&
           (!bias || aligned16(bias)) && (!gamma || aligned16(gamma)) && aligned16(out) &&
           (!res || aligned16(res));
}

// Fast-path eligibility of a call, decided before anything is enqueued.
template <bool LN>
bool takes_fast_path(hs_dtype dt, int N, int K, const void* x, const void* w, const float* bias,
                     const float* gamma, const void* out, const void* res, const LnArgs& la) {
    return fast_shape(dt, N, K, x, w, bias, gamma, out, res) &&
           (!LN || (aligned16(la.ln_w) && aligned16(la.ln_b)));
}

#ifndef HS_GEMM_F32_NARROW_TILES
#define HS_GEMM_F32_NARROW_TILES 512  // 128 x 128 tiles below which F32Narrow runs
#endif

// f32 matrix-core eligibility: shape and alignment.
bool f32_fast(hs_dtype dt, int N, int K, const void* x, const void* w, const float* bias,
              const float* gamma, const void* out, const void* res) {
    // K <= 2^19 keeps a tile's byte offsets (128 rows x K x 4) in 32 bits
    return dt == HS_F32 && N % F32Shape::kBN == 0 && K > 0 && K % F32Shape::kBK == 0 &&
           K <= (1 << 19) && aligned16(x) && aligned16(w) && (!bias || aligned16(bias)) &&
           (!gamma || aligned16(gamma)) && aligned16(out) && (!res || aligned16(res));
}

template <int EPI, typename P, bool LN>
void launch_f32(hipStream_t st, const void* x, const void* w, const float* bias, const float* gamma,
                const void* res, void* out, int M, int N, int K, const LnArgs& la, const QkvArgs& qa) {
    const int tiles_n = N / P::kBN;
    const int64_t ntiles = ceil_div(M, P::kBM) * tiles_n;
    const int64_t blocks = HS_GEMM_XCD ? ceil_div(ntiles, 8) * 8 : ntiles;
    gemm_f32_kernel<EPI, P, LN><<<dim3(static_cast<uint32_t>(blocks)), dim3(P::kThreads), 0, st>>>(
        static_cast<const float*>(x), static_cast<const float*>(w), bias, gamma,
        static_cast<const float*>(res), static_cast<float*>(out), M, N, K, tiles_n,
        static_cast<int>(ntiles), la, qa);
}

template <int EPI, bool LN = false>
hs_status launch(hipStream_t st, hs_dtype dt, const void* x, const void* w, const float* bias,
                 const float* gamma, const void* res, void* out, int M, int N, int K,
                 const char* op, const QkvArgs& qa = QkvArgs{}, const LnArgs& la = LnArgs{}) {
    if (f32_fast(dt, N, K, x, w, bias, gamma, out, res) &&
        (!LN || (aligned16(la.ln_w) && aligned16(la.ln_b)))) {
        if (ceil_div(M, F32Shape::kBM) * (N / F32Shape::kBN) < HS_GEMM_F32_NARROW_TILES)
            launch_f32<EPI, F32Narrow, LN>(st, x, w, bias, gamma, res, out, M, N, K, la, qa);
        else
            launch_f32<EPI, F32Shape, LN>(st, x, w, bias, gamma, res, out, M, N, K, la, qa);
        return check_launch(op);
    }
    if (takes_fast_path<LN>(dt, N, K, x, w, bias, gamma, out, res, la)) {
        const int tiles_n = N / kBN;
        const int64_t ntiles = ceil_div(M, kBM) * tiles_n;
        const int64_t blocks = HS_GEMM_XCD ? ceil_div(ntiles, 8) * 8 : ntiles;
        gemm_f16_kernel<EPI, LN><<<dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, st>>>(
            static_cast<const f16*>(x), static_cast<const f16*>(w), bias, gamma,
            static_cast<const f16*>(res), static_cast<f16*>(out), M, N, K, tiles_n,
            static_cast<int>(ntiles), qa, la);
        return check_launch(op);
    }
    if constexpr (EPI == EPI_QKV) {
        return fail(HS_EUNSUPPORTED,
                    "%s: needs K %% %d == 0 (f16) or %% %d == 0 (f32) and 16-byte aligned buffers", op,
                    kBK, F32Shape::kBK);
    } else {
        const int tiles_n = static_cast<int>(ceil_div(N, kGT));
        const int64_t blocks = ceil_div(M, kGT) * tiles_n;
        if (dt == HS_F16)
            gemm_generic_kernel<f16, EPI, LN><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, st>>>(
                static_cast<const f16*>(x), static_cast<const f16*>(w), bias, gamma,
                static_cast<const f16*>(res), static_cast<f16*>(out), M, N, K, tiles_n, la);
        else
            gemm_generic_kernel<float, EPI, LN><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, st>>>(
                static_cast<const float*>(x), static_cast<const float*>(w), bias, gamma,
                static_cast<const float*>(res), static_cast<float*>(out), M, N, K, tiles_n, la);
        return check_launch(op);
    }
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

namespace hs {
namespace {

// Validation and arguments of the q|k|v projection with heads (shared by
// hs_linear_qkv_heads and hs_linear_ln_qkv_heads). Returns HS_OK with
// *skip set for zero-size work.
hs_status qkv_setup(const char* op, hs_dtype dt, const void* x, const void* w_qkv,
                    const float* qn_w, const float* qn_b, const float* kn_w, const float* kn_b,
                    const float* sin_tab, const float* cos_tab, void* q_out, void* k_out,
                    void* v_out, int32_t S, int32_t T, int32_t H, int32_t d, int32_t k,
                    int32_t prefix, float eps, QkvArgs* qa, bool* skip) {
    *skip = false;
    if (!valid_dtype(dt)) return fail(HS_EINVAL, "%s: unknown dtype", op);
    if (S < 0 || T < 0 || H <= 0 || d <= 0 || k <= 0)
        return fail(HS_EINVAL, "%s: shape S=%d T=%d H=%d d=%d k=%d", op, S, T, H, d, k);
    if (prefix < 0 || prefix > T) return fail(HS_EINVAL, "%s: prefix %d outside [0, %d]", op, prefix, T);
    if ((qn_w == nullptr) != (qn_b == nullptr) || (kn_w == nullptr) != (kn_b == nullptr))
        return fail(HS_EINVAL, "%s: a norm needs both weight and bias", op);
    if ((sin_tab == nullptr) != (cos_tab == nullptr))
        return fail(HS_EINVAL, "%s: RoPE needs both tables", op);
    if (!(eps > 0.0f)) return fail(HS_EINVAL, "%s: eps must be positive", op);
    const int64_t M = int64_t{S} * T;
    const int64_t N = int64_t{3} * H * d;
    if (N >= (int64_t{1} << 31) || M >= (int64_t{1} << 31) || M * N >= (int64_t{1} << 40) ||
        M * k >= (int64_t{1} << 40))
        return fail(HS_EINVAL, "%s: too large", op);
    if (M == 0) {
        *skip = true;
        return HS_OK;
    }
    if (!x || !w_qkv || !q_out || !k_out || !v_out) return fail(HS_EINVAL, "%s: null buffer", op);
    const int64_t esz = dtype_size(dt), ob = M * H * d * esz;  // each of q, k, v
    const void* outs[3] = {q_out, k_out, v_out};
    for (int i = 0; i < 3; i++) {
        if (overlaps(outs[i], ob, x, M * k * esz) || overlaps(outs[i], ob, w_qkv, N * k * esz))
            return fail(HS_EINVAL, "%s: an output overlaps x or w", op);
        for (int j = 0; j < i; j++)
            if (overlaps(outs[i], ob, outs[j], ob)) return fail(HS_EINVAL, "%s: outputs overlap", op);
    }
    // The fused epilogue needs one head per wave (64 columns) and whole
    // column tiles (256 in f16, 128 in f32); other shapes run linear then
    // qknorm_rope.
    const int64_t tile_n = dt == HS_F16 ? kBN : F32Shape::kBN;
    if (d != 64 || N % tile_n != 0)
        return fail(HS_EUNSUPPORTED, "%s: needs head dim 64 and 3*H*64 %% %lld == 0", op,
                    static_cast<long long>(tile_n));
    const float* params[6] = {qn_w, qn_b, kn_w, kn_b, sin_tab, cos_tab};
    for (const float* p : params)
        if (p && !aligned16(p)) return fail(HS_EUNSUPPORTED, "%s: parameters must be 16-byte aligned", op);
    if (!aligned16(k_out) || !aligned16(v_out))
        return fail(HS_EUNSUPPORTED, "%s: outputs must be 16-byte aligned", op);
    *qa = QkvArgs{};
    qa->out[0] = q_out, qa->out[1] = k_out, qa->out[2] = v_out;
    qa->nw[0] = qn_w, qa->nb[0] = qn_b, qa->nw[1] = kn_w, qa->nb[1] = kn_b;
    qa->sin_tab = sin_tab, qa->cos_tab = cos_tab;
    qa->seq = T, qa->heads = H, qa->prefix = prefix, qa->eps = eps;
    return HS_OK;
}

// A byte range that the LayerNorm prologue's workspace must not overlap.
struct Span {
    const void* p;
    int64_t bytes;
};

// Checks of the LayerNorm prologue's operands: ln_w and ln_b (k f32 each)
// and the workspace (2 m floats, 8-byte aligned), which receives each x
// row's (mean, rstd) and so must not overlap any buffer the call reads or
// writes (`spans`).
hs_status ln_check(const char* op, const float* ln_w, const float* ln_b, const float* workspace,
                   int64_t M, int32_t K, float eps, std::initializer_list<Span> spans) {
    if (!ln_w || !ln_b || !workspace) return fail(HS_EINVAL, "%s: null buffer", op);
    if (!(eps > 0.0f)) return fail(HS_EINVAL, "%s: eps must be positive", op);
    if (reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
        return fail(HS_EINVAL, "%s: workspace must be 8-byte aligned", op);
    const int64_t wsb = M * 8;
    if (overlaps(workspace, wsb, ln_w, int64_t{K} * 4) ||
        overlaps(workspace, wsb, ln_b, int64_t{K} * 4))
        return fail(HS_EINVAL, "%s: workspace overlaps the LayerNorm parameters", op);
    for (const Span& sp : spans)
        if (sp.p && overlaps(workspace, wsb, sp.p, sp.bytes))
            return fail(HS_EINVAL, "%s: workspace overlaps an operand", op);
    return HS_OK;
}

// hs_linear_ln / hs_linear_ln_gelu (and the allocation-free variant): the
// row statistics into ws, then the product with the LayerNorm prologue.
template <int EPI>
hs_status linear_ln_entry(const char* op, hipStream_t st, hs_dtype dt, const void* x,
                          const float* ln_w, const float* ln_b, const void* w, const float* bias,
                          float* ws, void* out, int64_t m, int32_t n, int32_t k, float eps) {
    hs_status rc = check(op, dt, x, w, nullptr, out, m, n, k, false);
    if (rc != HS_OK || m == 0 || n == 0) return rc;
    if (k == 0) return fail(HS_EINVAL, "%s: k must be positive", op);
    const int64_t esz = dtype_size(dt);
    rc = ln_check(op, ln_w, ln_b, ws, m, k, eps,
                  {{x, m * k * esz}, {w, int64_t{n} * k * esz}, {bias, int64_t{n} * 4},
                   {out, m * n * esz}});
    if (rc != HS_OK) return rc;
    // (a failure keeps the statistics launch's own message)
    rc = hs_layernorm_stats(st, dt, x, ws, m, k, eps);
    if (rc != HS_OK) return rc;
    return launch<EPI, true>(st, dt, x, w, bias, nullptr, nullptr, out, static_cast<int>(m), n, k,
                             op, QkvArgs{}, LnArgs{ws, ln_w, ln_b});
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_linear_qkv_heads(hs_stream_t stream, hs_dtype dt, const void* x,
                                         const void* w_qkv, const float* b_qkv, const float* qn_w,
                                         const float* qn_b, const float* kn_w, const float* kn_b,
                                         const float* sin_tab, const float* cos_tab, void* q_out,
                                         void* k_out, void* v_out, int32_t S, int32_t T,
                                         int32_t H, int32_t d, int32_t k, int32_t prefix,
                                         float eps) {
    using namespace hs;
    const char* op = "linear_qkv_heads";
    QkvArgs qa;
    bool skip;
    const hs_status rc = qkv_setup(op, dt, x, w_qkv, qn_w, qn_b, kn_w, kn_b, sin_tab, cos_tab,
                                   q_out, k_out, v_out, S, T, H, d, k, prefix, eps, &qa, &skip);
    if (rc != HS_OK || skip) return rc;
    const int64_t M = int64_t{S} * T, N = int64_t{3} * H * d;
    return launch<EPI_QKV>(static_cast<hipStream_t>(stream), dt, x, w_qkv, b_qkv, nullptr, nullptr,
                           q_out, static_cast<int>(M), static_cast<int>(N), k, op, qa);
}

extern "C" hs_status hs_linear_ln(hs_stream_t stream, hs_dtype dt, const void* x,
                                  const float* ln_w, const float* ln_b, const void* w,
                                  const float* bias, float* workspace, void* out, int64_t m,
                                  int32_t n, int32_t k, float eps) {
    return hs::linear_ln_entry<hs::EPI_BIAS>("linear_ln", static_cast<hipStream_t>(stream), dt, x,
                                             ln_w, ln_b, w, bias, workspace, out, m, n, k, eps);
}

extern "C" hs_status hs_linear_ln_gelu(hs_stream_t stream, hs_dtype dt, const void* x,
                                       const float* ln_w, const float* ln_b, const void* w,
                                       const float* bias, float* workspace, void* out, int64_t m,
                                       int32_t n, int32_t k, float eps) {
    return hs::linear_ln_entry<hs::EPI_GELU>("linear_ln_gelu", static_cast<hipStream_t>(stream), dt,
                                             x, ln_w, ln_b, w, bias, workspace, out, m, n, k, eps);
}

extern "C" hs_status hs_linear_ln_qkv_heads(hs_stream_t stream, hs_dtype dt, const void* x,
                                            const float* ln_w, const float* ln_b,
                                            const void* w_qkv, const float* b_qkv,
                                            const float* qn_w, const float* qn_b,
                                            const float* kn_w, const float* kn_b,
                                            const float* sin_tab, const float* cos_tab,
                                            float* workspace, void* q_out, void* k_out,
                                            void* v_out, int32_t S, int32_t T, int32_t H,
                                            int32_t d, int32_t k, int32_t prefix, float eps) {
    using namespace hs;
    const char* op = "linear_ln_qkv_heads";
    QkvArgs qa;
    bool skip;
    hs_status rc = qkv_setup(op, dt, x, w_qkv, qn_w, qn_b, kn_w, kn_b, sin_tab, cos_tab, q_out,
                             k_out, v_out, S, T, H, d, k, prefix, eps, &qa, &skip);
    if (rc != HS_OK || skip) return rc;
    const int64_t M = int64_t{S} * T, N = int64_t{3} * H * d;
    const int64_t esz = dtype_size(dt), ob = M * H * d * esz;
    const int64_t tab = int64_t{T - prefix} * d * 4;
    rc = ln_check(op, ln_w, ln_b, workspace, M, k, eps,
                  {{x, M * k * esz}, {w_qkv, N * k * esz}, {b_qkv, N * 4}, {qn_w, d * 4},
                   {qn_b, d * 4}, {kn_w, d * 4}, {kn_b, d * 4}, {sin_tab, tab}, {cos_tab, tab},
                   {q_out, ob}, {k_out, ob}, {v_out, ob}});
    if (rc != HS_OK) return rc;
    const LnArgs la{workspace, ln_w, ln_b};
    // the q|k|v epilogue exists on the matrix-core path only: refuse other
    // calls before the statistics are enqueued
    const bool f32_ok = f32_fast(dt, static_cast<int>(N), k, x, w_qkv, b_qkv, nullptr, q_out, nullptr) &&
                        aligned16(ln_w) && aligned16(ln_b);
    if (!f32_ok && !takes_fast_path<true>(dt, static_cast<int>(N), k, x, w_qkv, b_qkv, nullptr, q_out,
                                          nullptr, la))
        return fail(HS_EUNSUPPORTED,
                    "%s: needs K %% %d == 0 (f16) or %% %d == 0 (f32) and 16-byte aligned buffers", op,
                    kBK, F32Shape::kBK);
    hipStream_t st = static_cast<hipStream_t>(stream);
    rc = hs_layernorm_stats(st, dt, x, workspace, M, k, eps);
    if (rc != HS_OK) return rc;
    return launch<EPI_QKV, true>(st, dt, x, w_qkv, b_qkv, nullptr, nullptr, q_out,
                                 static_cast<int>(M), static_cast<int>(N), k, op, qa, la);
}

// ---------------------------------------------------------------------------
// An allocation-free variant of hs_linear_ln_gelu: the row statistics live
// in a file-scope device array instead of a caller workspace. Each device the
// library runs on holds its own copy for the life of the process; its device
// address comes from hipGetSymbolAddress, taken once per device (with that
// device current) on the first call there. Every call on a device shares
// that device's array, so calls that overlap on one device race; the array
// keeps the last call's statistics, and each call writes every row it reads.

namespace hs {
namespace {

constexpr int64_t kNoAllocMaxRows = int64_t{1} << 19;  // 524,288 rows: 4 MiB of statistics
static __device__ __align__(256) float scratch[2 * kNoAllocMaxRows];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kScratchDevices];  // device address of `scratch` per device, once taken

// The current device's address of `scratch` (nullptr with *rc and the
// error message set on failure). The array's host-side name is not a device
// address: only the pointer returned by hipGetSymbolAddress goes to kernels.
float* scratch_address(const char* op, hs_status* rc) {
    int dev = 0;
    const hipError_t de = hipGetDevice(&dev);
    if (de != hipSuccess) {
        *rc = fail(HS_EHIP, "%s: hipGetDevice: %s", op, hipGetErrorString(de));
        return nullptr;
    }
    if (dev < 0 || dev >= kScratchDevices) {
        *rc = fail(HS_EUNSUPPORTED, "%s: device %d beyond the %d the library tracks", op, dev,
                   kScratchDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            *rc = fail(HS_EHIP, "%s: hipGetSymbolAddress(scratch): %s", op, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch[dev] = static_cast<float*>(ptr);
    }
    return g_scratch[dev];
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_linear_ln_gelu_noalloc(hs_stream_t stream, hs_dtype dt, const void* x,
                                               const float* ln_w, const float* ln_b,
                                               const void* w, const float* bias, void* out,
                                               int64_t m, int32_t n, int32_t k, float eps) {
    using namespace hs;
    const char* op = "linear_ln_gelu_noalloc";
    if (m > kNoAllocMaxRows)
        return fail(HS_EINVAL, "%s: m = %lld rows exceeds the statistics array's %lld", op,
                    static_cast<long long>(m), static_cast<long long>(kNoAllocMaxRows));
    if (m <= 0 || n <= 0)  // the shape checks and zero-size returns of the workspace entry
        return linear_ln_entry<EPI_GELU>(op, static_cast<hipStream_t>(stream), dt, x, ln_w, ln_b,
                                         w, bias, nullptr, out, m, n, k, eps);
    hs_status rc = HS_OK;
    float* ws = scratch_address(op, &rc);
    if (ws == nullptr) return rc;
    return linear_ln_entry<EPI_GELU>(op, static_cast<hipStream_t>(stream), dt, x, ln_w, ln_b, w,
                                     bias, ws, out, m, n, k, eps);
}
