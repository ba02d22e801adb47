// Patch-token assembly for gfx950: one pass that builds the (S*T, D) token
// matrix the first block reads (model/trunk.rs:68-85: per frame a camera
// token variant, R register token variants and the P patch tokens; the
// reference issues 3*S buffer copies plus a full f32 -> f16 cast pass, and
// DINO adds the patch-embed bias in its GEMM epilogue, model/dino.rs:76-93).
// Patch rows fold the patch bias and the positional-embedding add (the
// tiled_add.wesl semantics, out[i] = x[i] + table[i % block]) into the cast,
// so each patch element is read once in its input dtype and written once.
//
// Each lane moves LV = 4 consecutive channels per step, one 1 KiB chunk
// of the row per wave instruction (8 channels per lane, one 16-byte f16
// store each, measured slower: 66% of peak against 72.7% at S=32); the
// row's chunks are split over HS_AS_SPLIT waves. Rows are independent; the
// camera/register gather is row-granular, so no LDS staging is needed.
#include "hs_common.hpp"

namespace hs {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / 64;
// Launch shape (overridable at build time for tuning sweeps).
#ifndef HS_AS_BPC
#define HS_AS_BPC 8  // resident workgroups per CU (generic path)
#endif
#ifndef HS_AS_F
#define HS_AS_F 4  // frames per wave of one patch position
#endif
constexpr int kBlocksPerCu = HS_AS_BPC;
constexpr int kFramesPerWave = HS_AS_F;

// LV consecutive channels per lane (4 or 8), converted to f32.
template <int LV>
__device__ __forceinline__ void loadv(const float* p, float (&f)[LV]) {
#pragma unroll
    for (int i = 0; i < LV; i += 4) {
        const float4 v = ld_f32x4(p + i);
        f[i] = v.x, f[i + 1] = v.y, f[i + 2] = v.z, f[i + 3] = v.w;
    }
}
__device__ __forceinline__ void unpack_h(uint32_t u, float& a, float& b) {
    const f16x2 h = u2h2(u);
    a = static_cast<float>(h.x), b = static_cast<float>(h.y);
}
template <int LV>
__device__ __forceinline__ void loadv(const f16* p, float (&f)[LV]) {
    if constexpr (LV == 8) {
        const u32x4 v = ld16(p);
#pragma unroll
        for (int k = 0; k < 4; k++) unpack_h(v[k], f[2 * k], f[2 * k + 1]);
    } else {
        const u32x2 v = *reinterpret_cast<const u32x2*>(p);
        unpack_h(v[0], f[0], f[1]), unpack_h(v[1], f[2], f[3]);
    }
}
// Patch loads and token stores stream (non-temporal); camera/register rows
// and the positional table are reread across frames and stay cached.
template <int LV>
__device__ __forceinline__ void loadv_stream(const float* p, float (&f)[LV]) {
#pragma unroll
    for (int i = 0; i < LV; i += 4) {
        const u32x4 v = ld_stream(p + i);
        f[i] = u2f(v[0]), f[i + 1] = u2f(v[1]), f[i + 2] = u2f(v[2]), f[i + 3] = u2f(v[3]);
    }
}
template <int LV>
__device__ __forceinline__ void loadv_stream(const f16* p, float (&f)[LV]) {
    if constexpr (LV == 8) {
        const u32x4 v = ld_stream(p);
#pragma unroll
        for (int k = 0; k < 4; k++) unpack_h(v[k], f[2 * k], f[2 * k + 1]);
    } else {
        const u32x2 v = ld_stream_as(reinterpret_cast<const u32x2*>(p));
        unpack_h(v[0], f[0], f[1]), unpack_h(v[1], f[2], f[3]);
    }
}
template <int LV>
__device__ __forceinline__ void storev(float* p, const float (&f)[LV]) {
#pragma unroll
    for (int i = 0; i < LV; i += 4) {
        u32x4 v;
        v[0] = f2u(f[i]), v[1] = f2u(f[i + 1]), v[2] = f2u(f[i + 2]), v[3] = f2u(f[i + 3]);
        st_stream(p + i, v);
    }
}
__device__ __forceinline__ uint32_t pack_h(float a, float b) {
    f16x2 h;
    h.x = static_cast<f16>(a), h.y = static_cast<f16>(b);
    return h22u(h);
}
template <int LV>
__device__ __forceinline__ void storev(f16* p, const float (&f)[LV]) {
    if constexpr (LV == 8) {
        u32x4 v;
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = pack_h(f[2 * k], f[2 * k + 1]);
        st_stream(p, v);
    } else {
        u32x2 v;
        v[0] = pack_h(f[0], f[1]), v[1] = pack_h(f[2], f[3]);
        st_stream_as(reinterpret_cast<u32x2*>(p), v);
    }
}

// Patch-row value as the reference sequence stores it: the GEMM epilogue
// stores (x + bias) in the patch dtype, then tiled_add adds pos.
template <typename TP>
__device__ __forceinline__ float patch_value(float x, float b, float p, bool has_b, bool has_p) {
    if (has_b) x = storage_round(x + b, TP{});
    if (has_p) x = storage_round(x + p, TP{});
    return x;
}

// Workgroup -> rows, XCD-aware. Workgroups are dispatched round-robin over
// the XCDs (workgroup b runs on XCD b % kXcds), each XCD with its own L2.
// Patch rows come first. XCD x owns the patch positions [x PP, (x + 1) PP),
// PP = ceil(P / kXcds), so each XCD's L2 holds only its 1/kXcds share of the
// positional table. Within an XCD the workgroups walk the frames in groups of
// F = kFramesPerWave: workgroup b (local index l = b / kXcds) takes frame
// group l / C and positions x PP + n (l % C) + [0, n), n = 4 / SPLIT
// positions per workgroup, C = ceil(PP / n), SPLIT waves per position (each
// its share of the row's chunks), for the F frames of its group. A wave keeps its
// position's table row and the bias in registers across its F frames, the
// four waves of a workgroup read four consecutive patch rows of each frame,
// and the whole chip sweeps the frames in order, so the reads in flight at
// any time sit in a few frames' contiguous row ranges. (Position-major order,
// one position for all frames per workgroup, measured 9% slower at S=32.)
// Camera/register rows follow, 4 per workgroup.
constexpr int kXcds = 8;

#ifndef HS_AS_SPLIT
// waves per patch row, each taking 1/SPLIT of the row's 1 KiB chunks: at
// S=32 (D=1024, four chunks) 4 took 44.9-45.8 us warm / 46.2-46.4 cold
// against 46.5 / 47.1-47.6 for 1 (a whole row per wave) and 45.3-46.2 /
// 46.3-46.5 for 2
#define HS_AS_SPLIT 4
#endif

struct AssembleGrid {
    int64_t patch_blocks;  // kXcds * ceil(S / F) * C
    int64_t special_blocks;
    int chunks;            // C: workgroups per frame group per XCD
    int pp;                // PP: positions per XCD
    // SPL waves share a patch row: a workgroup covers kWavesPerBlock / SPL
    // positions
    __host__ __device__ static AssembleGrid make(int s, int np, int nr, int spl) {
        AssembleGrid g;
        g.pp = static_cast<int>(ceil_div(np, kXcds));
        g.chunks = static_cast<int>(ceil_div(g.pp, kWavesPerBlock / spl));
        g.patch_blocks = static_cast<int64_t>(kXcds) * ceil_div(s, kFramesPerWave) * g.chunks;
        g.special_blocks = ceil_div(static_cast<int64_t>(s) * (1 + nr), kWavesPerBlock);
        return g;
    }
};

template <typename TO, typename TP, int CHUNKS, int LV, int SPL>
__global__ __launch_bounds__(kBlock) void assemble_kernel(
    const TP* __restrict__ patches, const float* __restrict__ pbias, const float* __restrict__ pos,
    const TO* __restrict__ cam, const TO* __restrict__ reg, TO* __restrict__ out, int nframes,
    int seq, int np, int nr, int n_var) {
    constexpr int CW = 64 * LV;  // channels per chunk: LV per lane
    constexpr int D = CW * CHUNKS;
    const int lane = lane_id();
    const int w = wave_in_block();
    const AssembleGrid grid = AssembleGrid::make(nframes, np, nr, SPL);
    const int64_t b = blockIdx.x;
    if (b < grid.patch_blocks) {
        constexpr int F = kFramesPerWave;
        constexpr int CH = CHUNKS / SPL;  // chunks of the row this wave takes
        static_assert(CHUNKS % SPL == 0, "whole chunks per wave");
        const int x = static_cast<int>(b % kXcds);
        const int64_t l = b / kXcds;
        const int fg = static_cast<int>(l / grid.chunks);
        const int g = static_cast<int>(l - static_cast<int64_t>(fg) * grid.chunks);
        const int64_t p = static_cast<int64_t>(x) * grid.pp + g * (kWavesPerBlock / SPL) + w / SPL;
        const int c_lo = (w % SPL) * CH;  // first chunk of this wave's share
        const int f0 = fg * F;
        // wave-uniform; the kernel has no barriers
        if (p >= static_cast<int64_t>(x + 1) * grid.pp || p >= np || f0 >= nframes) return;
        const int f1 = f0 + F < nframes ? f0 + F : nframes;
        const bool has_b = pbias != nullptr, has_p = pos != nullptr;
        float pe[CH][LV], bv[CH][LV];
#pragma unroll
        for (int c = 0; c < CH; c++) {
#pragma unroll
            for (int k = 0; k < LV; k++) pe[c][k] = bv[c][k] = 0.0f;
            if (has_p) loadv(pos + p * D + (c_lo + c) * CW + lane * LV, pe[c]);
            if (has_b) loadv(pbias + (c_lo + c) * CW + lane * LV, bv[c]);
        }
        const TP* src = patches + (static_cast<int64_t>(f0) * np + p) * D + c_lo * CW + lane * LV;
        TO* orow = out + (static_cast<int64_t>(f0) * seq + 1 + nr + p) * D + c_lo * CW + lane * LV;
        const int64_t src_step = static_cast<int64_t>(np) * D, out_step = static_cast<int64_t>(seq) * D;
        auto load = [&](float (&x)[CH][LV], int f) {
#pragma unroll
            for (int c = 0; c < CH; c++) loadv_stream(src + (f - f0) * src_step + c * CW, x[c]);
        };
        auto emit = [&](float (&x)[CH][LV], int f) {
#pragma unroll
            for (int c = 0; c < CH; c++) {
#pragma unroll
                for (int k = 0; k < LV; k++)
                    x[c][k] = patch_value<TP>(x[c][k], bv[c][k], pe[c][k], has_b, has_p);
                storev(orow + (f - f0) * out_step + c * CW, x[c]);
            }
        };
        // two-buffer pipeline over the wave's frames: the next frame's row
        // is in flight while the current one is summed and stored
        float xa[CH][LV], xb[CH][LV];
        load(xa, f0);
#pragma unroll 1
        for (int f = f0; f < f1; f += 2) {
            if (f + 1 < f1) load(xb, f + 1);
            emit(xa, f);
            if (f + 1 >= f1) break;
            if (f + 2 < f1) load(xa, f + 2);
            emit(xb, f + 1);
        }
        return;
    }
    // camera / register rows
    const int64_t j = (b - grid.patch_blocks) * kWavesPerBlock + w;
    if (j >= static_cast<int64_t>(nframes) * (1 + nr)) return;
    const int f = static_cast<int>(j / (1 + nr));
    const int t = static_cast<int>(j - static_cast<int64_t>(f) * (1 + nr));
    const int v = (n_var == 2 && f != 0) ? 1 : 0;
    const TO* src = t == 0 ? cam + static_cast<int64_t>(v) * D
                           : reg + (static_cast<int64_t>(v) * nr + (t - 1)) * D;
    TO* orow = out + (static_cast<int64_t>(f) * seq + t) * D + lane * LV;
    float vals[CHUNKS][LV];
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) loadv(src + c * CW + lane * LV, vals[c]);
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) storev(orow + c * CW, vals[c]);
}

// Any D, any alignment: lanes strided over the row.
template <typename TO, typename TP>
__global__ __launch_bounds__(kBlock) void assemble_generic_kernel(
    const TP* patches, const float* pbias, const float* pos, const TO* cam, const TO* reg, TO* out,
    int64_t out_rows, int seq, int np, int nr, int d, int n_var) {
    const int lane = lane_id();
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
    const bool has_b = pbias != nullptr, has_p = pos != nullptr;
    for (int64_t row = wave; row < out_rows; row += nwaves) {
        const int64_t f = row / seq;
        const int t = static_cast<int>(row - f * seq);
        const int64_t v = (n_var == 2 && f != 0) ? 1 : 0;
        TO* orow = out + row * d;
        if (t <= nr) {
            const TO* src = t == 0 ? cam + v * d : reg + (v * nr + (t - 1)) * d;
            for (int j = lane; j < d; j += 64) orow[j] = src[j];
        } else {
            const int64_t p = t - 1 - nr;
            const TP* src = patches + (f * np + p) * d;
            for (int j = lane; j < d; j += 64) {
                float x = load_elem(src + j);
                x = patch_value<TP>(x, has_b ? pbias[j] : 0.0f, has_p ? pos[p * d + j] : 0.0f,
                                    has_b, has_p);
                store_elem(orow + j, x);
            }
        }
    }
}

int64_t persistent_blocks(int64_t work_waves) {
    const int64_t cap = static_cast<int64_t>(num_cus()) * kBlocksPerCu;
    const int64_t blocks = ceil_div(work_waves, kWavesPerBlock);
    return blocks < cap ? blocks : cap;
}

template <typename TO, typename TP>
hs_status launch(hipStream_t st, const void* patches, const float* pbias, const float* pos,
                 const void* cam, const void* reg, void* out, int s, int np, int nr, int d,
                 int n_var) {
    const int seq = 1 + nr + np;
    const int64_t out_rows = static_cast<int64_t>(s) * seq;
    const dim3 grid(static_cast<uint32_t>(persistent_blocks(out_rows)));
    const AssembleGrid ag = AssembleGrid::make(s, np, nr, d / 256 >= HS_AS_SPLIT ? HS_AS_SPLIT : 1);
    const auto* P = static_cast<const TP*>(patches);
    const auto* C = static_cast<const TO*>(cam);
    const auto* R = static_cast<const TO*>(reg);
    auto* O = static_cast<TO*>(out);
    // The dispatch packet counts work-items in 32 bits: one wave per row
    // caps the non-persistent grid, beyond which the persistent kernel runs.
    const int64_t vblocks = ag.patch_blocks + ag.special_blocks;
    const bool vec_ok = d % 256 == 0 && vblocks * kBlock < (int64_t{1} << 32) &&
                        aligned16(patches) && aligned16(out) && aligned16(cam) &&
                        (nr == 0 || aligned16(reg)) && (!pbias || aligned16(pbias)) &&
                        (!pos || aligned16(pos));
    const dim3 vgrid(static_cast<uint32_t>(vblocks));
    if (vec_ok) {
#define HS_AS_LAUNCH(CH, LV, SPL)                                                                  \
    assemble_kernel<TO, TP, CH, LV, SPL><<<vgrid, dim3(kBlock), 0, st>>>(P, pbias, pos, C, R, O, s, \
                                                                        seq, np, nr, n_var);      \
    return check_launch("assemble_tokens")
        constexpr int kS = HS_AS_SPLIT;
        switch (d / 256) {
            case 1: HS_AS_LAUNCH(1, 4, 1);
            case 2: HS_AS_LAUNCH(2, 4, (2 >= kS ? kS : 1));
            case 4: HS_AS_LAUNCH(4, 4, (4 >= kS ? kS : 1));
            case 8: HS_AS_LAUNCH(8, 4, (8 >= kS ? kS : 1));
            default: break;
        }
#undef HS_AS_LAUNCH
    }
    assemble_generic_kernel<TO, TP><<<grid, dim3(kBlock), 0, st>>>(P, pbias, pos, C, R, O, out_rows,
                                                                   seq, np, nr, d, n_var);
    return check_launch("assemble_tokens");
}

}  // namespace
}  // namespace hs

extern "C" hs_status hs_assemble_tokens(hs_stream_t stream, hs_dtype out_dt, const void* patches,
                                        hs_dtype patch_dt, const float* patch_bias,
                                        const float* pos, const void* cam, const void* reg,
                                        void* out, int32_t s, int32_t p, int32_t r, int32_t d,
                                        int32_t n_var) {
    using namespace hs;
    if (!valid_dtype(out_dt) || !valid_dtype(patch_dt))
        return fail(HS_EINVAL, "assemble_tokens: unknown dtype");
    if (s < 0 || p < 0 || r < 0 || d <= 0)
        return fail(HS_EINVAL, "assemble_tokens: shape S=%d P=%d R=%d D=%d", s, p, r, d);
    if (n_var != 1 && n_var != 2) return fail(HS_EINVAL, "assemble_tokens: n_var must be 1 or 2");
    const int64_t seq = int64_t{1} + r + p;
    const int64_t out_rows = static_cast<int64_t>(s) * seq;
    if (out_rows >= (int64_t{1} << 31) || seq >= (int64_t{1} << 31))
        return fail(HS_EINVAL, "assemble_tokens: S*T must be below 2^31");
    if (s == 0) return HS_OK;
    if (!out || !cam || (r > 0 && !reg) || (p > 0 && !patches))
        return fail(HS_EINVAL, "assemble_tokens: null buffer");
    const int64_t out_bytes = out_rows * d * dtype_size(out_dt);
    if (overlaps(out, out_bytes, patches, static_cast<int64_t>(s) * p * d * dtype_size(patch_dt)) ||
        overlaps(out, out_bytes, cam, n_var * d * dtype_size(out_dt)) ||
        overlaps(out, out_bytes, reg, static_cast<int64_t>(n_var) * r * d * dtype_size(out_dt)))
        return fail(HS_EINVAL, "assemble_tokens: out overlaps an input");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (out_dt == HS_F16)
        return patch_dt == HS_F32
                   ? launch<f16, float>(st, patches, patch_bias, pos, cam, reg, out, s, p, r, d, n_var)
                   : launch<f16, f16>(st, patches, patch_bias, pos, cam, reg, out, s, p, r, d, n_var);
    return patch_dt == HS_F32
               ? launch<float, float>(st, patches, patch_bias, pos, cam, reg, out, s, p, r, d, n_var)
               : launch<float, f16>(st, patches, patch_bias, pos, cam, reg, out, s, p, r, d, n_var);
}
