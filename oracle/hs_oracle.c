/*
 * hs_oracle.c — TEST INFRASTRUCTURE ONLY: the CPU restatement of headshot's
 * per-layer kernels that the HIP library is checked against. Built with
 * `-O2 -ffp-contract=off` (oracle/Makefile) so every f32 expression rounds
 * exactly as written, in the reference's operand order. Never linked into
 * the product library.
 *
 * Each function cites the reference file:line it restates; paths are under
 * crates/headshot-server/ unless noted.
 */
#include "hs_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* binary16 conversion (IEEE round-to-nearest-even, as half 2.7.1's
 * f16::from_f32 used by engine/tensor.rs:71-91 and the WGSL f16() cast).    */

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan: keep a quiet nan payload */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {
        /* |f| < 2^-14: binary16 subnormal (or zero). Scale by 2^24 (exact)
         * and round to an integer with ties-to-even. */
        float v = fabsf(f) * 16777216.0f;
        return (uint16_t)(sign | (uint32_t)nearbyintf(v));
    }
    uint32_t mant = ax & 0x7fffffu;
    uint32_t exp = (ax >> 23) - 127u + 15u;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: mant * 2^-24, exact in f32 */
            float v = (float)mant * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15u + 127u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void or_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = or_f32_to_f16(in[i]);
}

void or_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = or_f16_to_f32(in[i]);
}

/* Storage access: the WGSL `f32(x[i])` load and `Elem(v)` store. */
static inline float ld(int dt, const void* p, int64_t i) {
    if (dt == OR_F16) return or_f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static inline void st(int dt, void* p, int64_t i, float v) {
    if (dt == OR_F16)
        ((uint16_t*)p)[i] = or_f32_to_f16(v);
    else
        ((float*)p)[i] = v;
}

/* Round-trip through storage: the value a later dispatch reads back. */
static inline float rnd(int dt, float v) {
    return dt == OR_F16 ? or_f16_to_f32(or_f32_to_f16(v)) : v;
}

/* ------------------------------------------------------------------------ */
/* RoPE tables (engine/rope.rs)                                              */

/* engine/rope.rs:8-10: periods[i] = 100^(2i/32), evaluated in f32. */
void or_rope_periods(float out16[16]) {
    for (int i = 0; i < 16; i++) {
        float e = 2.0f * (float)i;
        e = e / 32.0f;
        out16[i] = powf(100.0f, e);
    }
}

/* engine/rope.rs:18-43. Channels [0,16) h-angles, [16,32) w-angles, [32,64)
 * a copy of [0,32). coord(i) = 2*((i+0.5)/max(h_p,w_p)) - 1;
 * angle = (TAU * coord) / period, all in f32 and in that order. */
void or_rope_tables(const float* periods16, int32_t h_p, int32_t w_p, float* sin_out,
                    float* cos_out) {
    const float side = (float)(h_p > w_p ? h_p : w_p);
    const float tau = 6.28318530717958647692f; /* std::f32::consts::TAU */
    for (int32_t row = 0; row < h_p; row++) {
        for (int32_t col = 0; col < w_p; col++) {
            int64_t idx = ((int64_t)row * w_p + col) * 64;
            float ch = ((float)row + 0.5f) / side;
            ch = 2.0f * ch;
            ch = ch - 1.0f;
            float cw = ((float)col + 0.5f) / side;
            cw = 2.0f * cw;
            cw = cw - 1.0f;
            for (int i = 0; i < 16; i++) {
                float ah = tau * ch;
                ah = ah / periods16[i];
                float aw = tau * cw;
                aw = aw / periods16[i];
                float sh = sinf(ah), chh = cosf(ah);
                float sw = sinf(aw), cww = cosf(aw);
                for (int half = 0; half <= 32; half += 32) {
                    sin_out[idx + half + 0 + i] = sh;
                    cos_out[idx + half + 0 + i] = chh;
                    sin_out[idx + half + 16 + i] = sw;
                    cos_out[idx + half + 16 + i] = cww;
                }
            }
        }
    }
}

/* engine/rope.rs:47-54: x' = x*cos + rot(x)*sin, rot(x) = concat(-x[32:], x[:32]). */
void or_rope_apply_cpu(const float* x, const float* sin_tab, const float* cos_tab,
                       int64_t table_row, float* out) {
    const float* s = sin_tab + table_row * 64;
    const float* c = cos_tab + table_row * 64;
    for (int i = 0; i < 64; i++) {
        float rot = i < 32 ? -x[i + 32] : x[i - 32];
        float a = x[i] * c[i];
        float b = rot * s[i];
        out[i] = a + b;
    }
}

/* ------------------------------------------------------------------------ */
/* LayerNorm (shaders/layernorm.wesl:27-78)                                  */

/* One row, f32 in/out; the WGSL's 256-lane strided partial sums followed by
 * its 8-level shared-memory tree, for the mean and then the variance. */
static void ln_row(const float* xr, int32_t dim, const float* w, const float* b, float eps,
                   float* out) {
    float scratch[256];
    for (int li = 0; li < 256; li++) {
        float partial = 0.0f;
        for (int j = li; j < dim; j += 256) partial += xr[j];
        scratch[li] = partial;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int li = 0; li < s; li++) scratch[li] += scratch[li + s];
    const float mu = scratch[0] / (float)dim;

    for (int li = 0; li < 256; li++) {
        float partial = 0.0f;
        for (int j = li; j < dim; j += 256) {
            float d = xr[j] - mu;
            float dd = d * d;
            partial += dd;
        }
        scratch[li] = partial;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int li = 0; li < s; li++) scratch[li] += scratch[li + s];
    float var = scratch[0] / (float)dim;
    var = var + eps;
    const float inv_sigma = 1.0f / sqrtf(var); /* WGSL inverseSqrt */

    for (int j = 0; j < dim; j++) {
        float v = xr[j] - mu;
        v = v * inv_sigma;
        v = v * w[j];
        out[j] = v + b[j];
    }
}

void or_layernorm(int dt, const void* x, const float* w, const float* b, void* out,
                  int64_t rows, int32_t dim, float eps) {
#pragma omp parallel
    {
        float* xr = (float*)malloc(sizeof(float) * (size_t)dim * 2);
        float* yr = xr + dim;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            int64_t base = r * dim;
            for (int j = 0; j < dim; j++) xr[j] = ld(dt, x, base + j);
            ln_row(xr, dim, w, b, eps, yr);
            for (int j = 0; j < dim; j++) st(dt, out, base + j, yr[j]);
        }
        free(xr);
    }
}

/* ------------------------------------------------------------------------ */
/* Head split / merge (shaders/split_heads.wesl:22-42, attn_merge.wesl)      */

void or_split_heads(int dt, const void* x, void* out, int32_t s, int32_t t, int32_t h,
                    int32_t d) {
    const int64_t hd = (int64_t)h * d;
#pragma omp parallel for collapse(2) schedule(static)
    for (int32_t si = 0; si < s; si++)
        for (int32_t hi = 0; hi < h; hi++)
            for (int32_t ti = 0; ti < t; ti++)
                for (int32_t di = 0; di < d; di++) {
                    int64_t o = (((int64_t)si * h + hi) * t + ti) * d + di;
                    int64_t i = ((int64_t)si * t + ti) * hd + (int64_t)hi * d + di;
                    if (dt == OR_F16)
                        ((uint16_t*)out)[o] = ((const uint16_t*)x)[i];
                    else
                        ((float*)out)[o] = ((const float*)x)[i];
                }
}

void or_attn_merge(int dt, const void* x, void* out, int32_t s, int32_t t, int32_t h,
                   int32_t d) {
    const int64_t hd = (int64_t)h * d;
#pragma omp parallel for collapse(2) schedule(static)
    for (int32_t si = 0; si < s; si++)
        for (int32_t hi = 0; hi < h; hi++)
            for (int32_t ti = 0; ti < t; ti++)
                for (int32_t di = 0; di < d; di++) {
                    int64_t i = (((int64_t)si * h + hi) * t + ti) * d + di;
                    int64_t o = ((int64_t)si * t + ti) * hd + (int64_t)hi * d + di;
                    if (dt == OR_F16)
                        ((uint16_t*)out)[o] = ((const uint16_t*)x)[i];
                    else
                        ((float*)out)[o] = ((const float*)x)[i];
                }
}

/* ------------------------------------------------------------------------ */
/* Linear (shaders/linear.wesl:29-68, the scalar path of engine/ops.rs:81-128) */

/* out (rows, n) = x (m, k) @ w (n, k)^T [+ bias]: f32 accumulation in k
 * order, bias added after the sum, stored as Elem. Only the rows listed in
 * rows_idx (nrows of them; NULL = all m in order) are computed, into
 * consecutive rows of out. */
void or_linear(int dt, const void* x, const void* w, const float* bias, void* out, int64_t m,
               int32_t n, int32_t k, const int64_t* rows_idx, int64_t nrows) {
    if (!rows_idx) nrows = m;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t j = 0; j < nrows; j++) {
        const int64_t row = rows_idx ? rows_idx[j] : j;
        for (int32_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (int32_t kk = 0; kk < k; kk++)
                acc += ld(dt, x, row * k + kk) * ld(dt, w, (int64_t)col * k + kk);
            if (bias) acc += bias[col];
            st(dt, out, j * n + col, acc);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Cache build (shaders/concat_channels.wesl, shaders/cast_f16_to_f32.wesl,
 * composed as model/cache.rs:37-44)                                        */

/* One output element per index, as the shader's thread: c = i % (c1 + c2),
 * row = i / (c1 + c2), from a or b. */
void or_concat_channels(int dt, const void* a, const void* b, void* out, int64_t rows,
                        int32_t c1, int32_t c2) {
    const int64_t c_out = (int64_t)c1 + c2;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows * c_out; i++) {
        const int64_t c = i % c_out, row = i / c_out;
        if (dt == OR_F16)
            ((uint16_t*)out)[i] = c < c1 ? ((const uint16_t*)a)[row * c1 + c]
                                         : ((const uint16_t*)b)[row * c2 + (c - c1)];
        else
            ((float*)out)[i] = c < c1 ? ((const float*)a)[row * c1 + c]
                                      : ((const float*)b)[row * c2 + (c - c1)];
    }
}

/* out[i] = f32(x[i]) */
void or_cast_f16_to_f32(const uint16_t* x, float* out, int64_t total) {
    or_f16_to_f32_array(x, out, total);
}

/* Cache::build for one row range: concat_channels, then cast_to_f32 when the
 * inputs are f16 (an f32 concatenation is stored as is). */
void or_cache_build(int dt, const void* frame_out, const void* inter_out, float* out,
                    int64_t rows, int32_t c1, int32_t c2) {
    const int64_t n = rows * ((int64_t)c1 + c2);
    if (dt == OR_F32) {
        or_concat_channels(OR_F32, frame_out, inter_out, out, rows, c1, c2);
        return;
    }
    uint16_t* cat = (uint16_t*)malloc((size_t)n * sizeof(uint16_t));
    if (!cat) return;
    or_concat_channels(OR_F16, frame_out, inter_out, cat, rows, c1, c2);
    or_cast_f16_to_f32(cat, out, n);
    free(cat);
}

/* ------------------------------------------------------------------------ */
/* Attention (shaders/attention.wesl:36-88, dispatched by engine/ops.rs:228-253) */

/* One query of one (frame, head) sequence at a time, exactly as the shader's
 * thread does: q in f32, per key a vec4-lane dot product summed x+y+z+w and
 * scaled, then the online softmax update (running max m, denominator l,
 * f32 accumulator), and finally acc / l stored as Elem. Queries listed in
 * q_idx (nq of them; q_idx NULL = all t in order) are computed for every
 * sequence; out is (S*H, nq, D). */
void or_attention(int dt, const void* q, const void* k, const void* v, void* out, int32_t s,
                  int32_t h, int32_t t, int32_t d, const int32_t* q_idx, int32_t nq) {
    const float scale = 1.0f / sqrtf((float)d); /* engine/ops.rs:242 */
    const int64_t nseq = (int64_t)s * h;
    if (!q_idx) nq = t;
    if (d > 128 || d % 4) return;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int64_t sh = 0; sh < nseq; sh++)
        for (int32_t j = 0; j < nq; j++) {
            const int64_t base = sh * t * d;
            const int32_t qi = q_idx ? q_idx[j] : j;
            float qv[128], acc[128];
            for (int32_t dd = 0; dd < d; dd++) {
                qv[dd] = ld(dt, q, base + (int64_t)qi * d + dd);
                acc[dd] = 0.0f;
            }
            float m = -3.4e38f, l = 0.0f;
            for (int32_t kk = 0; kk < t; kk++) {
                const int64_t kb = base + (int64_t)kk * d;
                float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int32_t dd = 0; dd < d; dd += 4)
                    for (int e = 0; e < 4; e++) s4[e] += qv[dd + e] * ld(dt, k, kb + dd + e);
                const float score = (s4[0] + s4[1] + s4[2] + s4[3]) * scale;
                const float m_new = fmaxf(m, score);
                const float corr = expf(m - m_new);
                const float e = expf(score - m_new);
                l = l * corr + e;
                for (int32_t dd = 0; dd < d; dd++)
                    acc[dd] = acc[dd] * corr + e * ld(dt, v, kb + dd);
                m = m_new;
            }
            const float inv_l = 1.0f / l;
            const int64_t o = (sh * nq + j) * d;
            for (int32_t dd = 0; dd < d; dd++) st(dt, out, o + dd, acc[dd] * inv_l);
        }
}

/* ------------------------------------------------------------------------ */
/* RoPE apply (shaders/rope_apply.wesl:30-57)                                */

/* One head vector in f32: pairs (dp, dp+half); table row (t - prefix). */
static void rope_vec(float* v, const float* sin_tab, const float* cos_tab, int64_t trow,
                     int32_t d) {
    const int32_t half = d / 2;
    const int64_t row = trow * d;
    for (int32_t dp = 0; dp < half; dp++) {
        float lo = v[dp], hi = v[dp + half];
        float a = lo * cos_tab[row + dp];
        float b = hi * sin_tab[row + dp];
        float c = hi * cos_tab[row + half + dp];
        float e = lo * sin_tab[row + half + dp];
        v[dp] = a - b;
        v[dp + half] = c + e;
    }
}

void or_rope_apply(int dt, void* x, const float* sin_tab, const float* cos_tab, int32_t s,
                   int32_t h, int32_t t, int32_t d, int32_t prefix) {
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for collapse(2) schedule(static)
        for (int32_t si = 0; si < s; si++)
            for (int32_t hi = 0; hi < h; hi++)
                for (int32_t ti = prefix; ti < t; ti++) {
                    int64_t base = (((int64_t)si * h + hi) * t + ti) * d;
                    for (int j = 0; j < d; j++) v[j] = ld(dt, x, base + j);
                    rope_vec(v, sin_tab, cos_tab, ti - prefix, d);
                    for (int j = 0; j < d; j++) st(dt, x, base + j, v[j]);
                }
        free(v);
    }
}

/* ------------------------------------------------------------------------ */
/* GELU (shaders/gelu.wesl)                                                  */

/* Abramowitz & Stegun 7.1.26, gelu.wesl:18-27, in the shader's operand order. */
float or_erf_as(float v) {
    float s = v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
    float a = fabsf(v);
    float t = 0.3275911f * a;
    t = 1.0f + t;
    t = 1.0f / t;
    float p = 1.061405429f * t;
    p = p - 1.453152027f;
    p = p * t;
    p = p + 1.421413741f;
    p = p * t;
    p = p - 0.284496736f;
    p = p * t;
    p = p + 0.254829592f;
    p = p * t;
    float na = -a;
    float e = na * a;
    e = expf(e);
    p = p * e;
    float y = 1.0f - p;
    return s * y;
}

/* gelu.wesl:36-38: 0.5*v*(1 + erf(v*0.70710678)) */
static inline float gelu_f(float v) {
    float z = v * 0.7071067811865475f;
    float e = or_erf_as(z);
    float h = 0.5f * v;
    float one = 1.0f + e;
    return h * one;
}

void or_gelu(int dt, const void* x, void* out, int64_t total) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++) st(dt, out, i, gelu_f(ld(dt, x, i)));
}

/* ------------------------------------------------------------------------ */
/* Residual + LayerScale, bias epilogue, casts, tiled add                    */

/* residual_ls.wesl:28: out = res + gamma[i % dim] * x */
static inline float ls_f(float res, float x, float g) {
    float m = g * x;
    return res + m;
}

void or_residual_ls(int dt, const void* res, const void* x, const float* gamma, void* out,
                    int64_t total, int32_t dim) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++)
        st(dt, out, i, ls_f(ld(dt, res, i), ld(dt, x, i), gamma[i % dim]));
}

/* linear_wmma.wgsl:69-74 / linear.wesl:57-61: Elem(acc + bias[col]). */
void or_add_bias(int dt, const void* x, const float* bias, void* out, int64_t rows,
                 int32_t cols) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int32_t c = 0; c < cols; c++) {
            int64_t i = r * cols + c;
            st(dt, out, i, ld(dt, x, i) + bias[c]);
        }
}

void or_cast_f32_to_f16(const float* x, uint16_t* out, int64_t total) {
    or_f32_to_f16_array(x, out, total);
}

void or_tiled_add(const float* x, const float* table, float* out, int64_t total,
                  int64_t block) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++) out[i] = x[i] + table[i % block];
}

/* ------------------------------------------------------------------------ */
/* Composites: the reference's unfused dispatch sequences                    */

void or_qknorm_rope(int dt, const void* x_tok, const float* nw, const float* nb,
                    const float* sin_tab, const float* cos_tab, void* out_head, int32_t s,
                    int32_t t, int32_t h, int32_t d, int32_t prefix, float eps) {
    const int64_t hd = (int64_t)h * d;
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)d * 2);
        float* y = v + d;
#pragma omp for collapse(2) schedule(static)
        for (int32_t si = 0; si < s; si++)
            for (int32_t hi = 0; hi < h; hi++)
                for (int32_t ti = 0; ti < t; ti++) {
                    /* split_heads: an exact copy into head-major storage */
                    int64_t src = ((int64_t)si * t + ti) * hd + (int64_t)hi * d;
                    for (int j = 0; j < d; j++) v[j] = ld(dt, x_tok, src + j);
                    /* QK-norm: layernorm over d, stored (block.rs:136-142) */
                    if (nw) {
                        ln_row(v, d, nw, nb, eps, y);
                        for (int j = 0; j < d; j++) v[j] = rnd(dt, y[j]);
                    }
                    /* rope_apply in place, stored (block.rs:143-146) */
                    if (sin_tab && ti >= prefix) {
                        rope_vec(v, sin_tab, cos_tab, ti - prefix, d);
                        for (int j = 0; j < d; j++) v[j] = rnd(dt, v[j]);
                    }
                    int64_t dst = (((int64_t)si * h + hi) * t + ti) * d;
                    for (int j = 0; j < d; j++) st(dt, out_head, dst + j, v[j]);
                }
        free(v);
    }
}

void or_bias_gelu(int dt, const void* x, const float* bias, void* out, int64_t rows,
                  int32_t cols, int round_bias) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int32_t c = 0; c < cols; c++) {
            int64_t i = r * cols + c;
            float v = ld(dt, x, i);
            if (bias) {
                v = v + bias[c];
                if (round_bias) v = rnd(dt, v);
            }
            st(dt, out, i, gelu_f(v));
        }
}

void or_bias_ls_residual(int dt, const void* res, const void* x, const float* bias,
                         const float* gamma, void* out, int64_t rows, int32_t dim) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int32_t c = 0; c < dim; c++) {
            int64_t i = r * dim + c;
            float v = ld(dt, x, i);
            if (bias) v = rnd(dt, v + bias[c]);
            st(dt, out, i, ls_f(ld(dt, res, i), v, gamma[c]));
        }
}

void or_assemble_tokens(int out_dt, const void* patches, int patch_dt, const float* patch_bias,
                        const float* pos, const void* cam, const void* reg, void* out, int32_t s,
                        int32_t p, int32_t r, int32_t d, int32_t n_var) {
    const int64_t t = (int64_t)p + 1 + r;
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < (int64_t)s * t; row++) {
        int64_t si = row / t, ti = row % t;
        int64_t v = (n_var == 2 && si != 0) ? 1 : 0;
        int64_t o = row * d;
        if (ti == 0) { /* camera token variant v: copy_rows (trunk.rs:82) */
            for (int j = 0; j < d; j++) st(out_dt, out, o + j, ld(out_dt, cam, v * d + j));
        } else if (ti <= r) { /* register tokens: copy_rows (trunk.rs:83) */
            int64_t src = (v * r + (ti - 1)) * d;
            for (int j = 0; j < d; j++) st(out_dt, out, o + j, ld(out_dt, reg, src + j));
        } else { /* patch rows: epilogue bias, pos add, cast, copy */
            int64_t pi = ti - 1 - r;
            int64_t src = (si * p + pi) * d;
            for (int j = 0; j < d; j++) {
                float val = ld(patch_dt, patches, src + j);
                if (patch_bias) val = rnd(patch_dt, val + patch_bias[j]);
                if (pos) val = rnd(patch_dt, val + pos[pi * d + j]);
                st(out_dt, out, o + j, val);
            }
        }
    }
}

void or_block_ops(int dt, const void* x, const float* ln1_w, const float* ln1_b,
                  const void* q_raw, const void* k_raw, const float* qn_w, const float* qn_b,
                  const float* kn_w, const float* kn_b, const float* sin_tab,
                  const float* cos_tab, int32_t prefix, const void* proj_raw,
                  const float* proj_b, const float* ls1, const float* ln2_w, const float* ln2_b,
                  const void* fc1_raw,
                  const float* fc1_b, const void* fc2_raw, const float* fc2_b,
                  const float* ls2, void* normed, void* q_head, void* k_head, void* x1,
                  void* normed2, void* act, void* x_out, int32_t s, int32_t t, int32_t dim,
                  int32_t heads, int32_t hidden, float eps) {
    const int64_t rows = (int64_t)s * t;
    const int32_t hd = dim / heads;
    or_layernorm(dt, x, ln1_w, ln1_b, normed, rows, dim, eps);
    or_qknorm_rope(dt, q_raw, qn_w, qn_b, sin_tab, cos_tab, q_head, s, t, heads, hd, prefix, eps);
    or_qknorm_rope(dt, k_raw, kn_w, kn_b, sin_tab, cos_tab, k_head, s, t, heads, hd, prefix, eps);
    or_bias_ls_residual(dt, x, proj_raw, proj_b, ls1, x1, rows, dim);
    or_layernorm(dt, x1, ln2_w, ln2_b, normed2, rows, dim, eps);
    or_bias_gelu(dt, fc1_raw, fc1_b, act, rows, hidden, 1);
    or_bias_ls_residual(dt, x1, fc2_raw, fc2_b, ls2, x_out, rows, dim);
}

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void or_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
