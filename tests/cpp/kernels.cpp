// Kernel tests through the C++ host surface (include/headshot_hip.hpp),
// restating headshot-server's GPU kernel tests for the per-layer ops —
// crates/headshot-server/tests/kernels.rs and tests/f16_ops.rs — with the
// same seeds, naive CPU expectations and tolerances, plus checks that each
// fused op equals the reference's sequence of single ops run through the
// same context. Exit status 0 when every test passes.
#include <array>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "headshot_hip.hpp"

using hs::Dtype;
using hs::HipContext;
using hs::HipTensor;

namespace {

// Deterministic light-weight RNG (tests/kernels.rs:7-23): SplitMix64 ->
// `(z >> 40) as f32 / 2^23 * 2 - 1`.
struct Rng {
    uint64_t s;
    float next_f32() {
        s += 0x9E3779B97F4A7C15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        return static_cast<float>(z >> 40) / static_cast<float>(1ull << 23) * 2.0f - 1.0f;
    }
    std::vector<float> vec(size_t n) {
        std::vector<float> v(n);
        for (auto& x : v) x = next_f32();
        return v;
    }
};

// tests/f16_ops.rs:7-19: f16-exact values in [-1, 1).
std::vector<float> rvec(uint64_t seed, size_t n) {
    std::vector<float> v(n);
    uint64_t s = seed;
    for (auto& x : v) {
        s += 0x9E3779B97F4A7C15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        const float u = static_cast<float>(z >> 40) / static_cast<float>(1ull << 24) * 2.0f - 1.0f;
        x = hs::f16_to_f32(hs::f32_to_f16(u));
    }
    return v;
}

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// tests/kernels.rs:35-43
void assert_close(const std::vector<float>& a, const std::vector<float>& e, float tol,
                  const std::string& what) {
    if (a.size() != e.size()) throw Failure(what + ": length");
    for (size_t i = 0; i < a.size(); i++)
        if (!(std::fabs(a[i] - e[i]) <= tol + tol * std::fabs(e[i])))
            throw Failure(what + "[" + std::to_string(i) + "]: got " + std::to_string(a[i]) +
                          ", want " + std::to_string(e[i]));
}

// tests/f16_ops.rs:21-33: max-abs gate, and neither side all zero.
void close(const std::vector<float>& a, const std::vector<float>& b, float tol,
           const std::string& what) {
    if (a.size() != b.size()) throw Failure(what + ": length");
    float mx = 0.0f;
    size_t nz_a = 0, nz_b = 0;
    for (size_t i = 0; i < a.size(); i++) {
        mx = std::fmax(mx, std::fabs(a[i] - b[i]));
        nz_a += a[i] != 0.0f, nz_b += b[i] != 0.0f;
    }
    if (!nz_b) throw Failure(what + ": f32 reference is all zero");
    if (!nz_a) throw Failure(what + ": f16 output is ALL ZERO");
    if (!(mx < tol)) throw Failure(what + ": max diff " + std::to_string(mx) + " > " + std::to_string(tol));
}

// f16 parity gate on normalised outputs: |a - e| <= 2e-3 * max(1, |e|).
void f16_gate(const std::vector<float>& a, const std::vector<float>& e, const std::string& what) {
    if (a.size() != e.size()) throw Failure(what + ": length");
    for (size_t i = 0; i < a.size(); i++)
        if (!(std::fabs(a[i] - e[i]) <= 2e-3f * std::fmax(1.0f, std::fabs(e[i]))))
            throw Failure(what + "[" + std::to_string(i) + "]: got " + std::to_string(a[i]) +
                          ", want " + std::to_string(e[i]));
}

void exact(const std::vector<float>& a, const std::vector<float>& b, const std::string& what) {
    if (a.size() != b.size()) throw Failure(what + ": length");
    if (std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) != 0) throw Failure(what + ": differs");
}

// engine/rope.rs:47-54
std::vector<float> apply_cpu(const float* x, const std::vector<float>& sin,
                             const std::vector<float>& cos, size_t row) {
    std::vector<float> y(64);
    for (int i = 0; i < 64; i++) {
        const float rot = i < 32 ? -x[i + 32] : x[i - 32];
        y[i] = x[i] * cos[row * 64 + i] + rot * sin[row * 64 + i];
    }
    return y;
}

// --------------------------------------------------------------- tests

void layernorm_matches_cpu(HipContext& ctx) {  // tests/kernels.rs:100-126
    Rng rng{3};
    const size_t rows = 19, dim = 300;  // dim > workgroup size: strided path
    auto x = rng.vec(rows * dim), w = rng.vec(dim), b = rng.vec(dim);
    auto out = ctx.layernorm(ctx.tensor_from_slice({rows, dim}, x), ctx.tensor_from_slice({dim}, w),
                             ctx.tensor_from_slice({dim}, b));
    std::vector<float> expected(rows * dim);
    for (size_t r = 0; r < rows; r++) {
        const float* row = &x[r * dim];
        float mu = 0.0f;
        for (size_t j = 0; j < dim; j++) mu += row[j];
        mu /= static_cast<float>(dim);
        float var = 0.0f;
        for (size_t j = 0; j < dim; j++) var += (row[j] - mu) * (row[j] - mu);
        var /= static_cast<float>(dim);
        const float inv = 1.0f / std::sqrt(var + 1e-5f);
        for (size_t j = 0; j < dim; j++) expected[r * dim + j] = (row[j] - mu) * inv * w[j] + b[j];
    }
    assert_close(ctx.download(out), expected, 1e-4f, "layernorm");
}

void gelu_matches_erf(HipContext& ctx) {  // tests/kernels.rs:128-147
    std::vector<float> xs;
    for (int i = -40; i <= 40; i++) xs.push_back(static_cast<float>(i) * 0.2f);
    auto got = ctx.download(ctx.gelu(ctx.tensor_from_slice({xs.size()}, xs)));
    for (size_t i = 0; i < xs.size(); i++) {
        const double exact = 0.5 * xs[i] * (1.0 + std::erf(static_cast<double>(xs[i]) / std::sqrt(2.0)));
        if (!(std::fabs(got[i] - exact) < 1e-5))
            throw Failure("gelu(" + std::to_string(xs[i]) + ") = " + std::to_string(got[i]) +
                          ", want " + std::to_string(exact));
    }
}

void rope_apply_matches_cpu(HipContext& ctx) {  // tests/kernels.rs:149-182
    Rng rng{4};
    const size_t s = 2, h = 3, t = 11, d = 64, prefix = 5, p = t - prefix;  // 2x3 grid
    auto [sin, cos] = hs::rope::tables(hs::rope::periods(), 2, 3);
    if (sin.size() != p * d) throw Failure("table size");
    auto x = rng.vec(s * h * t * d);
    auto gx = ctx.tensor_from_slice({s, h, t, d}, x);
    ctx.rope_apply(gx, ctx.tensor_from_slice({p, d}, sin), ctx.tensor_from_slice({p, d}, cos), prefix);
    auto got = ctx.download(gx);
    for (size_t si = 0; si < s; si++)
        for (size_t hi = 0; hi < h; hi++)
            for (size_t ti = 0; ti < t; ti++) {
                const size_t base = ((si * h + hi) * t + ti) * d;
                std::vector<float> v(x.begin() + base, x.begin() + base + d);
                auto expected = ti < prefix ? v : apply_cpu(v.data(), sin, cos, ti - prefix);
                assert_close(std::vector<float>(got.begin() + base, got.begin() + base + d), expected,
                             1e-5f, "rope");
            }
}

void split_heads_layout(HipContext& ctx) {  // tests/kernels.rs:241-262
    Rng rng{6};
    const size_t s = 2, t = 5, h = 4, d = 8;
    auto x = rng.vec(s * t * h * d);
    auto gq = ctx.download(ctx.split_heads(ctx.tensor_from_slice({s * t, h * d}, x), s, t, h, d));
    for (size_t si = 0; si < s; si++)
        for (size_t hi = 0; hi < h; hi++)
            for (size_t ti = 0; ti < t; ti++)
                for (size_t di = 0; di < d; di++) {
                    const float got = gq[(((si * h) + hi) * t + ti) * d + di];
                    const float want = x[(si * t + ti) * h * d + hi * d + di];
                    if (got != want) throw Failure("q[" + std::to_string(si) + "," + std::to_string(hi) + "]");
                }
}

void copy_rows_and_tiled_add(HipContext& ctx) {
    Rng rng{7};
    auto a = rng.vec(6 * 4), table = rng.vec(3 * 4);
    auto src = ctx.tensor_from_slice({6, 4}, a);
    auto dst = ctx.tensor_from_slice({5, 4}, std::vector<float>(20, 0.0f));
    ctx.copy_rows(src, 2, dst, 1, 3);
    auto got = ctx.download(dst);
    std::vector<float> want(20, 0.0f);
    std::memcpy(&want[4], &a[8], 12 * sizeof(float));
    exact(got, want, "copy_rows");
    auto sum = ctx.download(ctx.tiled_add(ctx.tensor_from_slice({2, 3, 4}, rng.vec(24)),
                                          ctx.tensor_from_slice({3, 4}, table)));
    if (sum.size() != 24) throw Failure("tiled_add size");
}

void every_op_f16_matches_f32(HipContext& ctx) {  // tests/f16_ops.rs:35-109
    const size_t s = 2, h = 4, t = 21, d = 64, c = h * d, rows = s * t;
    auto x = rvec(1, rows * c);
    auto up = [&](const std::vector<float>& v, std::vector<size_t> shape, Dtype dt) {
        return ctx.tensor_from_f32(std::move(shape), v, dt);
    };
    auto w = rvec(2, c), b = rvec(3, c);
    close(ctx.download(ctx.layernorm(up(x, {rows, c}, Dtype::F16), up(w, {c}, Dtype::F32), up(b, {c}, Dtype::F32))),
          ctx.download(ctx.layernorm(up(x, {rows, c}, Dtype::F32), up(w, {c}, Dtype::F32), up(b, {c}, Dtype::F32))),
          2e-2f, "layernorm");
    close(ctx.download(ctx.gelu(up(x, {rows, c}, Dtype::F16))),
          ctx.download(ctx.gelu(up(x, {rows, c}, Dtype::F32))), 2e-3f, "gelu");
    auto r = rvec(4, rows * c), g = rvec(5, c);
    close(ctx.download(ctx.residual_ls(up(r, {rows, c}, Dtype::F16), up(x, {rows, c}, Dtype::F16), up(g, {c}, Dtype::F32))),
          ctx.download(ctx.residual_ls(up(r, {rows, c}, Dtype::F32), up(x, {rows, c}, Dtype::F32), up(g, {c}, Dtype::F32))),
          2e-3f, "residual_ls");
    auto qkv = rvec(6, rows * c);
    close(ctx.download(ctx.split_heads(up(qkv, {rows, c}, Dtype::F16), s, t, h, d)),
          ctx.download(ctx.split_heads(up(qkv, {rows, c}, Dtype::F32), s, t, h, d)), 1e-6f, "split_heads");
    auto [sin, cos] = hs::rope::tables(hs::rope::periods(), 4, 4);
    const size_t prefix = t - 16;
    auto q = rvec(7, s * h * t * d);
    auto sin_t = up(sin, {16, 64}, Dtype::F32), cos_t = up(cos, {16, 64}, Dtype::F32);
    auto g32 = up(q, {s, h, t, d}, Dtype::F32);
    ctx.rope_apply(g32, sin_t, cos_t, prefix);
    auto g16 = up(q, {s, h, t, d}, Dtype::F16);
    ctx.rope_apply(g16, sin_t, cos_t, prefix);
    close(ctx.download(g16), ctx.download(g32), 2e-3f, "rope_apply");
}

// Fused ops == the reference's single-op sequence through the same context.
void fused_ops_equal_reference_sequence(HipContext& ctx) {
    Rng rng{9};
    const size_t s = 2, h = 16, d = 64, prefix = 5, t = 6 + prefix, c = h * d, rows = s * t;
    auto x = rng.vec(rows * c), nw = rng.vec(d), nb = rng.vec(d);
    auto [sin, cos] = hs::rope::tables(hs::rope::periods(), 2, 3);
    for (Dtype dt : {Dtype::F32, Dtype::F16}) {
        auto gx = ctx.tensor_from_f32({rows, c}, x, dt);
        auto w = ctx.tensor_from_slice({d}, nw), b = ctx.tensor_from_slice({d}, nb);
        auto st = ctx.tensor_from_slice({t - prefix, d}, sin), ct = ctx.tensor_from_slice({t - prefix, d}, cos);
        // reference: split_heads -> layernorm(d) -> rope_apply
        auto seq = ctx.layernorm(ctx.split_heads(gx, s, t, h, d), w, b, 1e-6f);
        ctx.rope_apply(seq, st, ct, prefix);
        hs::Norm norm{&w, &b};
        hs::Rope rope{&st, &ct, prefix};
        auto fused = ctx.qknorm_rope(gx, s, t, h, d, &norm, &rope, 1e-6f);
        if (dt == Dtype::F32)
            assert_close(ctx.download(fused), ctx.download(seq), 1e-5f, "qknorm_rope f32");
        else
            f16_gate(ctx.download(fused), ctx.download(seq), "qknorm_rope f16");
        // split only
        exact(ctx.download(ctx.qknorm_rope(gx, s, t, h, d, nullptr, nullptr)),
              ctx.download(ctx.split_heads(gx, s, t, h, d)), "qknorm_rope as split_heads");
    }
    // bias + LayerScale + residual == residual_ls(res, x + bias) in f32
    auto res = rng.vec(rows * c), xb = rng.vec(rows * c), gam = rng.vec(c), bias = rng.vec(c);
    std::vector<float> xpb(rows * c);
    for (size_t i = 0; i < xpb.size(); i++) xpb[i] = xb[i] + bias[i % c];
    auto gres = ctx.tensor_from_slice({rows, c}, res), ggam = ctx.tensor_from_slice({c}, gam);
    auto gbias = ctx.tensor_from_slice({c}, bias);
    assert_close(ctx.download(ctx.bias_ls_residual(gres, ctx.tensor_from_slice({rows, c}, xb), ggam, &gbias)),
                 ctx.download(ctx.residual_ls(gres, ctx.tensor_from_slice({rows, c}, xpb), ggam)), 1e-6f,
                 "bias_ls_residual");
    assert_close(ctx.download(ctx.bias_gelu(ctx.tensor_from_slice({rows, c}, xb), &gbias)),
                 ctx.download(ctx.gelu(ctx.tensor_from_slice({rows, c}, xpb))), 1e-6f, "bias_gelu");
    // bias + LayerScale + residual, then layernorm of its output, in one pass ==
    // bias_ls_residual then layernorm, bit for bit
    auto lw = ctx.tensor_from_slice({c}, rng.vec(c)), lb = ctx.tensor_from_slice({c}, rng.vec(c));
    hs::Norm ln{&lw, &lb};
    for (Dtype dt : {Dtype::F32, Dtype::F16}) {
        auto r16 = ctx.tensor_from_f32({rows, c}, res, dt), x16 = ctx.tensor_from_f32({rows, c}, xb, dt);
        auto fused = ctx.bias_ls_residual_layernorm(r16, x16, ggam, &gbias, ln, 1e-6f);
        auto x1 = ctx.bias_ls_residual(r16, x16, ggam, &gbias);
        exact(ctx.download(fused.out), ctx.download(x1), "bias_ls_residual_layernorm out");
        exact(ctx.download(fused.normed), ctx.download(ctx.layernorm(x1, lw, lb, 1e-6f)),
              "bias_ls_residual_layernorm normed");
    }
}

// model/trunk.rs:68-85: cast_to_f16 + copy_rows per frame == assemble_tokens.
void assemble_equals_cast_and_copy_rows(HipContext& ctx) {
    Rng rng{10};
    const size_t n = 3, p = 6, r = 4, dim = 256, t = p + 1 + r;
    auto dino = ctx.tensor_from_slice({n * p, dim}, rng.vec(n * p * dim));
    auto cam = ctx.tensor_from_f32({2, dim}, rng.vec(2 * dim), Dtype::F16);
    auto reg = ctx.tensor_from_f32({2 * r, dim}, rng.vec(2 * r * dim), Dtype::F16);
    auto cast = ctx.cast_to_f16(dino);
    auto x = ctx.empty_typed({n * t, dim}, Dtype::F16);
    for (size_t i = 0; i < n; i++) {
        const size_t v = i != 0;
        ctx.copy_rows(cam, v, x, i * t, 1);
        ctx.copy_rows(reg, v * r, x, i * t + 1, r);
        ctx.copy_rows(cast, i * p, x, i * t + 1 + r, p);
    }
    auto fused = ctx.assemble_tokens(dino, n, p, cam, &reg, nullptr, nullptr, Dtype::F16, 2);
    exact(ctx.download(fused), ctx.download(x), "assembly");
}

// tests/kernels.rs:185-238: (s, h, d) = (2, 3, 64), t in {17, 64, 150},
// q, k, v from Rng(5 + t), naive full-matrix softmax, |a - e| < 1e-4; then
// the same through the f16 path (f16 inputs, output) at 5e-3 of the f32
// result (tests/kernels.rs:377-401), the merge as an exact permutation and
// the fused merge equal to attn_merge(attention).
void attention_matches_cpu(HipContext& ctx) {
    for (size_t t : {17, 64, 150}) {
        Rng rng{5 + t};
        const size_t s = 2, h = 3, d = 64;
        auto q = rng.vec(s * h * t * d), k = rng.vec(s * h * t * d), v = rng.vec(s * h * t * d);
        auto gq = ctx.tensor_from_slice({s, h, t, d}, q), gk = ctx.tensor_from_slice({s, h, t, d}, k),
             gv = ctx.tensor_from_slice({s, h, t, d}, v);
        auto got = ctx.download(ctx.attention(gq, gk, gv));
        const float scale = 1.0f / std::sqrt(static_cast<float>(d));
        std::vector<float> sc(t);
        for (size_t sh = 0; sh < s * h; sh++)
            for (size_t qi = 0; qi < t; qi++) {
                const float* qv = &q[(sh * t + qi) * d];
                float mx = -3.4e38f;
                for (size_t ki = 0; ki < t; ki++) {
                    float acc = 0.0f;
                    for (size_t dd = 0; dd < d; dd++) acc += qv[dd] * k[(sh * t + ki) * d + dd];
                    sc[ki] = acc * scale;
                    mx = std::fmax(mx, sc[ki]);
                }
                float den = 0.0f;
                for (auto& x : sc) den += (x = std::exp(x - mx));
                for (size_t dd = 0; dd < d; dd++) {
                    float e = 0.0f;
                    for (size_t ki = 0; ki < t; ki++) e += sc[ki] * v[(sh * t + ki) * d + dd];
                    e /= den;
                    const float a = got[(sh * t + qi) * d + dd];
                    if (!(std::fabs(a - e) < 1e-4f))
                        throw Failure("attention t=" + std::to_string(t) + ": " + std::to_string(a) +
                                      " vs " + std::to_string(e));
                }
            }
        auto hq = ctx.tensor_from_f32({s, h, t, d}, q, Dtype::F16);
        auto hk = ctx.tensor_from_f32({s, h, t, d}, k, Dtype::F16);
        auto hv = ctx.tensor_from_f32({s, h, t, d}, v, Dtype::F16);
        auto att16 = ctx.attention(hq, hk, hv);
        assert_close(ctx.download(att16), got, 5e-3f, "attention f16 vs f32");
        auto merged = ctx.download(ctx.attn_merge(att16));
        auto head = ctx.download(att16);
        std::vector<float> want(merged.size());
        for (size_t si = 0; si < s; si++)
            for (size_t hi = 0; hi < h; hi++)
                for (size_t ti = 0; ti < t; ti++)
                    for (size_t dd = 0; dd < d; dd++)
                        want[((si * t + ti) * h + hi) * d + dd] = head[(((si * h) + hi) * t + ti) * d + dd];
        exact(merged, want, "attn_merge");
        exact(ctx.download(ctx.attention_merged(hq, hk, hv)), merged, "attention_merged");
    }
}

// tests/kernels.rs:63-99 and 313-365: linear against float64 sums on the
// (f16-rounded) inputs; the f16 cases also at a matrix-core shape
// (N % 256 == 0, K % 64 == 0), and the fused epilogues against the
// reference's two-dispatch sequences.
void linear_matches_cpu(HipContext& ctx) {
    auto reference = [](const std::vector<float>& x, const std::vector<float>& w,
                        const std::vector<float>* b, size_t m, size_t n, size_t k, bool f16_out) {
        std::vector<float> e(m * n);
        for (size_t r = 0; r < m; r++)
            for (size_t c = 0; c < n; c++) {
                double acc = 0.0;
                for (size_t kk = 0; kk < k; kk++) acc += double(x[r * k + kk]) * double(w[c * k + kk]);
                float v = static_cast<float>(acc) + (b ? (*b)[c] : 0.0f);
                e[r * n + c] = f16_out ? hs::f16_to_f32(hs::f32_to_f16(v)) : v;
            }
        return e;
    };
    {
        Rng rng{2};
        const size_t m = 37, k = 53, n = 29;
        auto x = rng.vec(m * k), w = rng.vec(n * k), b = rng.vec(n);
        auto gx = ctx.tensor_from_slice({m, k}, x), gw = ctx.tensor_from_slice({n, k}, w);
        auto gb = ctx.tensor_from_slice({n}, b);
        assert_close(ctx.download(ctx.linear(gx, gw, &gb)), reference(x, w, &b, m, n, k, false), 1e-4f,
                     "linear");
        assert_close(ctx.download(ctx.linear(gx, gw)), reference(x, w, nullptr, m, n, k, false), 1e-4f,
                     "linear-nobias");
    }
    for (auto [m, k, n] : {std::array<size_t, 3>{37, 96, 128}, std::array<size_t, 3>{37, 128, 256}}) {
        Rng rng{8};
        auto x = rng.vec(m * k), w = rng.vec(n * k), b = rng.vec(n);
        auto round = [](std::vector<float> v) {
            for (auto& e : v) e = hs::f16_to_f32(hs::f32_to_f16(e));
            return v;
        };
        auto xr = round(x), wr = round(w);
        auto gx = ctx.tensor_from_f32({m, k}, x, Dtype::F16), gw = ctx.tensor_from_f32({n, k}, w, Dtype::F16);
        auto gb = ctx.tensor_from_slice({n}, b);
        auto lin = ctx.linear(gx, gw, &gb);
        assert_close(ctx.download(lin), reference(xr, wr, &b, m, n, k, true), 1e-2f, "linear f16");
        // fused epilogues == the reference's sequences through the same context
        f16_gate(ctx.download(ctx.linear_gelu(gx, gw, &gb)), ctx.download(ctx.gelu(lin)), "linear_gelu");
        auto res = ctx.tensor_from_f32({m, n}, rng.vec(m * n), Dtype::F16);
        auto gam = ctx.tensor_from_slice({n}, rng.vec(n));
        f16_gate(ctx.download(ctx.linear_ls_residual(gx, gw, gam, res, &gb)),
                 ctx.download(ctx.residual_ls(res, lin, gam)), "linear_ls_residual");
    }
}

// The fused q|k|v projection == linear per third, then qknorm_rope
// (bit-exact for 16 heads: the same head-vector code), and its f32
// fallback == that sequence exactly.
void qkv_heads_equal_sequence(HipContext& ctx) {
    Rng rng{11};
    const size_t s = 2, h = 16, d = 64, prefix = 5, t = 6 + prefix, k = 128, n3 = 3 * h * d;
    auto x = rng.vec(s * t * k), w = rng.vec(n3 * k), b = rng.vec(n3), nw = rng.vec(d), nb = rng.vec(d);
    for (auto& e : w) e *= 0.1f;
    auto [sin, cos] = hs::rope::tables(hs::rope::periods(), 2, 3);
    auto gw_n = ctx.tensor_from_slice({d}, nw), gb_n = ctx.tensor_from_slice({d}, nb);
    auto st = ctx.tensor_from_slice({t - prefix, d}, sin), ct = ctx.tensor_from_slice({t - prefix, d}, cos);
    hs::Norm norm{&gw_n, &gb_n};
    hs::Rope rope{&st, &ct, prefix};
    auto gb = ctx.tensor_from_slice({n3}, b);
    for (Dtype dt : {Dtype::F16, Dtype::F32}) {
        auto gx = ctx.tensor_from_f32({s * t, k}, x, dt), gw = ctx.tensor_from_f32({n3, k}, w, dt);
        auto fused = ctx.linear_qkv_heads(gx, gw, &gb, s, t, h, &norm, &norm, &rope);
        const HipTensor* outs[3] = {&fused.q, &fused.k, &fused.v};
        for (size_t i = 0; i < 3; i++) {
            std::vector<float> wi(w.begin() + i * h * d * k, w.begin() + (i + 1) * h * d * k);
            std::vector<float> bi(b.begin() + i * h * d, b.begin() + (i + 1) * h * d);
            auto gwi = ctx.tensor_from_f32({h * d, k}, wi, dt);
            auto gbi = ctx.tensor_from_slice({h * d}, bi);
            auto proj = ctx.linear(gx, gwi, &gbi);
            auto seq = ctx.qknorm_rope(proj, s, t, h, d, i < 2 ? &norm : nullptr, i < 2 ? &rope : nullptr);
            exact(ctx.download(*outs[i]), ctx.download(seq),
                  dt == Dtype::F16 ? "linear_qkv_heads f16" : "linear_qkv_heads f32 fallback");
        }
    }
}

// q and k in one launch == two qknorm_rope calls, with and without RoPE.
void qknorm_rope_pair_equals_two_calls(HipContext& ctx) {
    Rng rng{13};
    const size_t s = 3, h = 16, d = 64, prefix = 5, t = 6 + prefix;
    auto [sin, cos] = hs::rope::tables(hs::rope::periods(), 2, 3);
    auto st = ctx.tensor_from_slice({t - prefix, d}, sin), ct = ctx.tensor_from_slice({t - prefix, d}, cos);
    auto qw = ctx.tensor_from_slice({d}, rng.vec(d)), qb = ctx.tensor_from_slice({d}, rng.vec(d));
    auto kw = ctx.tensor_from_slice({d}, rng.vec(d)), kb = ctx.tensor_from_slice({d}, rng.vec(d));
    hs::Norm qn{&qw, &qb}, kn{&kw, &kb};
    hs::Rope rope{&st, &ct, prefix};
    for (Dtype dt : {Dtype::F16, Dtype::F32})
        for (const hs::Rope* rp : {static_cast<const hs::Rope*>(&rope), static_cast<const hs::Rope*>(nullptr)}) {
            auto q = ctx.tensor_from_f32({s * t, h * d}, rng.vec(s * t * h * d), dt);
            auto k = ctx.tensor_from_f32({s * t, h * d}, rng.vec(s * t * h * d), dt);
            auto pair = ctx.qknorm_rope_pair(q, k, s, t, h, d, &qn, &kn, rp);
            exact(ctx.download(pair.q), ctx.download(ctx.qknorm_rope(q, s, t, h, d, &qn, rp)), "pair q");
            exact(ctx.download(pair.k), ctx.download(ctx.qknorm_rope(k, s, t, h, d, &kn, rp)), "pair k");
        }
}

// The LayerNorm as the product's prologue == layernorm then the product,
// bit for bit: the same statistics, the same normalised and rounded rows,
// the same accumulation order; likewise with GELU and with the q|k|v heads.
void layernorm_prologue_equals_sequence(HipContext& ctx) {
    for (auto [m, k, n] : {std::array<size_t, 3>{37, 128, 256}, std::array<size_t, 3>{19, 96, 48},
                           std::array<size_t, 3>{300, 1024, 512}}) {
        Rng rng{17 + n};
        auto x = rng.vec(m * k), w = rng.vec(n * k), b = rng.vec(n), g = rng.vec(k), be = rng.vec(k);
        for (auto& e : w) e *= 0.1f;
        for (auto& e : g) e = 1.0f + 0.1f * e;
        for (auto& e : be) e *= 0.1f;
        auto gg = ctx.tensor_from_slice({k}, g), gbe = ctx.tensor_from_slice({k}, be);
        auto gb = ctx.tensor_from_slice({n}, b);
        hs::Norm ln{&gg, &gbe};
        for (Dtype dt : {Dtype::F32, Dtype::F16}) {
            auto gx = ctx.tensor_from_f32({m, k}, x, dt), gw = ctx.tensor_from_f32({n, k}, w, dt);
            auto normed = ctx.layernorm(gx, gg, gbe, 1e-6f);
            exact(ctx.download(ctx.linear_ln(gx, ln, gw, &gb, 1e-6f)),
                  ctx.download(ctx.linear(normed, gw, &gb)), "linear_ln");
            exact(ctx.download(ctx.linear_ln_gelu(gx, ln, gw, &gb, 1e-6f)),
                  ctx.download(ctx.linear_gelu(normed, gw, &gb)), "linear_ln_gelu");
        }
    }
    // LN1 + q|k|v with heads, QK-norm and RoPE == layernorm then linear_qkv_heads
    Rng rng{23};
    const size_t s = 2, h = 16, d = 64, prefix = 5, t = 6 + prefix, k = 128, n3 = 3 * h * d;
    auto x = rng.vec(s * t * k), w = rng.vec(n3 * k), b = rng.vec(n3), g = rng.vec(k), be = rng.vec(k);
    for (auto& e : w) e = 0.1f * (e - 1.0f);
    for (auto& e : b) e = 0.1f * (e - 1.0f);
    for (auto& e : g) e = 1.0f + 0.1f * e;
    for (auto& e : be) e *= 0.1f;
    auto [sin, cos] = hs::rope::tables(hs::rope::periods(), 2, 3);
    auto nw = ctx.tensor_from_slice({d}, rng.vec(d)), nb = ctx.tensor_from_slice({d}, rng.vec(d));
    auto st = ctx.tensor_from_slice({t - prefix, d}, sin), ct = ctx.tensor_from_slice({t - prefix, d}, cos);
    hs::Norm norm{&nw, &nb};
    hs::Rope rope{&st, &ct, prefix};
    auto gg = ctx.tensor_from_slice({k}, g), gbe = ctx.tensor_from_slice({k}, be);
    auto gb = ctx.tensor_from_slice({n3}, b);
    hs::Norm ln{&gg, &gbe};
    for (Dtype dt : {Dtype::F16, Dtype::F32}) {  // f32 takes the layernorm-then-linear fallback
        auto gx = ctx.tensor_from_f32({s * t, k}, x, dt), gw = ctx.tensor_from_f32({n3, k}, w, dt);
        auto fused = ctx.linear_ln_qkv_heads(gx, ln, gw, &gb, s, t, h, &norm, &norm, &rope, 1e-6f);
        auto seq = ctx.linear_qkv_heads(ctx.layernorm(gx, gg, gbe, 1e-6f), gw, &gb, s, t, h, &norm,
                                        &norm, &rope, 1e-6f);
        const HipTensor* got[3] = {&fused.q, &fused.k, &fused.v};
        const HipTensor* want[3] = {&seq.q, &seq.k, &seq.v};
        for (int i = 0; i < 3; i++)
            exact(ctx.download(*got[i]), ctx.download(*want[i]),
                  std::string("linear_ln_qkv_heads ") + "qkv"[i] + (dt == Dtype::F16 ? " f16" : " f32"));
    }
}

void contract_violations_throw(HipContext& ctx) {
    auto x = ctx.tensor_from_slice({4, 8}, std::vector<float>(32, 1.0f));
    auto w = ctx.tensor_from_slice({7}, std::vector<float>(7, 1.0f));
    bool threw = false;
    try {
        (void)ctx.layernorm(x, w, w);
    } catch (const hs::ContractViolation&) {
        threw = true;
    }
    if (!threw) throw Failure("layernorm accepted a weight of the wrong length");
    threw = false;
    try {
        auto x16 = ctx.tensor_from_f32({4, 8}, std::vector<float>(32, 1.0f), Dtype::F16);
        auto g16 = ctx.tensor_from_f32({8}, std::vector<float>(8, 1.0f), Dtype::F16);
        (void)ctx.residual_ls(x16, x16, g16);
    } catch (const hs::ContractViolation&) {
        threw = true;
    }
    if (!threw) throw Failure("residual_ls accepted an f16 gamma");
}

}  // namespace

int main(int argc, char** argv) {
    const std::vector<std::pair<const char*, std::function<void(HipContext&)>>> tests = {
        {"layernorm_matches_cpu", layernorm_matches_cpu},
        {"gelu_matches_erf", gelu_matches_erf},
        {"rope_apply_matches_cpu", rope_apply_matches_cpu},
        {"split_heads_layout", split_heads_layout},
        {"copy_rows_and_tiled_add", copy_rows_and_tiled_add},
        {"every_op_f16_matches_f32", every_op_f16_matches_f32},
        {"fused_ops_equal_reference_sequence", fused_ops_equal_reference_sequence},
        {"assemble_equals_cast_and_copy_rows", assemble_equals_cast_and_copy_rows},
        {"attention_matches_cpu", attention_matches_cpu},
        {"linear_matches_cpu", linear_matches_cpu},
        {"qkv_heads_equal_sequence", qkv_heads_equal_sequence},
        {"qknorm_rope_pair_equals_two_calls", qknorm_rope_pair_equals_two_calls},
        {"layernorm_prologue_equals_sequence", layernorm_prologue_equals_sequence},
        {"contract_violations_throw", contract_violations_throw},
    };
    HipContext ctx;
    int failed = 0, ran = 0;
    for (const auto& [name, fn] : tests) {
        if (argc > 1 && std::strstr(name, argv[1]) == nullptr) continue;
        ran++;
        std::printf("test %s ... ", name);
        std::fflush(stdout);
        try {
            fn(ctx);
            std::printf("ok\n");
        } catch (const std::exception& e) {
            std::printf("FAILED: %s\n", e.what());
            failed++;
        }
        std::fflush(stdout);
    }
    std::printf("%d passed, %d failed\n", ran - failed, failed);
    return failed ? 1 : 0;
}
