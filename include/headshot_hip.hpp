// headshot_hip.hpp — C++ host surface over the C ABI in headshot_hip.h.
//
// Mirrors headshot-server's `GpuContext` / `GpuTensor` for the per-layer op
// path (crates/headshot-server/src/engine/ops.rs, engine/tensor.rs,
// engine/rope.rs): the same method names and argument meaning, tensors that
// own device memory (allocated on creation, freed on destruction), and the
// reference's contract checks. Where the reference panics on a violated
// contract (`assert!`), these methods throw hs::ContractViolation; a failed
// HIP call throws hs::HipError. Header-only; compile with hipcc and link
// libheadshot_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "headshot_hip.h"

namespace hs {

// engine/tensor.rs:12-25
enum class Dtype : int { F32 = HS_F32, F16 = HS_F16 };

inline size_t dtype_size(Dtype dt) { return dt == Dtype::F16 ? 2 : 4; }

// Shapes the fused q|k|v kernels cover: head dim 64, whole column tiles (256
// in f16, 128 in f32) and whole k stages (64 in f16, 32 in f32).
inline bool qkv_fused(Dtype dt, size_t d, size_t n3, size_t k) {
    if (d != 64) return false;
    return dt == Dtype::F16 ? n3 % 256 == 0 && k % 64 == 0 : n3 % 128 == 0 && k % 32 == 0;
}

struct ContractViolation : std::logic_error {
    using std::logic_error::logic_error;
};
struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define HS_REQUIRE(cond, msg)                                                  \
    do {                                                                       \
        if (!(cond)) throw ::hs::ContractViolation(std::string(msg));          \
    } while (0)

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}

inline void check(hs_status st, const char* op) {
    if (st == HS_OK) return;
    std::string msg = std::string(op) + ": " + hs_last_error();
    if (st == HS_EINVAL) throw ContractViolation(msg);
    throw HipError(msg + " (" + hs_status_string(st) + ")");
}

// binary16 <-> binary32 with round-to-nearest-even (what the reference's
// upload path does with half::f16::from_f32, engine/tensor.rs:71-91).
inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)
        return static_cast<uint16_t>(sign | (ax == 0x7f800000u ? 0x7c00u : 0x7e00u | ((ax >> 13) & 0x3ffu)));
    if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);
    if (ax < 0x38800000u)
        return static_cast<uint16_t>(sign | static_cast<uint32_t>(std::nearbyint(std::fabs(f) * 16777216.0f)));
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return static_cast<uint16_t>(sign | h);
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        float v = static_cast<float>(mant) * (1.0f / 16777216.0f);
        std::memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

// engine/tensor.rs:27-57: device buffer + shape + storage type.
class HipTensor {
   public:
    HipTensor() = default;
    HipTensor(std::vector<size_t> shape, Dtype dt) : shape_(std::move(shape)), dtype_(dt) {
        const size_t n = bytes();
        if (n) hip_check(hipMalloc(&ptr_, n), "hipMalloc");
    }
    ~HipTensor() {
        if (ptr_) (void)hipFree(ptr_);
    }
    HipTensor(HipTensor&& o) noexcept { *this = std::move(o); }
    HipTensor& operator=(HipTensor&& o) noexcept {
        if (this != &o) {
            if (ptr_) (void)hipFree(ptr_);
            ptr_ = o.ptr_, shape_ = std::move(o.shape_), dtype_ = o.dtype_;
            o.ptr_ = nullptr;
        }
        return *this;
    }
    HipTensor(const HipTensor&) = delete;
    HipTensor& operator=(const HipTensor&) = delete;

    size_t len() const {
        size_t n = 1;
        for (size_t s : shape_) n *= s;
        return n;
    }
    size_t bytes() const { return len() * dtype_size(dtype_); }
    size_t last() const { return shape_.empty() ? 0 : shape_.back(); }
    const std::vector<size_t>& shape() const { return shape_; }
    Dtype dtype() const { return dtype_; }
    void* data() { return ptr_; }
    const void* data() const { return ptr_; }
    const float* f32() const { return static_cast<const float*>(ptr_); }

    // engine/tensor.rs:52-56
    HipTensor reshaped(std::vector<size_t> shape) && {
        size_t n = 1;
        for (size_t s : shape) n *= s;
        HS_REQUIRE(n == len(), "reshape element count");
        shape_ = std::move(shape);
        return std::move(*this);
    }

   private:
    void* ptr_ = nullptr;
    std::vector<size_t> shape_;
    Dtype dtype_ = Dtype::F32;
};

// RoPE tables + unrotated prefix for one attention call (model/block.rs:42-47).
struct Rope {
    const HipTensor* sin;
    const HipTensor* cos;
    size_t prefix;
};

// A LayerNorm's weight and bias: one side's QK-norm (model/block.rs:35-40)
// or a pre-norm (LN1, LN2).
struct Norm {
    const HipTensor* weight;
    const HipTensor* bias;
};

class HipContext {
   public:
    HipContext() {
        HS_REQUIRE(hs_abi_version() == HS_ABI_VERSION, "libheadshot_hip ABI mismatch");
        hip_check(hipStreamCreate(&stream_), "hipStreamCreate");
    }
    ~HipContext() {
        if (stream_) {
            (void)hipStreamSynchronize(stream_);
            (void)hipStreamDestroy(stream_);
        }
    }
    HipContext(const HipContext&) = delete;
    HipContext& operator=(const HipContext&) = delete;

    hipStream_t stream() const { return stream_; }
    void sync() const { hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }

    // ------------------------------------------------------------- tensors

    HipTensor empty_typed(std::vector<size_t> shape, Dtype dt) const {
        return HipTensor(std::move(shape), dt);
    }

    // engine/tensor.rs:70-91: upload f32 data as dt storage
    HipTensor tensor_from_f32(std::vector<size_t> shape, const std::vector<float>& data,
                              Dtype dt) const {
        HipTensor t(std::move(shape), dt);
        HS_REQUIRE(data.size() == t.len(), "shape/data mismatch");
        if (dt == Dtype::F32) {
            hip_check(hipMemcpy(t.data(), data.data(), t.bytes(), hipMemcpyHostToDevice), "upload");
        } else {
            std::vector<uint16_t> h(data.size());
            for (size_t i = 0; i < data.size(); i++) h[i] = f32_to_f16(data[i]);
            hip_check(hipMemcpy(t.data(), h.data(), t.bytes(), hipMemcpyHostToDevice), "upload");
        }
        return t;
    }
    HipTensor tensor_from_slice(std::vector<size_t> shape, const std::vector<float>& data) const {
        return tensor_from_f32(std::move(shape), data, Dtype::F32);
    }

    // engine/tensor.rs:162-198: flush and read back as f32
    std::vector<float> download(const HipTensor& t) const {
        sync();
        std::vector<float> out(t.len());
        if (t.dtype() == Dtype::F32) {
            hip_check(hipMemcpy(out.data(), t.data(), t.bytes(), hipMemcpyDeviceToHost), "download");
        } else {
            std::vector<uint16_t> h(t.len());
            hip_check(hipMemcpy(h.data(), t.data(), t.bytes(), hipMemcpyDeviceToHost), "download");
            for (size_t i = 0; i < h.size(); i++) out[i] = f16_to_f32(h[i]);
        }
        return out;
    }

    // ------------------------------------------------------- reference ops

    // engine/ops.rs:130-153 (eps 1e-5 there)
    HipTensor layernorm(const HipTensor& x, const HipTensor& weight, const HipTensor& bias,
                        float eps = 1e-5f) const {
        const size_t dim = x.last();
        HS_REQUIRE(weight.len() == dim, "norm weight length");
        HS_REQUIRE(bias.len() == dim, "norm bias length");
        HS_REQUIRE(weight.dtype() == Dtype::F32, "norm weight must be f32");
        HS_REQUIRE(bias.dtype() == Dtype::F32, "norm bias must be f32");
        HipTensor out = empty_typed(x.shape(), x.dtype());
        check(hs_layernorm(stream_, hs_dtype(x.dtype()), x.data(), weight.f32(), bias.f32(),
                           out.data(), dim ? static_cast<int64_t>(x.len() / dim) : 0,
                           static_cast<int32_t>(dim), eps),
              "layernorm");
        return out;
    }

    // engine/ops.rs:155-165
    HipTensor gelu(const HipTensor& x) const {
        HipTensor out = empty_typed(x.shape(), x.dtype());
        check(hs_gelu(stream_, hs_dtype(x.dtype()), x.data(), out.data(),
                      static_cast<int64_t>(x.len())),
              "gelu");
        return out;
    }

    // engine/ops.rs:167-183
    HipTensor residual_ls(const HipTensor& res, const HipTensor& x, const HipTensor& gamma) const {
        HS_REQUIRE(res.len() == x.len(), "res/x length");
        HS_REQUIRE(res.dtype() == x.dtype(), "res/x dtype");
        HS_REQUIRE(gamma.dtype() == Dtype::F32, "gamma must be f32");
        const size_t dim = gamma.len();
        HS_REQUIRE(dim > 0 && x.len() % dim == 0, "gamma must tile x");
        HipTensor out = empty_typed(res.shape(), x.dtype());
        check(hs_residual_ls(stream_, hs_dtype(x.dtype()), res.data(), x.data(), gamma.f32(),
                             out.data(), static_cast<int64_t>(x.len()), static_cast<int32_t>(dim)),
              "residual_ls");
        return out;
    }

    // engine/ops.rs:185-200
    HipTensor split_heads(const HipTensor& x, size_t s, size_t t, size_t h, size_t d) const {
        HS_REQUIRE(x.len() == s * t * h * d, "split_heads size");
        HipTensor out = empty_typed({s, h, t, d}, x.dtype());
        check(hs_split_heads(stream_, hs_dtype(x.dtype()), x.data(), out.data(), i32(s), i32(t),
                             i32(h), i32(d)),
              "split_heads");
        return out;
    }

    // engine/ops.rs:202-223: in place on (S, H, T, D); tables (T - prefix, D)
    void rope_apply(HipTensor& x, const HipTensor& sin, const HipTensor& cos, size_t prefix) const {
        HS_REQUIRE(x.shape().size() == 4, "rope_apply wants (S,H,T,D)");
        const size_t s = x.shape()[0], h = x.shape()[1], t = x.shape()[2], d = x.shape()[3];
        HS_REQUIRE(prefix <= t, "prefix");
        HS_REQUIRE(sin.len() == (t - prefix) * d, "table size");
        HS_REQUIRE(cos.len() == sin.len(), "table size");
        HS_REQUIRE(sin.dtype() == Dtype::F32 && cos.dtype() == Dtype::F32, "rope tables must be f32");
        check(hs_rope_apply(stream_, hs_dtype(x.dtype()), x.data(), sin.f32(), cos.f32(), i32(s),
                            i32(h), i32(t), i32(d), i32(prefix)),
              "rope_apply");
    }

    // engine/ops.rs:81-128: out (m, n) = x (m, k) @ w (n, k)^T [+ bias]
    HipTensor linear(const HipTensor& x, const HipTensor& w, const HipTensor* bias = nullptr) const {
        size_t m, n, k;
        linear_shape(x, w, bias, m, n, k);
        HipTensor out = empty_typed({m, n}, x.dtype());
        check(hs_linear(stream_, hs_dtype(x.dtype()), x.data(), w.data(), bias ? bias->f32() : nullptr,
                        out.data(), static_cast<int64_t>(m), i32(n), i32(k)),
              "linear");
        return out;
    }

    // linear(fc1, bias) + GELU (model/block.rs:172-176) in one kernel
    HipTensor linear_gelu(const HipTensor& x, const HipTensor& w, const HipTensor* bias = nullptr) const {
        size_t m, n, k;
        linear_shape(x, w, bias, m, n, k);
        HipTensor out = empty_typed({m, n}, x.dtype());
        check(hs_linear_gelu(stream_, hs_dtype(x.dtype()), x.data(), w.data(),
                             bias ? bias->f32() : nullptr, out.data(), static_cast<int64_t>(m), i32(n),
                             i32(k)),
              "linear_gelu");
        return out;
    }

    // linear(proj | fc2, bias) + LayerScale + residual (model/block.rs:150-155)
    HipTensor linear_ls_residual(const HipTensor& x, const HipTensor& w, const HipTensor& gamma,
                                 const HipTensor& res, const HipTensor* bias = nullptr) const {
        size_t m, n, k;
        linear_shape(x, w, bias, m, n, k);
        HS_REQUIRE(gamma.dtype() == Dtype::F32 && gamma.len() == n, "gamma must be f32 (n)");
        HS_REQUIRE(res.dtype() == x.dtype() && res.len() == m * n, "res shape/dtype");
        HipTensor out = empty_typed({m, n}, x.dtype());
        check(hs_linear_ls_residual(stream_, hs_dtype(x.dtype()), x.data(), w.data(),
                                    bias ? bias->f32() : nullptr, gamma.f32(), res.data(), out.data(),
                                    static_cast<int64_t>(m), i32(n), i32(k)),
              "linear_ls_residual");
        return out;
    }

    // engine/ops.rs:302-318: a (rows, c1) ++ b (rows, c2) -> (rows, c1 + c2)
    HipTensor concat_channels(const HipTensor& a, const HipTensor& b) const {
        const size_t c1 = a.last(), c2 = b.last();
        HS_REQUIRE(c1 && c2, "concat_channels: empty rows");
        const size_t rows = a.len() / c1;
        HS_REQUIRE(b.len() / c2 == rows, "row mismatch");
        HS_REQUIRE(a.dtype() == b.dtype(), "concat_channels dtype");
        HipTensor out = empty_typed({rows, c1 + c2}, a.dtype());
        check(hs_concat_channels(stream_, hs_dtype(a.dtype()), a.data(), b.data(), out.data(),
                                 static_cast<int64_t>(rows), i32(c1), i32(c2)),
              "concat_channels");
        return out;
    }

    // engine/ops.rs:321-334 (f16 -> f32)
    HipTensor cast_to_f32(const HipTensor& x) const {
        HS_REQUIRE(x.dtype() == Dtype::F16, "cast_to_f32 wants f16");
        HipTensor out = empty_typed(x.shape(), Dtype::F32);
        check(hs_cast_f16_to_f32(stream_, x.data(), static_cast<float*>(out.data()),
                                 static_cast<int64_t>(x.len())),
              "cast_to_f32");
        return out;
    }

    // Cache::build (model/cache.rs:21-52) in one pass: concat + cast to f32
    HipTensor cache_build(const HipTensor& frame_out, const HipTensor& inter_out) const {
        const size_t c1 = frame_out.last(), c2 = inter_out.last();
        HS_REQUIRE(c1 && c2, "cache_build: empty rows");
        const size_t rows = frame_out.len() / c1;
        HS_REQUIRE(inter_out.len() / c2 == rows, "row mismatch");
        HS_REQUIRE(frame_out.dtype() == inter_out.dtype(), "cache_build dtype");
        HipTensor out = empty_typed({rows, c1 + c2}, Dtype::F32);
        check(hs_cache_build(stream_, hs_dtype(frame_out.dtype()), frame_out.data(), inter_out.data(),
                             static_cast<float*>(out.data()), static_cast<int64_t>(rows), i32(c1),
                             i32(c2)),
              "cache_build");
        return out;
    }

    // n_blocks copy_rows calls in one launch (model/trunk.rs:103-116)
    void copy_row_blocks(const HipTensor& src, size_t src_row, size_t src_stride, HipTensor& dst,
                         size_t dst_row, size_t dst_stride, size_t n_blocks,
                         size_t rows_per_block) const {
        HS_REQUIRE(src.dtype() == dst.dtype(), "copy_row_blocks dtype");
        const size_t row = src.last() * dtype_size(src.dtype());
        HS_REQUIRE(row == dst.last() * dtype_size(dst.dtype()), "copy_row_blocks row width");
        if (n_blocks && rows_per_block) {
            HS_REQUIRE((src_row + (n_blocks - 1) * src_stride + rows_per_block) * row <=
                           src.len() * dtype_size(src.dtype()), "src rows");
            HS_REQUIRE((dst_row + (n_blocks - 1) * dst_stride + rows_per_block) * row <=
                           dst.len() * dtype_size(dst.dtype()), "dst rows");
        }
        check(hs_copy_row_blocks(stream_, src.data(), static_cast<int64_t>(src_row),
                                 static_cast<int64_t>(src_stride), dst.data(),
                                 static_cast<int64_t>(dst_row), static_cast<int64_t>(dst_stride),
                                 static_cast<int64_t>(n_blocks), static_cast<int64_t>(rows_per_block),
                                 static_cast<int64_t>(row)),
              "copy_row_blocks");
    }

    // engine/ops.rs:225-253: non-causal attention over head-major (S, H, T, D)
    HipTensor attention(const HipTensor& q, const HipTensor& k, const HipTensor& v) const {
        HS_REQUIRE(q.shape().size() == 4, "attention wants (S,H,T,D)");
        HS_REQUIRE(k.shape() == q.shape() && v.shape() == q.shape(), "attention: q/k/v shapes");
        HS_REQUIRE(k.dtype() == q.dtype() && v.dtype() == q.dtype(), "attention: dtype");
        const auto& sh = q.shape();
        HipTensor out = empty_typed(sh, q.dtype());
        check(hs_attention(stream_, hs_dtype(q.dtype()), q.data(), k.data(), v.data(), out.data(),
                           i32(sh[0]), i32(sh[1]), i32(sh[2]), i32(sh[3])),
              "attention");
        return out;
    }

    // engine/ops.rs:255-267: (S, H, T, D) -> (S*T, H*D)
    HipTensor attn_merge(const HipTensor& x) const {
        HS_REQUIRE(x.shape().size() == 4, "attn_merge wants (S,H,T,D)");
        const auto& sh = x.shape();
        HipTensor out = empty_typed({sh[0] * sh[2], sh[1] * sh[3]}, x.dtype());
        check(hs_attn_merge(stream_, hs_dtype(x.dtype()), x.data(), out.data(), i32(sh[0]),
                            i32(sh[1]), i32(sh[2]), i32(sh[3])),
              "attn_merge");
        return out;
    }

    // attention + attn_merge (model/block.rs:148-149) in one pass
    HipTensor attention_merged(const HipTensor& q, const HipTensor& k, const HipTensor& v) const {
        HS_REQUIRE(q.shape().size() == 4, "attention wants (S,H,T,D)");
        HS_REQUIRE(k.shape() == q.shape() && v.shape() == q.shape(), "attention: q/k/v shapes");
        HS_REQUIRE(k.dtype() == q.dtype() && v.dtype() == q.dtype(), "attention: dtype");
        const auto& sh = q.shape();
        HipTensor out = empty_typed({sh[0] * sh[2], sh[1] * sh[3]}, q.dtype());
        check(hs_attention_merged(stream_, hs_dtype(q.dtype()), q.data(), k.data(), v.data(),
                                  out.data(), i32(sh[0]), i32(sh[1]), i32(sh[2]), i32(sh[3])),
              "attention_merged");
        return out;
    }

    // engine/ops.rs:336-348
    HipTensor cast_to_f16(const HipTensor& x) const {
        HS_REQUIRE(x.dtype() == Dtype::F32, "cast_to_f16 wants f32");
        HipTensor out = empty_typed(x.shape(), Dtype::F16);
        check(hs_cast_f32_to_f16(stream_, x.f32(), out.data(), static_cast<int64_t>(x.len())),
              "cast_to_f16");
        return out;
    }

    // engine/tensor.rs:146-160
    void copy_rows(const HipTensor& src, size_t src_row, HipTensor& dst, size_t dst_row,
                   size_t n_rows) const {
        HS_REQUIRE(src.dtype() == dst.dtype(), "copy_rows dtype");
        const size_t row = src.last() * dtype_size(src.dtype());
        HS_REQUIRE(row == dst.last() * dtype_size(dst.dtype()), "copy_rows row width");
        HS_REQUIRE((src_row + n_rows) * row <= src.bytes(), "copy_rows source rows");
        HS_REQUIRE((dst_row + n_rows) * row <= dst.bytes(), "copy_rows destination rows");
        check(hs_copy_rows(stream_, src.data(), static_cast<int64_t>(src_row), dst.data(),
                           static_cast<int64_t>(dst_row), static_cast<int64_t>(n_rows),
                           static_cast<int64_t>(row)),
              "copy_rows");
    }

    // engine/ops.rs:374-389 (f32 only)
    HipTensor tiled_add(const HipTensor& x, const HipTensor& table) const {
        HS_REQUIRE(x.dtype() == Dtype::F32 && table.dtype() == Dtype::F32, "tiled_add is f32");
        HS_REQUIRE(table.len() > 0 && x.len() % table.len() == 0, "table must tile x");
        HipTensor out = empty_typed(x.shape(), Dtype::F32);
        check(hs_tiled_add(stream_, x.f32(), table.f32(), static_cast<float*>(out.data()),
                           static_cast<int64_t>(x.len()), static_cast<int64_t>(table.len())),
              "tiled_add");
        return out;
    }

    // ----------------------------------------------------------- fused ops

    // split_heads + QK-norm + RoPE (model/block.rs:130-146) in one pass:
    // (S*T, H*D) token-major -> (S, H, T, D) head-major.
    HipTensor qknorm_rope(const HipTensor& x_tok, size_t s, size_t t, size_t h, size_t d,
                          const Norm* norm, const Rope* rope, float eps = 1e-5f) const {
        HS_REQUIRE(x_tok.len() == s * t * h * d, "qknorm_rope size");
        const float *nw = nullptr, *nb = nullptr, *sn = nullptr, *cs = nullptr;
        size_t prefix = 0;
        if (norm) {
            HS_REQUIRE(norm->weight->len() == d && norm->bias->len() == d, "qk-norm length");
            HS_REQUIRE(norm->weight->dtype() == Dtype::F32 && norm->bias->dtype() == Dtype::F32,
                       "qk-norm parameters must be f32");
            nw = norm->weight->f32(), nb = norm->bias->f32();
        }
        if (rope) {
            prefix = rope->prefix;
            HS_REQUIRE(prefix <= t, "prefix");
            HS_REQUIRE(rope->sin->len() == (t - prefix) * d && rope->cos->len() == rope->sin->len(),
                       "table size");
            HS_REQUIRE(rope->sin->dtype() == Dtype::F32 && rope->cos->dtype() == Dtype::F32,
                       "rope tables must be f32");
            sn = rope->sin->f32(), cs = rope->cos->f32();
        }
        HipTensor out = empty_typed({s, h, t, d}, x_tok.dtype());
        check(hs_qknorm_rope(stream_, hs_dtype(x_tok.dtype()), x_tok.data(), nw, nb, sn, cs,
                             out.data(), i32(s), i32(t), i32(h), i32(d), i32(prefix), eps),
              "qknorm_rope");
        return out;
    }

    // qknorm_rope on q (norm qn) and k (norm kn) in one launch; both norms
    // or neither. Bit-identical to two qknorm_rope calls.
    struct QkHeads {
        HipTensor q, k;
    };
    QkHeads qknorm_rope_pair(const HipTensor& q_tok, const HipTensor& k_tok, size_t s, size_t t,
                             size_t h, size_t d, const Norm* qn, const Norm* kn, const Rope* rope,
                             float eps = 1e-5f) const {
        HS_REQUIRE(q_tok.len() == s * t * h * d && k_tok.len() == q_tok.len(), "qk size");
        HS_REQUIRE(q_tok.dtype() == k_tok.dtype(), "q/k dtype");
        HS_REQUIRE((qn == nullptr) == (kn == nullptr), "QK-norm for both q and k or neither");
        const float *qw = nullptr, *qb = nullptr, *kw = nullptr, *kb = nullptr;
        const float *sn = nullptr, *cs = nullptr;
        size_t prefix = 0;
        for (const Norm* n : {qn, kn}) {
            if (!n) continue;
            HS_REQUIRE(n->weight->len() == d && n->bias->len() == d, "qk-norm length");
            HS_REQUIRE(n->weight->dtype() == Dtype::F32 && n->bias->dtype() == Dtype::F32,
                       "qk-norm parameters must be f32");
        }
        if (qn) qw = qn->weight->f32(), qb = qn->bias->f32(), kw = kn->weight->f32(),
                kb = kn->bias->f32();
        if (rope) {
            prefix = rope->prefix;
            HS_REQUIRE(prefix <= t, "prefix");
            HS_REQUIRE(rope->sin->len() == (t - prefix) * d && rope->cos->len() == rope->sin->len(),
                       "table size");
            HS_REQUIRE(rope->sin->dtype() == Dtype::F32 && rope->cos->dtype() == Dtype::F32,
                       "rope tables must be f32");
            sn = rope->sin->f32(), cs = rope->cos->f32();
        }
        QkHeads out{empty_typed({s, h, t, d}, q_tok.dtype()), empty_typed({s, h, t, d}, q_tok.dtype())};
        check(hs_qknorm_rope_pair(stream_, hs_dtype(q_tok.dtype()), q_tok.data(), k_tok.data(), qw,
                                  qb, kw, kb, sn, cs, out.q.data(), out.k.data(), i32(s), i32(t),
                                  i32(h), i32(d), i32(prefix), eps),
              "qknorm_rope_pair");
        return out;
    }

    // The q|k|v projection with split_heads, QK-norm and RoPE
    // (model/block.rs:128-146) in one launch on the fused (3*h*d, k) weight.
    // Returns head-major q, k, v. Shapes the fused kernels do not cover
    // (d != 64, 3*h*64 not a multiple of 256 in f16 or 128 in f32) run
    // linear then qknorm_rope per third.
    struct Qkv {
        HipTensor q, k, v;
    };
    Qkv linear_qkv_heads(const HipTensor& x, const HipTensor& w_qkv, const HipTensor* b_qkv,
                         size_t s, size_t t, size_t h, const Norm* qn, const Norm* kn,
                         const Rope* rope, float eps = 1e-5f) const {
        HS_REQUIRE(w_qkv.shape().size() == 2 && w_qkv.shape()[0] % (3 * h) == 0, "w_qkv shape");
        const size_t n3 = w_qkv.shape()[0], k = w_qkv.shape()[1], d = n3 / (3 * h), hd = h * d;
        HS_REQUIRE(x.len() == s * t * k && x.dtype() == w_qkv.dtype(), "x shape/dtype");
        HS_REQUIRE(!b_qkv || (b_qkv->dtype() == Dtype::F32 && b_qkv->len() == n3), "qkv bias");
        const bool fused = qkv_fused(x.dtype(), d, n3, k);
        if (!fused) {
            Qkv out;
            HipTensor* dst[3] = {&out.q, &out.k, &out.v};
            const Norm* norms[3] = {qn, kn, nullptr};
            const size_t esz = dtype_size(x.dtype());
            for (int i = 0; i < 3; i++) {
                // third i of the weight rows and of the bias
                HipTensor proj = empty_typed({s * t, hd}, x.dtype());
                check(hs_linear(stream_, hs_dtype(x.dtype()), x.data(),
                                static_cast<const char*>(w_qkv.data()) + i * hd * k * esz,
                                b_qkv ? b_qkv->f32() + i * hd : nullptr, proj.data(),
                                static_cast<int64_t>(s * t), i32(hd), i32(k)),
                      "linear");
                *dst[i] = qknorm_rope(proj, s, t, h, d, norms[i], i < 2 ? rope : nullptr, eps);
            }
            return out;
        }
        const float *qw = nullptr, *qb = nullptr, *kw = nullptr, *kb = nullptr;
        const float *sn = nullptr, *cs = nullptr;
        size_t prefix = 0;
        for (const auto& [n, w, b] : {std::tuple{qn, &qw, &qb}, std::tuple{kn, &kw, &kb}}) {
            if (!n) continue;
            HS_REQUIRE(n->weight->len() == d && n->bias->len() == d, "qk-norm length");
            HS_REQUIRE(n->weight->dtype() == Dtype::F32 && n->bias->dtype() == Dtype::F32,
                       "qk-norm parameters must be f32");
            *w = n->weight->f32(), *b = n->bias->f32();
        }
        if (rope) {
            prefix = rope->prefix;
            HS_REQUIRE(prefix <= t, "prefix");
            HS_REQUIRE(rope->sin->len() == (t - prefix) * d && rope->cos->len() == rope->sin->len(),
                       "table size");
            sn = rope->sin->f32(), cs = rope->cos->f32();
        }
        Qkv out{empty_typed({s, h, t, d}, x.dtype()), empty_typed({s, h, t, d}, x.dtype()),
                empty_typed({s, h, t, d}, x.dtype())};
        check(hs_linear_qkv_heads(stream_, hs_dtype(x.dtype()), x.data(), w_qkv.data(),
                                  b_qkv ? b_qkv->f32() : nullptr, qw, qb, kw, kb, sn, cs,
                                  out.q.data(), out.k.data(), out.v.data(), i32(s), i32(t), i32(h),
                                  i32(d), i32(k), i32(prefix), eps),
              "linear_qkv_heads");
        return out;
    }

    // layernorm(x, norm) then linear(w, bias) (LN1 -> q|k|v,
    // model/block.rs:128-131) in one product: the normalised rows, rounded to
    // the storage type as layernorm stores them, exist only on the way to the
    // matrix cores. The row statistics go to a workspace owned by the call.
    HipTensor linear_ln(const HipTensor& x, const Norm& norm, const HipTensor& w,
                        const HipTensor* bias, float eps = 1e-5f) const {
        return ln_call(x, norm, w, bias, eps, false);
    }
    // gelu(linear(layernorm(x))): LN2, fc1 with its bias, GELU
    // (model/block.rs:153, 172-176)
    HipTensor linear_ln_gelu(const HipTensor& x, const Norm& norm, const HipTensor& w,
                             const HipTensor* bias, float eps = 1e-5f) const {
        return ln_call(x, norm, w, bias, eps, true);
    }
    // LN1 and the q|k|v projection with heads, QK-norm and RoPE
    // (model/block.rs:128-146) in one product. Shapes the fused kernels do
    // not cover (see qkv_fused) run layernorm then linear_qkv_heads.
    Qkv linear_ln_qkv_heads(const HipTensor& x, const Norm& norm, const HipTensor& w_qkv,
                            const HipTensor* b_qkv, size_t s, size_t t, size_t h, const Norm* qn,
                            const Norm* kn, const Rope* rope, float eps = 1e-5f) const {
        HS_REQUIRE(w_qkv.shape().size() == 2 && w_qkv.shape()[0] % (3 * h) == 0, "w_qkv shape");
        const size_t n3 = w_qkv.shape()[0], k = w_qkv.shape()[1], d = n3 / (3 * h);
        HS_REQUIRE(x.len() == s * t * k && x.dtype() == w_qkv.dtype(), "x shape/dtype");
        HS_REQUIRE(!b_qkv || (b_qkv->dtype() == Dtype::F32 && b_qkv->len() == n3), "qkv bias");
        ln_params(norm, k);
        if (!qkv_fused(x.dtype(), d, n3, k))
            return linear_qkv_heads(layernorm(x, *norm.weight, *norm.bias, eps), w_qkv, b_qkv, s, t,
                                    h, qn, kn, rope, eps);
        const float *qw = nullptr, *qb = nullptr, *kw = nullptr, *kb = nullptr;
        const float *sn = nullptr, *cs = nullptr;
        size_t prefix = 0;
        for (const auto& [n, w, b] : {std::tuple{qn, &qw, &qb}, std::tuple{kn, &kw, &kb}}) {
            if (!n) continue;
            HS_REQUIRE(n->weight->len() == d && n->bias->len() == d, "qk-norm length");
            HS_REQUIRE(n->weight->dtype() == Dtype::F32 && n->bias->dtype() == Dtype::F32,
                       "qk-norm parameters must be f32");
            *w = n->weight->f32(), *b = n->bias->f32();
        }
        if (rope) {
            prefix = rope->prefix;
            HS_REQUIRE(prefix <= t, "prefix");
            HS_REQUIRE(rope->sin->len() == (t - prefix) * d && rope->cos->len() == rope->sin->len(),
                       "table size");
            sn = rope->sin->f32(), cs = rope->cos->f32();
        }
        HipTensor ws = empty_typed({2 * s * t}, Dtype::F32);
        Qkv out{empty_typed({s, h, t, d}, x.dtype()), empty_typed({s, h, t, d}, x.dtype()),
                empty_typed({s, h, t, d}, x.dtype())};
        check(hs_linear_ln_qkv_heads(stream_, hs_dtype(x.dtype()), x.data(), norm.weight->f32(),
                                     norm.bias->f32(), w_qkv.data(), b_qkv ? b_qkv->f32() : nullptr,
                                     qw, qb, kw, kb, sn, cs, static_cast<float*>(ws.data()),
                                     out.q.data(), out.k.data(), out.v.data(), i32(s), i32(t),
                                     i32(h), i32(d), i32(k), i32(prefix), eps),
              "linear_ln_qkv_heads");
        return out;
    }

    // fc1 bias epilogue + GELU (model/block.rs:173-174)
    HipTensor bias_gelu(const HipTensor& x, const HipTensor* bias) const {
        const size_t cols = x.last();
        if (bias) HS_REQUIRE(bias->len() == cols && bias->dtype() == Dtype::F32, "bias");
        HipTensor out = empty_typed(x.shape(), x.dtype());
        check(hs_bias_gelu(stream_, hs_dtype(x.dtype()), x.data(), bias ? bias->f32() : nullptr,
                           out.data(), cols ? static_cast<int64_t>(x.len() / cols) : 0, i32(cols)),
              "bias_gelu");
        return out;
    }

    // proj/fc2 bias epilogue + LayerScale + residual (model/block.rs:150-155)
    HipTensor bias_ls_residual(const HipTensor& res, const HipTensor& x, const HipTensor& gamma,
                               const HipTensor* bias) const {
        HS_REQUIRE(res.len() == x.len() && res.dtype() == x.dtype(), "res/x");
        const size_t dim = x.last();
        HS_REQUIRE(gamma.len() == dim && gamma.dtype() == Dtype::F32, "gamma");
        if (bias) HS_REQUIRE(bias->len() == dim && bias->dtype() == Dtype::F32, "bias");
        HipTensor out = empty_typed(res.shape(), x.dtype());
        check(hs_bias_ls_residual(stream_, hs_dtype(x.dtype()), res.data(), x.data(),
                                  bias ? bias->f32() : nullptr, gamma.f32(), out.data(),
                                  dim ? static_cast<int64_t>(x.len() / dim) : 0, i32(dim)),
              "bias_ls_residual");
        return out;
    }

    // bias_ls_residual then layernorm of its output in one pass
    // (model/block.rs:150-153: x1 into LN2; a block's output into the next
    // block's LN1): bit-identical to the two calls.
    struct ResidualNormed {
        HipTensor out, normed;
    };
    ResidualNormed bias_ls_residual_layernorm(const HipTensor& res, const HipTensor& x,
                                              const HipTensor& gamma, const HipTensor* bias,
                                              const Norm& norm, float eps = 1e-5f) const {
        HS_REQUIRE(res.len() == x.len() && res.dtype() == x.dtype(), "res/x");
        const size_t dim = x.last();
        HS_REQUIRE(gamma.len() == dim && gamma.dtype() == Dtype::F32, "gamma");
        if (bias) HS_REQUIRE(bias->len() == dim && bias->dtype() == Dtype::F32, "bias");
        ln_params(norm, dim);
        ResidualNormed r{empty_typed(res.shape(), x.dtype()), empty_typed(res.shape(), x.dtype())};
        check(hs_bias_ls_residual_layernorm(stream_, hs_dtype(x.dtype()), res.data(), x.data(),
                                            bias ? bias->f32() : nullptr, gamma.f32(),
                                            norm.weight->f32(), norm.bias->f32(), r.out.data(),
                                            r.normed.data(),
                                            dim ? static_cast<int64_t>(x.len() / dim) : 0, i32(dim),
                                            eps),
              "bias_ls_residual_layernorm");
        return r;
    }

    // model/trunk.rs:68-85: per frame [cam[v], reg[v*R..], patches + bias + pos]
    HipTensor assemble_tokens(const HipTensor& patches, size_t s, size_t p, const HipTensor& cam,
                              const HipTensor* reg, const HipTensor* patch_bias,
                              const HipTensor* pos, Dtype out_dt, int n_var = 2) const {
        const size_t d = patches.last();
        HS_REQUIRE(patches.len() == s * p * d, "patches shape");
        HS_REQUIRE(cam.dtype() == out_dt && cam.len() == static_cast<size_t>(n_var) * d,
                   "camera token shape/dtype");
        const size_t r = reg ? reg->len() / (static_cast<size_t>(n_var) * d) : 0;
        if (reg) HS_REQUIRE(reg->dtype() == out_dt, "register token dtype");
        if (patch_bias) HS_REQUIRE(patch_bias->len() == d && patch_bias->dtype() == Dtype::F32, "bias");
        if (pos) HS_REQUIRE(pos->len() == p * d && pos->dtype() == Dtype::F32, "pos embed");
        HipTensor out = empty_typed({s * (1 + r + p), d}, out_dt);
        check(hs_assemble_tokens(stream_, hs_dtype(out_dt), patches.data(),
                                 hs_dtype(patches.dtype()), patch_bias ? patch_bias->f32() : nullptr,
                                 pos ? pos->f32() : nullptr, cam.data(), reg ? reg->data() : nullptr,
                                 out.data(), i32(s), i32(p), i32(r), i32(d), n_var),
              "assemble_tokens");
        return out;
    }

   private:
    static ::hs_dtype hs_dtype(Dtype dt) { return static_cast<::hs_dtype>(static_cast<int>(dt)); }
    static void ln_params(const Norm& norm, size_t k) {
        HS_REQUIRE(norm.weight && norm.bias, "layernorm needs weight and bias");
        HS_REQUIRE(norm.weight->dtype() == Dtype::F32 && norm.weight->len() == k &&
                       norm.bias->dtype() == Dtype::F32 && norm.bias->len() == k,
                   "layernorm parameters must be f32 (k)");
    }
    HipTensor ln_call(const HipTensor& x, const Norm& norm, const HipTensor& w,
                      const HipTensor* bias, float eps, bool gelu) const {
        size_t m, n, k;
        linear_shape(x, w, bias, m, n, k);
        ln_params(norm, k);
        HipTensor ws = empty_typed({2 * m}, Dtype::F32);
        HipTensor out = empty_typed({m, n}, x.dtype());
        check((gelu ? hs_linear_ln_gelu : hs_linear_ln)(
                  stream_, hs_dtype(x.dtype()), x.data(), norm.weight->f32(), norm.bias->f32(),
                  w.data(), bias ? bias->f32() : nullptr, static_cast<float*>(ws.data()),
                  out.data(), static_cast<int64_t>(m), i32(n), i32(k), eps),
              gelu ? "linear_ln_gelu" : "linear_ln");
        return out;
    }
    static void linear_shape(const HipTensor& x, const HipTensor& w, const HipTensor* bias, size_t& m,
                             size_t& n, size_t& k) {
        k = x.last();
        HS_REQUIRE(k > 0 && w.shape().size() == 2 && w.shape()[1] == k, "weight k mismatch");
        HS_REQUIRE(w.dtype() == x.dtype(), "weight/activation dtype");
        m = x.len() / k, n = w.shape()[0];
        if (bias) HS_REQUIRE(bias->dtype() == Dtype::F32 && bias->len() == n, "bias must be f32 (n)");
    }

    static int32_t i32(size_t v) {
        HS_REQUIRE(v <= 0x7fffffffu, "dimension exceeds int32");
        return static_cast<int32_t>(v);
    }
    hipStream_t stream_ = nullptr;
};

namespace rope {

// engine/rope.rs:8-10
inline std::array<float, 16> periods() {
    std::array<float, 16> p{};
    hs_rope_periods(p.data());
    return p;
}

// engine/rope.rs:18-43: (sin, cos), each (h_p*w_p, 64)
inline std::pair<std::vector<float>, std::vector<float>> tables(const std::array<float, 16>& per,
                                                                size_t h_p, size_t w_p) {
    std::vector<float> sin(h_p * w_p * 64), cos(h_p * w_p * 64);
    check(hs_rope_tables(per.data(), static_cast<int32_t>(h_p), static_cast<int32_t>(w_p),
                         sin.data(), cos.data()),
          "rope_tables");
    return {std::move(sin), std::move(cos)};
}

}  // namespace rope
}  // namespace hs
