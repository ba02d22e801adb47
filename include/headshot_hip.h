/*
 * headshot_hip.h — C ABI of libheadshot_hip.so: headshot's fused per-layer
 * ops (LayerNorm, QK-norm + 2D RoPE, bias + erf-GELU, bias + LayerScale +
 * residual, patch-token assembly) as hand-written HIP kernels for gfx950.
 *
 * The entry points replace the op-dispatch methods of the reference's
 * `GpuContext` (crates/headshot-server/src/engine/ops.rs, engine/tensor.rs,
 * engine/rope.rs); each declaration names the method it stands in for. The
 * reference has no FFI layer: its string-keyed `dispatch(name, params,
 * buffers, grid)` registry (engine/mod.rs:216-258) is what these exports
 * replace, one function per kernel family.
 *
 * Conventions (all entry points):
 *  - Device pointers are caller-owned; the library never allocates device
 *    memory and keeps no per-call state. Work is enqueued on `stream` (a
 *    hipStream_t; NULL is the default stream) and is stream-ordered.
 *  - Activations are row-major. Token matrices are (rows, channels); the
 *    attention layout is head-major (S, H, T, D) (engine/ops.rs:1-3).
 *  - `dt` selects the storage type of activations (HS_F32 or HS_F16, the
 *    reference's `Elem`); norm weights, biases, LayerScale gammas,
 *    positional tables and RoPE tables are always f32 (engine/ops.rs:5-8).
 *    Arithmetic is f32 in both variants; f16 results are rounded to nearest
 *    even once, when stored.
 *  - Returns HS_OK, or HS_EINVAL for a contract violation (the reference
 *    panics on these: engine/ops.rs:134-137, 169-173, 206-208), HS_EHIP when
 *    a HIP call or kernel launch fails, HS_EUNSUPPORTED for a shape the
 *    library does not implement. hs_last_error() gives the message. Nothing
 *    is enqueued when a call fails validation.
 *  - Zero-sized work (rows == 0, S == 0, ...) is a valid no-op.
 *  - Tensors of 2^40 elements or more are refused with HS_EINVAL (several
 *    entry points also keep row or token counts below 2^31, as noted).
 *  - Calls are reentrant; calls on one stream execute in order.
 */
#ifndef HEADSHOT_HIP_H
#define HEADSHOT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* hs_stream_t; /* hipStream_t */

typedef enum { HS_F32 = 0, HS_F16 = 1 } hs_dtype;

typedef int32_t hs_status;
#define HS_OK 0
#define HS_EINVAL (-1)
#define HS_EHIP (-2)
#define HS_EUNSUPPORTED (-3)

#define HS_ABI_VERSION 1

/* ABI version of the loaded library (HS_ABI_VERSION it was built with). */
int32_t hs_abi_version(void);
/* Static name of a status code. */
const char* hs_status_string(hs_status status);
/* Message of the last failing call on this thread ("" if none). */
const char* hs_last_error(void);

/* ---------------------------------------------------------------------- */
/* Reference op surface (one export per GpuContext method on the path)      */

/* GpuContext::layernorm (engine/ops.rs:130-153; shaders/layernorm.wesl).
 * out[r, :] = (x[r, :] - mean) * rsqrt(var + eps) * w + b over `dim`, with
 * f32 statistics. The reference hardcodes eps = 1e-5 (engine/ops.rs:139);
 * here the caller passes it. out may equal x. Serves the block pre-norm
 * (dim 1024) and the head-major QK-norm (dim 64, rows S*H*T). */
hs_status hs_layernorm(hs_stream_t stream, hs_dtype dt, const void* x, const float* w,
                       const float* b, void* out, int64_t rows, int32_t dim, float eps);

/* GpuContext::gelu (engine/ops.rs:155-165; shaders/gelu.wesl): exact-erf
 * GELU 0.5*v*(1 + erf(v/sqrt(2))), erf by Abramowitz & Stegun 7.1.26.
 * out may equal x. */
hs_status hs_gelu(hs_stream_t stream, hs_dtype dt, const void* x, void* out, int64_t total);

/* GpuContext::residual_ls (engine/ops.rs:167-183; shaders/residual_ls.wesl):
 * out[i] = res[i] + gamma[i % dim] * x[i]. total must be a multiple of dim.
 * out may equal res or x. */
hs_status hs_residual_ls(hs_stream_t stream, hs_dtype dt, const void* res, const void* x,
                         const float* gamma, void* out, int64_t total, int32_t dim);

/* GpuContext::split_heads (engine/ops.rs:185-200; shaders/split_heads.wesl):
 * (S*T, H*D) token-major -> (S, H, T, D) head-major, an exact copy.
 * out must not overlap x. */
hs_status hs_split_heads(hs_stream_t stream, hs_dtype dt, const void* x, void* out, int32_t s,
                         int32_t t, int32_t h, int32_t d);

/* GpuContext::rope_apply (engine/ops.rs:202-223; shaders/rope_apply.wesl),
 * in place on head-major x (S, H, T, D), D even. Tables are f32
 * (T - prefix, D); token t >= prefix uses table row t - prefix:
 *   x[dp]     = x[dp] * cos[dp] - x[dp+D/2] * sin[dp]
 *   x[dp+D/2] = x[dp+D/2] * cos[D/2+dp] + x[dp] * sin[D/2+dp]
 * The first `prefix` tokens of every sequence are left untouched. */
hs_status hs_rope_apply(hs_stream_t stream, hs_dtype dt, void* x, const float* sin_tab,
                        const float* cos_tab, int32_t s, int32_t h, int32_t t, int32_t d,
                        int32_t prefix);

/* GpuContext::cast_to_f16 (engine/ops.rs:336-348; cast_f32_to_f16.wesl):
 * f32 -> f16, round to nearest even. out (f16) must not overlap x. */
hs_status hs_cast_f32_to_f16(hs_stream_t stream, const float* x, void* out, int64_t total);

/* GpuContext::copy_rows (engine/tensor.rs:146-160): copy n_rows rows of
 * row_bytes bytes from src row src_row to dst row dst_row (stream-ordered
 * device-to-device copy). Source and destination ranges must not overlap. */
hs_status hs_copy_rows(hs_stream_t stream, const void* src, int64_t src_row, void* dst,
                       int64_t dst_row, int64_t n_rows, int64_t row_bytes);

/* GpuContext::tiled_add (engine/ops.rs:374-389; shaders/tiled_add.wesl),
 * f32 only: out[i] = x[i] + table[i % block]; total a multiple of block.
 * out may equal x. */
hs_status hs_tiled_add(hs_stream_t stream, const float* x, const float* table, float* out,
                       int64_t total, int64_t block);

/* ---------------------------------------------------------------------- */
/* Fused per-layer ops (each replaces a run of reference dispatches)        */

/* split_heads + QK-norm + RoPE in one pass (model/block.rs:130-146:
 * split_heads, layernorm(q|k) over head_dim, rope_apply). Reads token-major
 * x_tok (S*T, H*D), writes head-major out_head (S, H, T, D). nw/nb (D) are
 * the QK-norm weight and bias; both NULL skips the norm (DINO blocks).
 * sin_tab/cos_tab (T - prefix, D) apply RoPE to tokens t >= prefix; both
 * NULL skips it (global-attention blocks, model/trunk.rs:123-125). With
 * norm and RoPE both off this is exactly hs_split_heads. out_head must not
 * overlap x_tok. */
hs_status hs_qknorm_rope(hs_stream_t stream, hs_dtype dt, const void* x_tok, const float* nw,
                         const float* nb, const float* sin_tab, const float* cos_tab,
                         void* out_head, int32_t s, int32_t t, int32_t h, int32_t d,
                         int32_t prefix, float eps);

/* hs_qknorm_rope on q and on k in one launch (the six dispatches of
 * model/block.rs:130-146): q_tok -> q_head with norm qn_w/qn_b, k_tok ->
 * k_head with kn_w/kn_b, both with the same shape, RoPE tables and prefix.
 * Either both norms are given or neither. Results are bit-identical to two
 * hs_qknorm_rope calls. No output may overlap an input or the other
 * output. */
hs_status hs_qknorm_rope_pair(hs_stream_t stream, hs_dtype dt, const void* q_tok,
                              const void* k_tok, const float* qn_w, const float* qn_b,
                              const float* kn_w, const float* kn_b, const float* sin_tab,
                              const float* cos_tab, void* q_head, void* k_head, int32_t s,
                              int32_t t, int32_t h, int32_t d, int32_t prefix, float eps);

/* fc1 bias epilogue + GELU (shaders/linear_wmma.wgsl:69-74 then
 * engine/ops.rs:155-165): out[r, c] = gelu(x[r, c] + bias[c]) over
 * (rows, cols); bias NULL is plain GELU. The sum stays in f32 and the
 * result rounds once (the reference's epilogue stores x + bias in the
 * storage type before its GELU dispatch; the difference is within the f16
 * parity tolerance). out may equal x. */
hs_status hs_bias_gelu(hs_stream_t stream, hs_dtype dt, const void* x, const float* bias,
                       void* out, int64_t rows, int32_t cols);

/* proj/fc2 bias epilogue + LayerScale + residual (linear_wmma.wgsl:69-74
 * then engine/ops.rs:167-183): out[r, c] = res[r, c] + gamma[c] * (x[r, c]
 * + bias[c]); bias NULL is plain residual_ls. out may equal res or x. */
hs_status hs_bias_ls_residual(hs_stream_t stream, hs_dtype dt, const void* res, const void* x,
                              const float* bias, const float* gamma, void* out, int64_t rows,
                              int32_t dim);

/* hs_bias_ls_residual, then GpuContext::layernorm (engine/ops.rs:130-153)
 * of its output, in one pass: the pre-norm block's residual_ls -> layernorm
 * pairs (model/block.rs:150-153, x1 into LN2; a block's output into the next
 * block's LN1, :128). out[r, c] = res[r, c] + gamma[c] * dt(x[r, c] +
 * bias[c]) stored in dt, as hs_bias_ls_residual; normed = layernorm(out,
 * ln_w, ln_b, eps) computed from out's stored values, as hs_layernorm. Both
 * are bit-identical to the two calls. bias may be NULL; ln_w, ln_b, gamma
 * (dim) f32. out may equal res or x; normed must not overlap res, x or
 * out. */
hs_status hs_bias_ls_residual_layernorm(hs_stream_t stream, hs_dtype dt, const void* res,
                                        const void* x, const float* bias, const float* gamma,
                                        const float* ln_w, const float* ln_b, void* out,
                                        void* normed, int64_t rows, int32_t dim, float eps);

/* Patch-token assembly (model/trunk.rs:68-85 with engine/ops.rs:337-348,
 * model/dino.rs:76-93; pos-embed add as shaders/tiled_add.wesl:23). Output
 * (S*T, D) in out_dt with T = 1 + R + P; for frame f and v = (f != 0 && n_var
 * == 2) ? 1 : 0:
 *   row f*T          = cam[v]                  (cam: (n_var, D), out_dt)
 *   rows f*T+1..+R   = reg[v*R .. v*R+R-1]     (reg: (n_var*R, D), out_dt)
 *   row f*T+1+R+p    = out_dt((patches[f*P+p] + patch_bias) + pos[p])
 * patches (S*P, D) are in patch_dt; patch_bias (D) and pos (P, D) are f32
 * and each may be NULL. The sums run in f32 in that order and round once.
 * cam/reg may be NULL only when R == 0 / never for cam. n_var is 1 or 2. */
hs_status hs_assemble_tokens(hs_stream_t stream, hs_dtype out_dt, const void* patches,
                             hs_dtype patch_dt, const float* patch_bias, const float* pos,
                             const void* cam, const void* reg, void* out, int32_t s, int32_t p,
                             int32_t r, int32_t d, int32_t n_var);

/* ---------------------------------------------------------------------- */
/* Trunk cache build and register-token gather/scatter                      */

/* GpuContext::concat_channels (engine/ops.rs:302-318;
 * shaders/concat_channels.wesl): a (rows, c1) ++ b (rows, c2) -> out
 * (rows, c1 + c2), exact. out must not overlap a or b. */
hs_status hs_concat_channels(hs_stream_t stream, hs_dtype dt, const void* a, const void* b,
                             void* out, int64_t rows, int32_t c1, int32_t c2);

/* GpuContext::cast_to_f32 (engine/ops.rs:321-334; shaders/cast_f16_to_f32.wesl):
 * f16 x -> f32 out, exact. */
hs_status hs_cast_f16_to_f32(hs_stream_t stream, const void* x, float* out, int64_t total);

/* Cache::build's per-group body (model/cache.rs:21-52): concat_channels of
 * the frame- and inter-block outputs, then cast to f32 (f16 inputs), in one
 * pass: out (rows, c1 + c2) f32 = [frame_out row | inter_out row]. The
 * reference streams frame groups to stay under wgpu's 2 GiB buffer cap; the
 * operation is row-independent, so any row range may be passed. */
hs_status hs_cache_build(hs_stream_t stream, hs_dtype in_dt, const void* frame_out,
                         const void* inter_out, float* out, int64_t rows, int32_t c1, int32_t c2);

/* n_blocks copy_rows calls in one launch (model/trunk.rs:103-116 gathers the
 * PREFIX rows of every frame with src_stride T, dst_stride PREFIX, and
 * scatters them back with the strides swapped): for j in [0, n_blocks), rows
 * [src_row0 + j*src_stride, + rows_per_block) of src go to rows
 * [dst_row0 + j*dst_stride, ...) of dst; rows are row_bytes wide. src and dst
 * must not overlap; strides must be at least rows_per_block. */
hs_status hs_copy_row_blocks(hs_stream_t stream, const void* src, int64_t src_row0,
                             int64_t src_stride, void* dst, int64_t dst_row0, int64_t dst_stride,
                             int64_t n_blocks, int64_t rows_per_block, int64_t row_bytes);

/* ---------------------------------------------------------------------- */
/* Linear layers (GEMM) with the trunk's epilogues fused                     */

/* GpuContext::linear (engine/ops.rs:81-128; shaders/linear_wmma.wgsl,
 * shaders/linear.wesl): out (m, n) = x (m, k) @ w (n, k)^T + bias (n),
 * accumulated in f32, stored in dt. bias (f32) may be NULL. out must not
 * overlap x or w. */
hs_status hs_linear(hs_stream_t stream, hs_dtype dt, const void* x, const void* w,
                    const float* bias, void* out, int64_t m, int32_t n, int32_t k);

/* linear(fc1, bias) then gelu (model/block.rs:172-176) in one kernel:
 * out = gelu(x @ w^T + bias), the sum kept in f32 and rounded once (as
 * hs_bias_gelu does). */
hs_status hs_linear_gelu(hs_stream_t stream, hs_dtype dt, const void* x, const void* w,
                         const float* bias, void* out, int64_t m, int32_t n, int32_t k);

/* linear(proj | fc2, bias) then residual_ls (model/block.rs:150-155) in one
 * kernel: out = res + gamma * dt(x @ w^T + bias), keeping the linear's
 * storage rounding. gamma (n) f32; res (m, n) in dt; out may equal res. */
hs_status hs_linear_ls_residual(hs_stream_t stream, hs_dtype dt, const void* x, const void* w,
                                const float* bias, const float* gamma, const void* res, void* out,
                                int64_t m, int32_t n, int32_t k);

/* The attention input projection of model/block.rs:128-146 in one kernel:
 * linear(x, w_qkv, b_qkv) with w_qkv (3*H*d, k) holding q | k | v stacked on
 * its output rows (the checkpoint's attn.qkv layout, which Block::load
 * splits), then split_heads (engine/ops.rs:185-200) of q, k and v into
 * head-major (S, H, T, d) outputs, QK-norm (layernorm over d, f32
 * statistics) and rotate-half RoPE (engine/ops.rs:202-223) of q and k.
 * Results are bit-identical to hs_linear followed by hs_qknorm_rope on each
 * third when H is 8, 16 or 32 (the head counts hs_qknorm_rope's row kernel
 * covers, whose head-vector code this shares), within one f16 ulp for
 * other H. qn_w/qn_b, kn_w/kn_b (d, f32) NULL = no QK-norm; sin/cos (T -
 * prefix, d) f32 NULL = no RoPE; b_qkv (3*H*d) f32 may be NULL. x is (S*T,
 * k). Fused kernels only: d == 64 and 16-byte aligned buffers with, in f16,
 * 3*H*64 % 256 == 0 and k % 64 == 0, in f32, 3*H*64 % 128 == 0 and k % 32
 * == 0; other shapes return HS_EUNSUPPORTED (run hs_linear then
 * hs_qknorm_rope). Outputs must not overlap x, w_qkv or each other. */
hs_status hs_linear_qkv_heads(hs_stream_t stream, hs_dtype dt, const void* x, const void* w_qkv,
                              const float* b_qkv, const float* qn_w, const float* qn_b,
                              const float* kn_w, const float* kn_b, const float* sin_tab,
                              const float* cos_tab, void* q_out, void* k_out, void* v_out,
                              int32_t S, int32_t T, int32_t H, int32_t d, int32_t k,
                              int32_t prefix, float eps);

/* ---------------------------------------------------------------------- */
/* LayerNorm fused into the linear layer after it (the pre-norm blocks'     */
/* layernorm -> linear pairs, model/block.rs:128-131 and 153, 172-174)       */

/* The statistics half of GpuContext::layernorm (engine/ops.rs:130-153):
 * stats[2 r] = mean of row r of x (rows, dim), stats[2 r + 1] = rsqrt(var +
 * eps), f32, from the kernel and arithmetic that hs_layernorm normalises
 * the same x with (bit-identical when hs_layernorm's buffers are 16-byte
 * aligned). stats is 8-byte aligned, 2 * rows floats, and must not overlap
 * x. */
hs_status hs_layernorm_stats(hs_stream_t stream, hs_dtype dt, const void* x, float* stats,
                             int64_t rows, int32_t dim, float eps);

/* GpuContext::layernorm (engine/ops.rs:130-153) then GpuContext::linear
 * (engine/ops.rs:81-128) as Block::forward pairs them (LN1 -> q|k|v,
 * model/block.rs:128-131): out (m, n) = dt(layernorm(x, ln_w, ln_b, eps)) @
 * w^T + bias, where each element of the normalised row is rounded to the
 * storage type exactly as hs_layernorm stores it (shaders/layernorm.wesl:76
 * stores Elem) before the product reads it. The normalised row never
 * reaches memory: each row's mean and rstd go to workspace (2 * m floats,
 * 8-byte aligned; it must not overlap x, w, bias, ln_w, ln_b or out), and
 * the product normalises its x tiles on the way to the matrix cores. With
 * 16-byte aligned buffers the result is bit-identical to hs_layernorm then
 * hs_linear. ln_w, ln_b (k) f32; bias (n) f32 may be NULL; k > 0. */
hs_status hs_linear_ln(hs_stream_t stream, hs_dtype dt, const void* x, const float* ln_w,
                       const float* ln_b, const void* w, const float* bias, float* workspace,
                       void* out, int64_t m, int32_t n, int32_t k, float eps);

/* hs_linear_ln then GELU (LN2 -> fc1 -> gelu, model/block.rs:153, 172-176):
 * out = dt(gelu(dt(layernorm(x)) @ w^T + bias)), the sum kept in f32 and
 * rounded once, as hs_linear_gelu. Bit-identical to hs_layernorm then
 * hs_linear_gelu under the same conditions as hs_linear_ln. */
hs_status hs_linear_ln_gelu(hs_stream_t stream, hs_dtype dt, const void* x, const float* ln_w,
                            const float* ln_b, const void* w, const float* bias, float* workspace,
                            void* out, int64_t m, int32_t n, int32_t k, float eps);

/* hs_linear_ln then the q|k|v heads epilogue of hs_linear_qkv_heads
 * (model/block.rs:128-146: LN1, the q|k|v projection, split_heads,
 * QK-norm, RoPE): bit-identical to hs_layernorm then hs_linear_qkv_heads
 * under the conditions of both. eps serves the LayerNorm and the QK-norm
 * (the block uses one). Same shape rules as hs_linear_qkv_heads (fast path
 * only, checked before anything is enqueued; ln_w, ln_b 16-byte aligned);
 * workspace as hs_linear_ln. */
hs_status hs_linear_ln_qkv_heads(hs_stream_t stream, hs_dtype dt, const void* x,
                                 const float* ln_w, const float* ln_b, const void* w_qkv,
                                 const float* b_qkv, const float* qn_w, const float* qn_b,
                                 const float* kn_w, const float* kn_b, const float* sin_tab,
                                 const float* cos_tab, float* workspace, void* q_out, void* k_out,
                                 void* v_out, int32_t S, int32_t T, int32_t H, int32_t d,
                                 int32_t k, int32_t prefix, float eps);

/* hs_linear_ln_gelu without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc); no counterpart in the reference. The row statistics go
 * to a 4 MiB array the library holds in each device's memory for the life
 * of the process, so m is at most 524,288 rows (HS_EINVAL beyond), and calls
 * that overlap on one device race on that array. It calls no allocating
 * routine. */
hs_status hs_linear_ln_gelu_noalloc(hs_stream_t stream, hs_dtype dt, const void* x,
                                    const float* ln_w, const float* ln_b, const void* w,
                                    const float* bias, void* out, int64_t m, int32_t n, int32_t k,
                                    float eps);

/* ---------------------------------------------------------------------- */
/* Attention                                                                */

/* GpuContext::attention (engine/ops.rs:225-253; shaders/attention.wesl):
 * non-causal softmax(q k^T / sqrt(D)) v for each of the S*H sequences of
 * head-major q, k, v (S, H, T, D); out is (S, H, T, D) in the same dtype.
 * Softmax statistics and accumulation are f32. D is 64 (f32 or f16) or 128
 * (f32 only), as the reference's kernel variants; other combinations return
 * HS_EUNSUPPORTED. out must not overlap q, k or v. */
hs_status hs_attention(hs_stream_t stream, hs_dtype dt, const void* q, const void* k,
                       const void* v, void* out, int32_t s, int32_t h, int32_t t, int32_t d);

/* GpuContext::attn_merge (engine/ops.rs:255-267; shaders/attn_merge.wesl):
 * (S, H, T, D) head-major -> (S*T, H*D) token-major, an exact copy. out must
 * not overlap x. */
hs_status hs_attn_merge(hs_stream_t stream, hs_dtype dt, const void* x, void* out, int32_t s,
                        int32_t h, int32_t t, int32_t d);

/* attention followed by attn_merge (model/block.rs:148-149) in one pass: the
 * same values as hs_attention, written token-major (S*T, H*D) into out, so
 * the head-major attention output never reaches memory. */
hs_status hs_attention_merged(hs_stream_t stream, hs_dtype dt, const void* q, const void* k,
                              const void* v, void* out, int32_t s, int32_t h, int32_t t,
                              int32_t d);

/* ---------------------------------------------------------------------- */
/* Host-side RoPE tables (computed once per session, as the reference does) */

/* rope::periods (engine/rope.rs:5-10): out16[i] = 100^(2i/32) in f32. */
void hs_rope_periods(float* out16);

/* rope::tables (engine/rope.rs:12-43), bit-exact: sin_out/cos_out are host
 * arrays of (h_p*w_p, 64) f32, rows in h-outer/w-inner patch order.
 * Channels [0,16) carry h-angles, [16,32) w-angles, [32,64) repeat [0,32);
 * angle = (2*pi * (2*((i+0.5)/max(h_p,w_p)) - 1)) / periods16[k]. */
hs_status hs_rope_tables(const float* periods16, int32_t h_p, int32_t w_p, float* sin_out,
                         float* cos_out);

#ifdef __cplusplus
}
#endif

#endif /* HEADSHOT_HIP_H */
