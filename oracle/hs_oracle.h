/*
 * hs_oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement (plain C, f32 arithmetic, no FMA contraction) of headshot's
 * per-layer WGSL kernels and of its host-side RoPE tables, used as the
 * checker for the HIP library. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never links it.
 *
 * Storage dtypes mirror the reference's Elem alias: 0 = f32, 1 = f16 (IEEE
 * binary16 bits in uint16_t). Every kernel reads Elem, computes in f32 and
 * writes Elem, rounding to nearest-even exactly where the reference stores.
 *
 * Pins (what independently checks each function) are listed in oracle.py.
 */
#ifndef HS_ORACLE_H
#define HS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_F16 = 1 };

/* binary16 <-> binary32, round-to-nearest-even (half 2.7.1 f16::from_f32). */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
void or_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* crates/headshot-server/src/engine/rope.rs:8-10 */
void or_rope_periods(float out16[16]);
/* crates/headshot-server/src/engine/rope.rs:18-43; sin/cos are (h_p*w_p, 64). */
void or_rope_tables(const float* periods16, int32_t h_p, int32_t w_p, float* sin_out,
                    float* cos_out);
/* crates/headshot-server/src/engine/rope.rs:47-54 */
void or_rope_apply_cpu(const float* x64, const float* sin_tab, const float* cos_tab,
                       int64_t table_row, float* out64);

/* shaders/layernorm.wesl:27-78 (256-way strided partials + LDS tree). */
void or_layernorm(int dt, const void* x, const float* w, const float* b, void* out,
                  int64_t rows, int32_t dim, float eps);
/* shaders/split_heads.wesl:22-42: (S*T, H*D) -> (S, H, T, D). */
void or_split_heads(int dt, const void* x, void* out, int32_t s, int32_t t, int32_t h, int32_t d);
/* shaders/attn_merge.wesl: (S, H, T, D) -> (S*T, H*D). */
void or_attn_merge(int dt, const void* x, void* out, int32_t s, int32_t t, int32_t h, int32_t d);
/* shaders/linear.wesl:29-68: out = x @ w^T [+ bias], f32 accumulation in k
 * order; rows_idx (nrows) selects rows of x (NULL: all m). */
void or_linear(int dt, const void* x, const void* w, const float* bias, void* out, int64_t m,
               int32_t n, int32_t k, const int64_t* rows_idx, int64_t nrows);
/* shaders/concat_channels.wesl: a (rows, c1) ++ b (rows, c2). */
void or_concat_channels(int dt, const void* a, const void* b, void* out, int64_t rows,
                        int32_t c1, int32_t c2);
/* shaders/cast_f16_to_f32.wesl */
void or_cast_f16_to_f32(const uint16_t* x, float* out, int64_t total);
/* model/cache.rs:37-44: concat_channels, then cast_to_f32 for f16 inputs. */
void or_cache_build(int dt, const void* frame_out, const void* inter_out, float* out,
                    int64_t rows, int32_t c1, int32_t c2);
/* shaders/attention.wesl:36-88 (engine/ops.rs:228-253): head-major q, k, v
 * (S, H, T, D), D a multiple of 4 up to 128, scale 1/sqrt(D). Computes the
 * queries q_idx[0..nq) (q_idx NULL: all T) of every sequence into out
 * (S*H, nq, D). */
void or_attention(int dt, const void* q, const void* k, const void* v, void* out, int32_t s,
                  int32_t h, int32_t t, int32_t d, const int32_t* q_idx, int32_t nq);
/* shaders/rope_apply.wesl:30-57, in place on (S, H, T, D). */
void or_rope_apply(int dt, void* x, const float* sin_tab, const float* cos_tab, int32_t s,
                   int32_t h, int32_t t, int32_t d, int32_t prefix);
/* shaders/gelu.wesl:18-27 */
float or_erf_as(float v);
/* shaders/gelu.wesl:29-40 */
void or_gelu(int dt, const void* x, void* out, int64_t total);
/* shaders/residual_ls.wesl:20-30 */
void or_residual_ls(int dt, const void* res, const void* x, const float* gamma, void* out,
                    int64_t total, int32_t dim);
/* Bias epilogue of linear: shaders/linear_wmma.wgsl:69-74, shaders/linear.wesl:57-61. */
void or_add_bias(int dt, const void* x, const float* bias, void* out, int64_t rows, int32_t cols);
/* shaders/cast_f32_to_f16.wesl:14-24 */
void or_cast_f32_to_f16(const float* x, uint16_t* out, int64_t total);
/* shaders/tiled_add.wesl:15-25 (f32 only in the reference) */
void or_tiled_add(const float* x, const float* table, float* out, int64_t total, int64_t block);

/*
 * Composites: the reference's unfused op sequence for each fused operation,
 * with storage rounding after every reference dispatch.
 */
/* split_heads -> [layernorm(d) if nw] -> [rope_apply if sin_tab]
 * (model/block.rs:130-146). */
void or_qknorm_rope(int dt, const void* x_tok, const float* nw, const float* nb,
                    const float* sin_tab, const float* cos_tab, void* out_head, int32_t s,
                    int32_t t, int32_t h, int32_t d, int32_t prefix, float eps);
/* [bias epilogue] -> gelu (model/block.rs:173-174). round_bias = 1 stores
 * x + bias in the storage type first, as the reference's GEMM epilogue does;
 * 0 keeps it in f32 (the fused operation's single-rounding semantics). */
void or_bias_gelu(int dt, const void* x, const float* bias, void* out, int64_t rows, int32_t cols,
                  int round_bias);
/* [bias epilogue] -> residual_ls (model/block.rs:150-151, 154-155). */
void or_bias_ls_residual(int dt, const void* res, const void* x, const float* bias,
                         const float* gamma, void* out, int64_t rows, int32_t dim);
/* Patch rows: [bias epilogue in patch dtype] -> [tiled_add pos (P,D)] ->
 * cast to out dtype; then copy_rows of [camera[v], register[v*R..], patches]
 * per frame with v = (frame != 0) when n_var == 2 (model/trunk.rs:68-85,
 * model/dino.rs:76-93). cam/reg are in the out dtype. */
void or_assemble_tokens(int out_dt, const void* patches, int patch_dt, const float* patch_bias,
                        const float* pos, const void* cam, const void* reg, void* out, int32_t s,
                        int32_t p, int32_t r, int32_t d, int32_t n_var);

/* One pre-norm block's per-layer op sequence as the reference dispatches it
 * (model/block.rs:118-159 minus GEMMs and attention): used by bench.py's
 * CPU baseline. Buffers are caller-owned; see oracle.py for the layout. */
void or_block_ops(int dt, const void* x, const float* ln1_w, const float* ln1_b,
                  const void* q_raw, const void* k_raw, const float* qn_w, const float* qn_b,
                  const float* kn_w, const float* kn_b, const float* sin_tab,
                  const float* cos_tab, int32_t prefix, const void* proj_raw,
                  const float* proj_b, const float* ls1, const float* ln2_w, const float* ln2_b,
                  const void* fc1_raw,
                  const float* fc1_b, const void* fc2_raw, const float* fc2_b,
                  const float* ls2, void* normed, void* q_head, void* k_head, void* x1,
                  void* normed2, void* act, void* x_out, int32_t s, int32_t t, int32_t dim,
                  int32_t heads, int32_t hidden, float eps);

/* Number of OpenMP threads the oracle runs with (1 when built without). */
int or_num_threads(void);
void or_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
