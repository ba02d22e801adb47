//! Raw bindings of `include/headshot_hip.h` (libheadshot_hip.so) and the
//! few HIP runtime calls the safe layer needs for memory and streams.
//!
//! The `headshot_hip` block mirrors the header one declaration per export,
//! with the header's argument names and C types mapped as
//! `hs_stream_t` -> [`HsStream`], `hs_dtype` -> [`HsDtype`], `hs_status` ->
//! [`HsStatus`], `int32_t` -> `i32`, `int64_t` -> `i64`, `float` -> `f32`,
//! `const T*` -> `*const T`, `T*` -> `*mut T`, `void` -> `c_void`.
#![allow(non_camel_case_types, non_snake_case)]

use std::os::raw::{c_char, c_int, c_uint, c_void};

/// `hipStream_t`; null is the default stream.
pub type HsStream = *mut c_void;
/// `hs_dtype`: storage type of activations.
pub type HsDtype = i32;
/// `hs_status`: 0 or a negative error code.
pub type HsStatus = i32;

pub const HS_F32: HsDtype = 0;
pub const HS_F16: HsDtype = 1;

pub const HS_OK: HsStatus = 0;
pub const HS_EINVAL: HsStatus = -1;
pub const HS_EHIP: HsStatus = -2;
pub const HS_EUNSUPPORTED: HsStatus = -3;

pub const HS_ABI_VERSION: i32 = 1;

#[link(name = "headshot_hip")]
extern "C" {
    pub fn hs_abi_version() -> i32;
    pub fn hs_status_string(status: HsStatus) -> *const c_char;
    pub fn hs_last_error() -> *const c_char;

    // reference op surface (GpuContext methods)
    pub fn hs_layernorm(stream: HsStream, dt: HsDtype, x: *const c_void, w: *const f32,
                        b: *const f32, out: *mut c_void, rows: i64, dim: i32, eps: f32)
                        -> HsStatus;
    pub fn hs_gelu(stream: HsStream, dt: HsDtype, x: *const c_void, out: *mut c_void,
                   total: i64) -> HsStatus;
    pub fn hs_residual_ls(stream: HsStream, dt: HsDtype, res: *const c_void, x: *const c_void,
                          gamma: *const f32, out: *mut c_void, total: i64, dim: i32)
                          -> HsStatus;
    pub fn hs_split_heads(stream: HsStream, dt: HsDtype, x: *const c_void, out: *mut c_void,
                          s: i32, t: i32, h: i32, d: i32) -> HsStatus;
    pub fn hs_rope_apply(stream: HsStream, dt: HsDtype, x: *mut c_void, sin_tab: *const f32,
                         cos_tab: *const f32, s: i32, h: i32, t: i32, d: i32, prefix: i32)
                         -> HsStatus;
    pub fn hs_cast_f32_to_f16(stream: HsStream, x: *const f32, out: *mut c_void, total: i64)
                              -> HsStatus;
    pub fn hs_copy_rows(stream: HsStream, src: *const c_void, src_row: i64, dst: *mut c_void,
                        dst_row: i64, n_rows: i64, row_bytes: i64) -> HsStatus;
    pub fn hs_tiled_add(stream: HsStream, x: *const f32, table: *const f32, out: *mut f32,
                        total: i64, block: i64) -> HsStatus;

    // fused per-layer ops
    pub fn hs_qknorm_rope(stream: HsStream, dt: HsDtype, x_tok: *const c_void, nw: *const f32,
                          nb: *const f32, sin_tab: *const f32, cos_tab: *const f32,
                          out_head: *mut c_void, s: i32, t: i32, h: i32, d: i32, prefix: i32,
                          eps: f32) -> HsStatus;
    pub fn hs_qknorm_rope_pair(stream: HsStream, dt: HsDtype, q_tok: *const c_void,
                               k_tok: *const c_void, qn_w: *const f32, qn_b: *const f32,
                               kn_w: *const f32, kn_b: *const f32, sin_tab: *const f32,
                               cos_tab: *const f32, q_head: *mut c_void, k_head: *mut c_void,
                               s: i32, t: i32, h: i32, d: i32, prefix: i32, eps: f32)
                               -> HsStatus;
    pub fn hs_bias_gelu(stream: HsStream, dt: HsDtype, x: *const c_void, bias: *const f32,
                        out: *mut c_void, rows: i64, cols: i32) -> HsStatus;
    pub fn hs_bias_ls_residual(stream: HsStream, dt: HsDtype, res: *const c_void,
                               x: *const c_void, bias: *const f32, gamma: *const f32,
                               out: *mut c_void, rows: i64, dim: i32) -> HsStatus;
    pub fn hs_bias_ls_residual_layernorm(stream: HsStream, dt: HsDtype, res: *const c_void,
                                         x: *const c_void, bias: *const f32, gamma: *const f32,
                                         ln_w: *const f32, ln_b: *const f32, out: *mut c_void,
                                         normed: *mut c_void, rows: i64, dim: i32, eps: f32)
                                         -> HsStatus;
    pub fn hs_assemble_tokens(stream: HsStream, out_dt: HsDtype, patches: *const c_void,
                              patch_dt: HsDtype, patch_bias: *const f32, pos: *const f32,
                              cam: *const c_void, reg: *const c_void, out: *mut c_void, s: i32,
                              p: i32, r: i32, d: i32, n_var: i32) -> HsStatus;

    // trunk cache build and register gather/scatter
    pub fn hs_concat_channels(stream: HsStream, dt: HsDtype, a: *const c_void, b: *const c_void,
                              out: *mut c_void, rows: i64, c1: i32, c2: i32) -> HsStatus;
    pub fn hs_cast_f16_to_f32(stream: HsStream, x: *const c_void, out: *mut f32, total: i64)
                              -> HsStatus;
    pub fn hs_cache_build(stream: HsStream, in_dt: HsDtype, frame_out: *const c_void,
                          inter_out: *const c_void, out: *mut f32, rows: i64, c1: i32, c2: i32)
                          -> HsStatus;
    pub fn hs_copy_row_blocks(stream: HsStream, src: *const c_void, src_row0: i64,
                              src_stride: i64, dst: *mut c_void, dst_row0: i64, dst_stride: i64,
                              n_blocks: i64, rows_per_block: i64, row_bytes: i64) -> HsStatus;

    // linear layers with fused epilogues
    pub fn hs_linear(stream: HsStream, dt: HsDtype, x: *const c_void, w: *const c_void,
                     bias: *const f32, out: *mut c_void, m: i64, n: i32, k: i32) -> HsStatus;
    pub fn hs_linear_gelu(stream: HsStream, dt: HsDtype, x: *const c_void, w: *const c_void,
                          bias: *const f32, out: *mut c_void, m: i64, n: i32, k: i32)
                          -> HsStatus;
    pub fn hs_linear_ls_residual(stream: HsStream, dt: HsDtype, x: *const c_void,
                                 w: *const c_void, bias: *const f32, gamma: *const f32,
                                 res: *const c_void, out: *mut c_void, m: i64, n: i32, k: i32)
                                 -> HsStatus;
    pub fn hs_linear_qkv_heads(stream: HsStream, dt: HsDtype, x: *const c_void,
                               w_qkv: *const c_void, b_qkv: *const f32, qn_w: *const f32,
                               qn_b: *const f32, kn_w: *const f32, kn_b: *const f32,
                               sin_tab: *const f32, cos_tab: *const f32, q_out: *mut c_void,
                               k_out: *mut c_void, v_out: *mut c_void, S: i32, T: i32, H: i32,
                               d: i32, k: i32, prefix: i32, eps: f32) -> HsStatus;

    // LayerNorm as the prologue of the linear layer after it
    pub fn hs_layernorm_stats(stream: HsStream, dt: HsDtype, x: *const c_void, stats: *mut f32,
                              rows: i64, dim: i32, eps: f32) -> HsStatus;
    pub fn hs_linear_ln(stream: HsStream, dt: HsDtype, x: *const c_void, ln_w: *const f32,
                        ln_b: *const f32, w: *const c_void, bias: *const f32,
                        workspace: *mut f32, out: *mut c_void, m: i64, n: i32, k: i32, eps: f32)
                        -> HsStatus;
    pub fn hs_linear_ln_gelu(stream: HsStream, dt: HsDtype, x: *const c_void, ln_w: *const f32,
                             ln_b: *const f32, w: *const c_void, bias: *const f32,
                             workspace: *mut f32, out: *mut c_void, m: i64, n: i32, k: i32,
                             eps: f32) -> HsStatus;
    pub fn hs_linear_ln_qkv_heads(stream: HsStream, dt: HsDtype, x: *const c_void,
                                  ln_w: *const f32, ln_b: *const f32, w_qkv: *const c_void,
                                  b_qkv: *const f32, qn_w: *const f32, qn_b: *const f32,
                                  kn_w: *const f32, kn_b: *const f32, sin_tab: *const f32,
                                  cos_tab: *const f32, workspace: *mut f32, q_out: *mut c_void,
                                  k_out: *mut c_void, v_out: *mut c_void, S: i32, T: i32, H: i32,
                                  d: i32, k: i32, prefix: i32, eps: f32) -> HsStatus;
    pub fn hs_linear_ln_gelu_noalloc(stream: HsStream, dt: HsDtype, x: *const c_void,
                                     ln_w: *const f32, ln_b: *const f32, w: *const c_void,
                                     bias: *const f32, out: *mut c_void, m: i64, n: i32, k: i32,
                                     eps: f32) -> HsStatus;

    // attention
    pub fn hs_attention(stream: HsStream, dt: HsDtype, q: *const c_void, k: *const c_void,
                        v: *const c_void, out: *mut c_void, s: i32, h: i32, t: i32, d: i32)
                        -> HsStatus;
    pub fn hs_attn_merge(stream: HsStream, dt: HsDtype, x: *const c_void, out: *mut c_void,
                         s: i32, h: i32, t: i32, d: i32) -> HsStatus;
    pub fn hs_attention_merged(stream: HsStream, dt: HsDtype, q: *const c_void,
                               k: *const c_void, v: *const c_void, out: *mut c_void, s: i32,
                               h: i32, t: i32, d: i32) -> HsStatus;

    // host-side RoPE tables
    pub fn hs_rope_periods(out16: *mut f32);
    pub fn hs_rope_tables(periods16: *const f32, h_p: i32, w_p: i32, sin_out: *mut f32,
                          cos_out: *mut f32) -> HsStatus;
}

/// `hipMemcpyKind` values used here.
pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

#[link(name = "amdhip64")]
extern "C" {
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> c_int;
    pub fn hipFree(ptr: *mut c_void) -> c_int;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> c_int;
    pub fn hipStreamCreateWithFlags(stream: *mut HsStream, flags: c_uint) -> c_int;
    pub fn hipStreamDestroy(stream: HsStream) -> c_int;
    pub fn hipStreamSynchronize(stream: HsStream) -> c_int;
    pub fn hipGetErrorString(err: c_int) -> *const c_char;
}
