//! headshot-hip: headshot-server's per-layer op surface on MI355X.
//!
//! [`HipContext`] keeps the method names, argument meaning and panics of the
//! reference's `GpuContext` (crates/headshot-server/src/engine/ops.rs,
//! engine/tensor.rs) for the ops that run between the aggregator's GEMMs
//! and attention, plus the fused ops that replace runs of them. Every method
//! enqueues one libheadshot_hip call (hand-written gfx950 kernels) on the
//! context's HIP stream. As in the reference, every op except `rope_apply`
//! and `copy_rows` allocates and returns a new [`HipTensor`]; inputs are
//! borrowed, and contract violations panic (the library validates first and
//! enqueues nothing on a failure; its message becomes the panic text).
//!
//! Norm weights, biases, LayerScale gammas, positional and RoPE tables are
//! f32 tensors (engine/ops.rs:5-8); activations are f32 or f16 storage with
//! f32 arithmetic.

pub mod ffi;

use std::ffi::CStr;
use std::os::raw::c_void;
use std::ptr;

use half::f16;

/// Storage type of a tensor (the reference's `Dtype`, engine/tensor.rs:12-25).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Dtype {
    F32,
    F16,
}

impl Dtype {
    pub fn size(self) -> usize {
        match self {
            Dtype::F32 => 4,
            Dtype::F16 => 2,
        }
    }

    fn raw(self) -> ffi::HsDtype {
        match self {
            Dtype::F32 => ffi::HS_F32,
            Dtype::F16 => ffi::HS_F16,
        }
    }
}

fn hip_check(err: i32, what: &str) {
    if err != 0 {
        let msg = unsafe { CStr::from_ptr(ffi::hipGetErrorString(err)) };
        panic!("{what}: {}", msg.to_string_lossy());
    }
}

/// Turns a library status into the reference's behaviour: panic on any
/// failure, with the library's message.
fn check(status: ffi::HsStatus, op: &str) {
    if status != ffi::HS_OK {
        let (name, msg) = unsafe {
            (CStr::from_ptr(ffi::hs_status_string(status)), CStr::from_ptr(ffi::hs_last_error()))
        };
        panic!("{op}: {} ({})", msg.to_string_lossy(), name.to_string_lossy());
    }
}

/// A device tensor: `hipMalloc` on creation, `hipFree` on drop (hipFree
/// waits for the device's outstanding work first, so a buffer is reclaimed
/// only after the kernels using it have run, as engine/mod.rs:69-84 does
/// for wgpu buffers).
pub struct HipTensor {
    ptr: *mut c_void,
    pub shape: Vec<usize>,
    pub dtype: Dtype,
}

impl HipTensor {
    fn alloc(shape: &[usize], dtype: Dtype) -> HipTensor {
        let bytes = shape.iter().product::<usize>() * dtype.size();
        let mut p = ptr::null_mut();
        if bytes > 0 {
            hip_check(unsafe { ffi::hipMalloc(&mut p, bytes) }, "hipMalloc");
        }
        HipTensor { ptr: p, shape: shape.to_vec(), dtype }
    }

    pub fn len(&self) -> usize {
        self.shape.iter().product()
    }

    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }

    pub fn byte_len(&self) -> usize {
        self.len() * self.dtype.size()
    }

    /// Width of one row of the last dimension in bytes (engine/tensor.rs:48).
    pub fn row_bytes(&self) -> usize {
        self.shape.last().copied().unwrap_or(0) * self.dtype.size()
    }

    /// Same buffer, new shape of the same length (engine/tensor.rs:53).
    pub fn reshaped(mut self, shape: &[usize]) -> HipTensor {
        assert_eq!(shape.iter().product::<usize>(), self.len(), "reshape length");
        self.shape = shape.to_vec();
        self
    }

    fn cptr(&self) -> *const c_void {
        self.ptr
    }

    fn mptr(&self) -> *mut c_void {
        self.ptr
    }

    fn f32p(&self, what: &str) -> *const f32 {
        assert_eq!(self.dtype, Dtype::F32, "{what} must be f32");
        self.ptr as *const f32
    }

    fn dims(&self) -> (usize, usize) {
        let dim = *self.shape.last().expect("tensor needs a shape");
        (if dim == 0 { 0 } else { self.len() / dim }, dim)
    }
}

impl Drop for HipTensor {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe {
                ffi::hipFree(self.ptr);
            }
        }
    }
}

/// RoPE tables for a frame-block call: (T - prefix, 64) f32 sin and cos and
/// the number of leading tokens left unrotated (model/block.rs:143-146).
pub struct Rope<'a> {
    pub sin: &'a HipTensor,
    pub cos: &'a HipTensor,
    pub prefix: usize,
}

fn opt_f32(t: Option<&HipTensor>, n: usize, what: &str) -> *const f32 {
    match t {
        None => ptr::null(),
        Some(t) => {
            assert_eq!(t.len(), n, "{what} length");
            t.f32p(what)
        }
    }
}

fn i32_of(v: usize, what: &str) -> i32 {
    i32::try_from(v).unwrap_or_else(|_| panic!("{what} {v} exceeds i32"))
}

/// One device's op surface on one HIP stream.
pub struct HipContext {
    stream: ffi::HsStream,
}

// The stream handle is only used through stream-ordered library calls.
unsafe impl Send for HipContext {}
unsafe impl Sync for HipContext {}

impl Default for HipContext {
    fn default() -> Self {
        Self::new()
    }
}

impl Drop for HipContext {
    fn drop(&mut self) {
        unsafe {
            ffi::hipStreamSynchronize(self.stream);
            ffi::hipStreamDestroy(self.stream);
        }
    }
}

impl HipContext {
    /// A context on a new non-blocking stream of the current device (default
    /// priority).
    pub fn new() -> HipContext {
        let got = unsafe { ffi::hs_abi_version() };
        assert_eq!(got, ffi::HS_ABI_VERSION, "libheadshot_hip ABI mismatch");
        let mut stream = ptr::null_mut();
        hip_check(unsafe { ffi::hipStreamCreateWithFlags(&mut stream, 1) }, "hipStreamCreate");
        HipContext { stream }
    }

    /// Waits for every op enqueued so far.
    pub fn flush(&self) {
        hip_check(unsafe { ffi::hipStreamSynchronize(self.stream) }, "hipStreamSynchronize");
    }

    // ------------------------------------------------------------- tensors

    /// engine/tensor.rs:132-141: an uninitialised device tensor.
    pub fn empty_typed(&self, shape: &[usize], dtype: Dtype) -> HipTensor {
        HipTensor::alloc(shape, dtype)
    }

    pub fn empty(&self, shape: &[usize]) -> HipTensor {
        self.empty_typed(shape, Dtype::F32)
    }

    /// engine/tensor.rs:71-91: upload f32 data as `dtype` storage (f16 by
    /// round-to-nearest-even).
    pub fn tensor_from_f32(&self, shape: &[usize], data: &[f32], dtype: Dtype) -> HipTensor {
        assert_eq!(data.len(), shape.iter().product::<usize>(), "shape/data mismatch");
        let t = HipTensor::alloc(shape, dtype);
        self.flush();
        match dtype {
            Dtype::F32 => upload(&t, data.as_ptr() as *const c_void),
            Dtype::F16 => {
                let halves: Vec<f16> = data.iter().map(|&v| f16::from_f32(v)).collect();
                upload(&t, halves.as_ptr() as *const c_void)
            }
        }
        t
    }

    pub fn tensor_from_slice(&self, shape: &[usize], data: &[f32]) -> HipTensor {
        self.tensor_from_f32(shape, data, Dtype::F32)
    }

    /// engine/tensor.rs:98-115: raw f16 bits (weight loading).
    pub fn tensor_from_f16_bits(&self, shape: &[usize], data: &[f16]) -> HipTensor {
        assert_eq!(data.len(), shape.iter().product::<usize>(), "shape/data mismatch");
        let t = HipTensor::alloc(shape, Dtype::F16);
        self.flush();
        upload(&t, data.as_ptr() as *const c_void);
        t
    }

    /// engine/tensor.rs:162-198: waits for pending work, reads back as f32.
    pub fn download(&self, t: &HipTensor) -> Vec<f32> {
        self.flush();
        match t.dtype {
            Dtype::F32 => {
                let mut v = vec![0f32; t.len()];
                download(t, v.as_mut_ptr() as *mut c_void);
                v
            }
            Dtype::F16 => {
                let mut v = vec![f16::ZERO; t.len()];
                download(t, v.as_mut_ptr() as *mut c_void);
                v.iter().map(|h| h.to_f32()).collect()
            }
        }
    }

    /// engine/tensor.rs:146-160: copy `n_rows` rows of the last dimension.
    pub fn copy_rows(&self, src: &HipTensor, src_row: usize, dst: &HipTensor, dst_row: usize,
                     n_rows: usize) {
        assert_eq!(src.dtype, dst.dtype, "copy_rows dtype");
        assert_eq!(src.row_bytes(), dst.row_bytes(), "copy_rows row width");
        let row = src.row_bytes();
        assert!((src_row + n_rows) * row <= src.byte_len(), "copy_rows src rows");
        assert!((dst_row + n_rows) * row <= dst.byte_len(), "copy_rows dst rows");
        check(unsafe {
            ffi::hs_copy_rows(self.stream, src.cptr(), src_row as i64, dst.mptr(),
                              dst_row as i64, n_rows as i64, row as i64)
        }, "copy_rows");
    }

    // ------------------------------------------------------- reference ops

    /// engine/ops.rs:81-128: `x (m, k) @ weight (n, k)^T [+ bias]`.
    pub fn linear(&self, x: &HipTensor, weight: &HipTensor, bias: Option<&HipTensor>) -> HipTensor {
        let (m, k) = x.dims();
        let (n, wk) = weight.dims();
        assert_eq!(wk, k, "linear weight k");
        assert_eq!(weight.dtype, x.dtype, "linear weight dtype");
        let out = self.empty_typed(&[m, n], x.dtype);
        check(unsafe {
            ffi::hs_linear(self.stream, x.dtype.raw(), x.cptr(), weight.cptr(),
                           opt_f32(bias, n, "bias"), out.mptr(), m as i64, i32_of(n, "n"),
                           i32_of(k, "k"))
        }, "linear");
        out
    }

    /// engine/ops.rs:130-153 (eps 1e-5 as there).
    pub fn layernorm(&self, x: &HipTensor, weight: &HipTensor, bias: &HipTensor) -> HipTensor {
        self.layernorm_eps(x, weight, bias, 1e-5)
    }

    /// `layernorm` with an explicit eps (the benchmark configs use 1e-6).
    pub fn layernorm_eps(&self, x: &HipTensor, weight: &HipTensor, bias: &HipTensor,
                         eps: f32) -> HipTensor {
        let (rows, dim) = x.dims();
        assert_eq!(weight.len(), dim, "norm weight len");
        assert_eq!(bias.len(), dim, "norm bias len");
        let out = self.empty_typed(&x.shape, x.dtype);
        check(unsafe {
            ffi::hs_layernorm(self.stream, x.dtype.raw(), x.cptr(), weight.f32p("norm weight"),
                              bias.f32p("norm bias"), out.mptr(), rows as i64,
                              i32_of(dim, "dim"), eps)
        }, "layernorm");
        out
    }

    /// engine/ops.rs:155-165.
    pub fn gelu(&self, x: &HipTensor) -> HipTensor {
        let out = self.empty_typed(&x.shape, x.dtype);
        check(unsafe {
            ffi::hs_gelu(self.stream, x.dtype.raw(), x.cptr(), out.mptr(), x.len() as i64)
        }, "gelu");
        out
    }

    /// engine/ops.rs:167-183: `res + gamma * x`.
    pub fn residual_ls(&self, res: &HipTensor, x: &HipTensor, gamma: &HipTensor) -> HipTensor {
        assert_eq!(res.len(), x.len(), "residual_ls length");
        assert_eq!(res.dtype, x.dtype, "residual_ls dtype");
        let out = self.empty_typed(&res.shape, x.dtype);
        check(unsafe {
            ffi::hs_residual_ls(self.stream, x.dtype.raw(), res.cptr(), x.cptr(),
                                gamma.f32p("gamma"), out.mptr(), x.len() as i64,
                                i32_of(gamma.len(), "dim"))
        }, "residual_ls");
        out
    }

    /// engine/ops.rs:185-200: (S*T, H*D) -> (S, H, T, D).
    pub fn split_heads(&self, x: &HipTensor, s: usize, t: usize, h: usize, d: usize) -> HipTensor {
        assert_eq!(x.len(), s * t * h * d, "split_heads size");
        let out = self.empty_typed(&[s, h, t, d], x.dtype);
        check(unsafe {
            ffi::hs_split_heads(self.stream, x.dtype.raw(), x.cptr(), out.mptr(), i32_of(s, "s"),
                                i32_of(t, "t"), i32_of(h, "h"), i32_of(d, "d"))
        }, "split_heads");
        out
    }

    /// engine/ops.rs:202-223: in place on (S, H, T, D).
    pub fn rope_apply(&self, x: &HipTensor, sin: &HipTensor, cos: &HipTensor, prefix: usize) {
        let [s, h, t, d] = x.shape[..] else { panic!("rope_apply wants (S,H,T,D)") };
        assert!(prefix <= t, "rope prefix");
        assert_eq!(sin.len(), (t - prefix) * d, "rope table size");
        assert_eq!(cos.len(), sin.len(), "rope table size");
        check(unsafe {
            ffi::hs_rope_apply(self.stream, x.dtype.raw(), x.mptr(), sin.f32p("sin"),
                               cos.f32p("cos"), i32_of(s, "s"), i32_of(h, "h"), i32_of(t, "t"),
                               i32_of(d, "d"), i32_of(prefix, "prefix"))
        }, "rope_apply");
    }

    /// engine/ops.rs:225-253: non-causal attention over head-major q, k, v.
    pub fn attention(&self, q: &HipTensor, k: &HipTensor, v: &HipTensor) -> HipTensor {
        let [s, h, t, d] = q.shape[..] else { panic!("attention wants (S,H,T,D)") };
        assert_eq!(q.shape, k.shape, "attention k shape");
        assert_eq!(q.shape, v.shape, "attention v shape");
        let out = self.empty_typed(&q.shape, q.dtype);
        check(unsafe {
            ffi::hs_attention(self.stream, q.dtype.raw(), q.cptr(), k.cptr(), v.cptr(),
                              out.mptr(), i32_of(s, "s"), i32_of(h, "h"), i32_of(t, "t"),
                              i32_of(d, "d"))
        }, "attention");
        out
    }

    /// engine/ops.rs:255-267: (S, H, T, D) -> (S*T, H*D).
    pub fn attn_merge(&self, x: &HipTensor) -> HipTensor {
        let [s, h, t, d] = x.shape[..] else { panic!("attn_merge wants (S,H,T,D)") };
        let out = self.empty_typed(&[s * t, h * d], x.dtype);
        check(unsafe {
            ffi::hs_attn_merge(self.stream, x.dtype.raw(), x.cptr(), out.mptr(), i32_of(s, "s"),
                               i32_of(h, "h"), i32_of(t, "t"), i32_of(d, "d"))
        }, "attn_merge");
        out
    }

    /// engine/ops.rs:302-318: a (rows, c1) ++ b (rows, c2).
    pub fn concat_channels(&self, a: &HipTensor, b: &HipTensor) -> HipTensor {
        let (rows, c1) = a.dims();
        let (rows_b, c2) = b.dims();
        assert_eq!(rows, rows_b, "concat_channels rows");
        assert_eq!(a.dtype, b.dtype, "concat_channels dtype");
        let out = self.empty_typed(&[rows, c1 + c2], a.dtype);
        check(unsafe {
            ffi::hs_concat_channels(self.stream, a.dtype.raw(), a.cptr(), b.cptr(), out.mptr(),
                                    rows as i64, i32_of(c1, "c1"), i32_of(c2, "c2"))
        }, "concat_channels");
        out
    }

    /// engine/ops.rs:321-334: f16 -> f32.
    pub fn cast_to_f32(&self, x: &HipTensor) -> HipTensor {
        assert_eq!(x.dtype, Dtype::F16, "cast_to_f32 wants f16");
        let out = self.empty_typed(&x.shape, Dtype::F32);
        check(unsafe {
            ffi::hs_cast_f16_to_f32(self.stream, x.cptr(), out.mptr() as *mut f32, x.len() as i64)
        }, "cast_to_f32");
        out
    }

    /// engine/ops.rs:336-348: f32 -> f16.
    pub fn cast_to_f16(&self, x: &HipTensor) -> HipTensor {
        let out = self.empty_typed(&x.shape, Dtype::F16);
        check(unsafe {
            ffi::hs_cast_f32_to_f16(self.stream, x.f32p("cast_to_f16 input"), out.mptr(),
                                    x.len() as i64)
        }, "cast_to_f16");
        out
    }

    /// engine/ops.rs:374-389 (f32): `x[i] + table[i % table.len()]`.
    pub fn tiled_add(&self, x: &HipTensor, table: &HipTensor) -> HipTensor {
        let out = self.empty(&x.shape);
        check(unsafe {
            ffi::hs_tiled_add(self.stream, x.f32p("tiled_add x"), table.f32p("table"),
                              out.mptr() as *mut f32, x.len() as i64, table.len() as i64)
        }, "tiled_add");
        out
    }

    // ------------------------------------------------------------ fused ops

    /// split_heads + QK-norm + RoPE (model/block.rs:130-146) in one pass:
    /// token-major (S*T, H*D) in, head-major (S, H, T, D) out.
    #[allow(clippy::too_many_arguments)]
    pub fn qknorm_rope(&self, x: &HipTensor, s: usize, t: usize, h: usize, d: usize,
                       norm: Option<(&HipTensor, &HipTensor)>, rope: Option<Rope>, eps: f32)
                       -> HipTensor {
        assert_eq!(x.len(), s * t * h * d, "qknorm_rope size");
        let (nw, nb) = match norm {
            Some((w, b)) => (opt_f32(Some(w), d, "qk-norm weight"), opt_f32(Some(b), d, "qk-norm bias")),
            None => (ptr::null(), ptr::null()),
        };
        let (sn, cs, prefix) = rope_ptrs(rope.as_ref(), t, d);
        let out = self.empty_typed(&[s, h, t, d], x.dtype);
        check(unsafe {
            ffi::hs_qknorm_rope(self.stream, x.dtype.raw(), x.cptr(), nw, nb, sn, cs, out.mptr(),
                                i32_of(s, "s"), i32_of(t, "t"), i32_of(h, "h"), i32_of(d, "d"),
                                prefix, eps)
        }, "qknorm_rope");
        out
    }

    /// `qknorm_rope` on q and k in one launch, bit-identical to two calls.
    #[allow(clippy::too_many_arguments)]
    pub fn qknorm_rope_pair(&self, q: &HipTensor, k: &HipTensor, s: usize, t: usize, h: usize,
                            d: usize, norms: Option<[(&HipTensor, &HipTensor); 2]>,
                            rope: Option<Rope>, eps: f32) -> (HipTensor, HipTensor) {
        assert_eq!(q.len(), s * t * h * d, "qknorm_rope_pair size");
        assert_eq!(k.len(), q.len(), "qknorm_rope_pair k size");
        assert_eq!(q.dtype, k.dtype, "qknorm_rope_pair dtype");
        let mut p = [ptr::null::<f32>(); 4];
        if let Some([(qw, qb), (kw, kb)]) = norms {
            p = [opt_f32(Some(qw), d, "q-norm weight"), opt_f32(Some(qb), d, "q-norm bias"),
                 opt_f32(Some(kw), d, "k-norm weight"), opt_f32(Some(kb), d, "k-norm bias")];
        }
        let (sn, cs, prefix) = rope_ptrs(rope.as_ref(), t, d);
        let qh = self.empty_typed(&[s, h, t, d], q.dtype);
        let kh = self.empty_typed(&[s, h, t, d], q.dtype);
        check(unsafe {
            ffi::hs_qknorm_rope_pair(self.stream, q.dtype.raw(), q.cptr(), k.cptr(), p[0], p[1],
                                     p[2], p[3], sn, cs, qh.mptr(), kh.mptr(), i32_of(s, "s"),
                                     i32_of(t, "t"), i32_of(h, "h"), i32_of(d, "d"), prefix, eps)
        }, "qknorm_rope_pair");
        (qh, kh)
    }

    /// fc1 bias epilogue + GELU (model/block.rs:172-176).
    pub fn bias_gelu(&self, x: &HipTensor, bias: Option<&HipTensor>) -> HipTensor {
        let (rows, cols) = x.dims();
        let out = self.empty_typed(&x.shape, x.dtype);
        check(unsafe {
            ffi::hs_bias_gelu(self.stream, x.dtype.raw(), x.cptr(), opt_f32(bias, cols, "bias"),
                              out.mptr(), rows as i64, i32_of(cols, "cols"))
        }, "bias_gelu");
        out
    }

    /// proj/fc2 bias epilogue + LayerScale + residual (model/block.rs:150-155).
    pub fn bias_ls_residual(&self, res: &HipTensor, x: &HipTensor, gamma: &HipTensor,
                            bias: Option<&HipTensor>) -> HipTensor {
        assert_eq!(res.len(), x.len(), "bias_ls_residual length");
        assert_eq!(res.dtype, x.dtype, "bias_ls_residual dtype");
        let (rows, dim) = x.dims();
        let out = self.empty_typed(&res.shape, x.dtype);
        check(unsafe {
            ffi::hs_bias_ls_residual(self.stream, x.dtype.raw(), res.cptr(), x.cptr(),
                                     opt_f32(bias, dim, "bias"), opt_f32(Some(gamma), dim, "gamma"),
                                     out.mptr(), rows as i64, i32_of(dim, "dim"))
        }, "bias_ls_residual");
        out
    }

    /// `bias_ls_residual` then `layernorm` of its output in one pass
    /// (model/block.rs:150-153: x1 into LN2; a block's output into the next
    /// block's LN1). Returns (out, normed), bit-identical to the two calls.
    pub fn bias_ls_residual_layernorm(&self, res: &HipTensor, x: &HipTensor, gamma: &HipTensor,
                                      bias: Option<&HipTensor>, ln: (&HipTensor, &HipTensor),
                                      eps: f32) -> (HipTensor, HipTensor) {
        assert_eq!(res.len(), x.len(), "bias_ls_residual length");
        assert_eq!(res.dtype, x.dtype, "bias_ls_residual dtype");
        let (rows, dim) = x.dims();
        let out = self.empty_typed(&res.shape, x.dtype);
        let normed = self.empty_typed(&res.shape, x.dtype);
        check(unsafe {
            ffi::hs_bias_ls_residual_layernorm(self.stream, x.dtype.raw(), res.cptr(), x.cptr(),
                                               opt_f32(bias, dim, "bias"),
                                               opt_f32(Some(gamma), dim, "gamma"),
                                               opt_f32(Some(ln.0), dim, "norm weight"),
                                               opt_f32(Some(ln.1), dim, "norm bias"), out.mptr(),
                                               normed.mptr(), rows as i64, i32_of(dim, "dim"), eps)
        }, "bias_ls_residual_layernorm");
        (out, normed)
    }

    /// Token assembly (model/trunk.rs:68-85, model/dino.rs:76-93): per frame
    /// `[cam[v], reg[v*R..v*R+R], patches + bias + pos]`, v = 1 for frames
    /// after the first when `n_var` is 2.
    #[allow(clippy::too_many_arguments)]
    pub fn assemble_tokens(&self, patches: &HipTensor, s: usize, p: usize, cam: &HipTensor,
                           reg: Option<&HipTensor>, patch_bias: Option<&HipTensor>,
                           pos: Option<&HipTensor>, out_dtype: Dtype, n_var: usize) -> HipTensor {
        let d = *patches.shape.last().expect("patches shape");
        assert_eq!(patches.len(), s * p * d, "patches shape");
        assert_eq!(cam.dtype, out_dtype, "camera token dtype");
        assert_eq!(cam.len(), n_var * d, "camera token shape");
        let r = reg.map_or(0, |t| t.len() / (n_var * d));
        if let Some(t) = reg {
            assert_eq!(t.dtype, out_dtype, "register token dtype");
            assert_eq!(t.len(), n_var * r * d, "register token shape");
        }
        let out = self.empty_typed(&[s * (1 + r + p), d], out_dtype);
        check(unsafe {
            ffi::hs_assemble_tokens(self.stream, out_dtype.raw(), patches.cptr(),
                                    patches.dtype.raw(), opt_f32(patch_bias, d, "patch bias"),
                                    opt_f32(pos, p * d, "pos embed"), cam.cptr(),
                                    reg.map_or(ptr::null(), |t| t.cptr()), out.mptr(),
                                    i32_of(s, "s"), i32_of(p, "p"), i32_of(r, "r"),
                                    i32_of(d, "d"), i32_of(n_var, "n_var"))
        }, "assemble_tokens");
        out
    }

    /// linear(fc1, bias) + GELU in one kernel.
    pub fn linear_gelu(&self, x: &HipTensor, weight: &HipTensor, bias: Option<&HipTensor>)
                       -> HipTensor {
        let (m, k) = x.dims();
        let (n, wk) = weight.dims();
        assert_eq!(wk, k, "linear_gelu weight k");
        assert_eq!(weight.dtype, x.dtype, "linear_gelu weight dtype");
        let out = self.empty_typed(&[m, n], x.dtype);
        check(unsafe {
            ffi::hs_linear_gelu(self.stream, x.dtype.raw(), x.cptr(), weight.cptr(),
                                opt_f32(bias, n, "bias"), out.mptr(), m as i64, i32_of(n, "n"),
                                i32_of(k, "k"))
        }, "linear_gelu");
        out
    }

    /// linear(proj | fc2, bias) + LayerScale + residual in one kernel.
    pub fn linear_ls_residual(&self, x: &HipTensor, weight: &HipTensor, gamma: &HipTensor,
                              res: &HipTensor, bias: Option<&HipTensor>) -> HipTensor {
        let (m, k) = x.dims();
        let (n, wk) = weight.dims();
        assert_eq!(wk, k, "linear_ls_residual weight k");
        assert_eq!(weight.dtype, x.dtype, "linear_ls_residual weight dtype");
        assert_eq!(res.dtype, x.dtype, "linear_ls_residual res dtype");
        assert_eq!(res.len(), m * n, "linear_ls_residual res shape");
        let out = self.empty_typed(&[m, n], x.dtype);
        check(unsafe {
            ffi::hs_linear_ls_residual(self.stream, x.dtype.raw(), x.cptr(), weight.cptr(),
                                       opt_f32(bias, n, "bias"), opt_f32(Some(gamma), n, "gamma"),
                                       res.cptr(), out.mptr(), m as i64, i32_of(n, "n"),
                                       i32_of(k, "k"))
        }, "linear_ls_residual");
        out
    }

    /// The attention input projection (model/block.rs:128-146) in one kernel:
    /// the fused q|k|v weight (3*H*d, k), split into head-major q, k, v with
    /// QK-norm and RoPE on q and k.
    #[allow(clippy::too_many_arguments)]
    pub fn linear_qkv_heads(&self, x: &HipTensor, w_qkv: &HipTensor, b_qkv: Option<&HipTensor>,
                            s: usize, t: usize, h: usize,
                            norms: Option<[(&HipTensor, &HipTensor); 2]>, rope: Option<Rope>,
                            eps: f32) -> (HipTensor, HipTensor, HipTensor) {
        let (n3, k) = w_qkv.dims();
        assert_eq!(n3 % (3 * h), 0, "w_qkv rows must be 3 * H * d");
        let d = n3 / (3 * h);
        assert_eq!(x.len(), s * t * k, "x shape");
        assert_eq!(x.dtype, w_qkv.dtype, "x/w_qkv dtype");
        let mut p = [ptr::null::<f32>(); 4];
        if let Some([(qw, qb), (kw, kb)]) = norms {
            p = [opt_f32(Some(qw), d, "q-norm weight"), opt_f32(Some(qb), d, "q-norm bias"),
                 opt_f32(Some(kw), d, "k-norm weight"), opt_f32(Some(kb), d, "k-norm bias")];
        }
        let (sn, cs, prefix) = rope_ptrs(rope.as_ref(), t, d);
        let outs = [0, 1, 2].map(|_| self.empty_typed(&[s, h, t, d], x.dtype));
        check(unsafe {
            ffi::hs_linear_qkv_heads(self.stream, x.dtype.raw(), x.cptr(), w_qkv.cptr(),
                                     opt_f32(b_qkv, n3, "qkv bias"), p[0], p[1], p[2], p[3], sn,
                                     cs, outs[0].mptr(), outs[1].mptr(), outs[2].mptr(),
                                     i32_of(s, "S"), i32_of(t, "T"), i32_of(h, "H"),
                                     i32_of(d, "d"), i32_of(k, "k"), prefix, eps)
        }, "linear_qkv_heads");
        let [q, kk, v] = outs;
        (q, kk, v)
    }

    /// The statistics half of `layernorm`: (rows, 2) f32 mean and
    /// rsqrt(var + eps) per row.
    pub fn layernorm_stats(&self, x: &HipTensor, eps: f32) -> HipTensor {
        let (rows, dim) = x.dims();
        let out = self.empty(&[rows, 2]);
        check(unsafe {
            ffi::hs_layernorm_stats(self.stream, x.dtype.raw(), x.cptr(), out.mptr() as *mut f32,
                                    rows as i64, i32_of(dim, "dim"), eps)
        }, "layernorm_stats");
        out
    }

    /// Operands of the `linear_ln*` calls: x (m, k), the LayerNorm's weight
    /// and bias (k, f32), the linear weight (n, k); a statistics workspace.
    fn ln_operands(&self, x: &HipTensor, ln: (&HipTensor, &HipTensor), weight: &HipTensor)
                   -> (usize, usize, usize, *const f32, *const f32, HipTensor) {
        let (m, k) = x.dims();
        let (n, wk) = weight.dims();
        assert_eq!(wk, k, "linear_ln weight k");
        assert_eq!(weight.dtype, x.dtype, "linear_ln weight dtype");
        let lw = opt_f32(Some(ln.0), k, "norm weight");
        let lb = opt_f32(Some(ln.1), k, "norm bias");
        (m, n, k, lw, lb, self.empty(&[m, 2]))
    }

    /// layernorm(x) then linear(weight, bias) (model/block.rs:128-131) in one
    /// product: the normalised rows, rounded to the storage type as
    /// `layernorm` stores them, exist only on the way to the matrix cores.
    pub fn linear_ln(&self, x: &HipTensor, ln: (&HipTensor, &HipTensor), weight: &HipTensor,
                     bias: Option<&HipTensor>, eps: f32) -> HipTensor {
        let (m, n, k, lw, lb, ws) = self.ln_operands(x, ln, weight);
        let out = self.empty_typed(&[m, n], x.dtype);
        check(unsafe {
            ffi::hs_linear_ln(self.stream, x.dtype.raw(), x.cptr(), lw, lb, weight.cptr(),
                              opt_f32(bias, n, "bias"), ws.mptr() as *mut f32, out.mptr(),
                              m as i64, i32_of(n, "n"), i32_of(k, "k"), eps)
        }, "linear_ln");
        out
    }

    /// gelu(linear(layernorm(x))) in one product (LN2, fc1, GELU,
    /// model/block.rs:153, 172-176).
    pub fn linear_ln_gelu(&self, x: &HipTensor, ln: (&HipTensor, &HipTensor), weight: &HipTensor,
                          bias: Option<&HipTensor>, eps: f32) -> HipTensor {
        let (m, n, k, lw, lb, ws) = self.ln_operands(x, ln, weight);
        let out = self.empty_typed(&[m, n], x.dtype);
        check(unsafe {
            ffi::hs_linear_ln_gelu(self.stream, x.dtype.raw(), x.cptr(), lw, lb, weight.cptr(),
                                   opt_f32(bias, n, "bias"), ws.mptr() as *mut f32, out.mptr(),
                                   m as i64, i32_of(n, "n"), i32_of(k, "k"), eps)
        }, "linear_ln_gelu");
        out
    }

    /// `linear_ln_gelu` into a caller's output without any device
    /// allocation by the library (the row statistics use the library's own
    /// per-device array): for callers that cannot allocate. At most 524,288
    /// rows; calls that overlap on one device race.
    pub fn linear_ln_gelu_noalloc(&self, x: &HipTensor, ln: (&HipTensor, &HipTensor),
                                  weight: &HipTensor, bias: Option<&HipTensor>, eps: f32,
                                  out: &HipTensor) {
        let (m, k) = x.dims();
        let (n, wk) = weight.dims();
        assert_eq!(wk, k, "linear_ln weight k");
        assert_eq!(weight.dtype, x.dtype, "linear_ln weight dtype");
        assert_eq!(out.len(), m * n, "out shape");
        assert_eq!(out.dtype, x.dtype, "out dtype");
        check(unsafe {
            ffi::hs_linear_ln_gelu_noalloc(self.stream, x.dtype.raw(), x.cptr(),
                                           opt_f32(Some(ln.0), k, "norm weight"),
                                           opt_f32(Some(ln.1), k, "norm bias"), weight.cptr(),
                                           opt_f32(bias, n, "bias"), out.mptr(), m as i64,
                                           i32_of(n, "n"), i32_of(k, "k"), eps)
        }, "linear_ln_gelu_noalloc");
    }

    /// LN1 + the q|k|v projection with heads, QK-norm and RoPE
    /// (model/block.rs:128-146) in one product.
    #[allow(clippy::too_many_arguments)]
    pub fn linear_ln_qkv_heads(&self, x: &HipTensor, ln: (&HipTensor, &HipTensor),
                               w_qkv: &HipTensor, b_qkv: Option<&HipTensor>, s: usize, t: usize,
                               h: usize, norms: Option<[(&HipTensor, &HipTensor); 2]>,
                               rope: Option<Rope>, eps: f32) -> (HipTensor, HipTensor, HipTensor) {
        let (m, n3, k, lw, lb, ws) = self.ln_operands(x, ln, w_qkv);
        assert_eq!(m, s * t, "x rows must be S*T");
        assert_eq!(n3 % (3 * h), 0, "w_qkv rows must be 3 * H * d");
        let d = n3 / (3 * h);
        let mut p = [ptr::null::<f32>(); 4];
        if let Some([(qw, qb), (kw, kb)]) = norms {
            p = [opt_f32(Some(qw), d, "q-norm weight"), opt_f32(Some(qb), d, "q-norm bias"),
                 opt_f32(Some(kw), d, "k-norm weight"), opt_f32(Some(kb), d, "k-norm bias")];
        }
        let (sn, cs, prefix) = rope_ptrs(rope.as_ref(), t, d);
        let outs = [0, 1, 2].map(|_| self.empty_typed(&[s, h, t, d], x.dtype));
        check(unsafe {
            ffi::hs_linear_ln_qkv_heads(self.stream, x.dtype.raw(), x.cptr(), lw, lb, w_qkv.cptr(),
                                        opt_f32(b_qkv, n3, "qkv bias"), p[0], p[1], p[2], p[3],
                                        sn, cs, ws.mptr() as *mut f32, outs[0].mptr(),
                                        outs[1].mptr(), outs[2].mptr(), i32_of(s, "S"),
                                        i32_of(t, "T"), i32_of(h, "H"), i32_of(d, "d"),
                                        i32_of(k, "k"), prefix, eps)
        }, "linear_ln_qkv_heads");
        let [q, kk, v] = outs;
        (q, kk, v)
    }

    /// Cache::build (model/cache.rs:21-52) in one pass: [frame_out | inter_out]
    /// as f32.
    pub fn cache_build(&self, frame_out: &HipTensor, inter_out: &HipTensor) -> HipTensor {
        let (rows, c1) = frame_out.dims();
        let (rows_i, c2) = inter_out.dims();
        assert_eq!(rows, rows_i, "cache_build rows");
        assert_eq!(frame_out.dtype, inter_out.dtype, "cache_build dtype");
        let out = self.empty(&[rows, c1 + c2]);
        check(unsafe {
            ffi::hs_cache_build(self.stream, frame_out.dtype.raw(), frame_out.cptr(),
                                inter_out.cptr(), out.mptr() as *mut f32, rows as i64,
                                i32_of(c1, "c1"), i32_of(c2, "c2"))
        }, "cache_build");
        out
    }

    /// `n_blocks` copy_rows calls in one launch (model/trunk.rs:103-116).
    #[allow(clippy::too_many_arguments)]
    pub fn copy_row_blocks(&self, src: &HipTensor, src_row0: usize, src_stride: usize,
                           dst: &HipTensor, dst_row0: usize, dst_stride: usize, n_blocks: usize,
                           rows_per_block: usize) {
        assert_eq!(src.dtype, dst.dtype, "copy_row_blocks dtype");
        assert_eq!(src.row_bytes(), dst.row_bytes(), "copy_row_blocks row width");
        check(unsafe {
            ffi::hs_copy_row_blocks(self.stream, src.cptr(), src_row0 as i64, src_stride as i64,
                                    dst.mptr(), dst_row0 as i64, dst_stride as i64,
                                    n_blocks as i64, rows_per_block as i64,
                                    src.row_bytes() as i64)
        }, "copy_row_blocks");
    }

    /// attention + attn_merge (model/block.rs:148-149) in one pass.
    pub fn attention_merged(&self, q: &HipTensor, k: &HipTensor, v: &HipTensor) -> HipTensor {
        let [s, h, t, d] = q.shape[..] else { panic!("attention wants (S,H,T,D)") };
        assert_eq!(q.shape, k.shape, "attention k shape");
        assert_eq!(q.shape, v.shape, "attention v shape");
        let out = self.empty_typed(&[s * t, h * d], q.dtype);
        check(unsafe {
            ffi::hs_attention_merged(self.stream, q.dtype.raw(), q.cptr(), k.cptr(), v.cptr(),
                                     out.mptr(), i32_of(s, "s"), i32_of(h, "h"), i32_of(t, "t"),
                                     i32_of(d, "d"))
        }, "attention_merged");
        out
    }
}

fn rope_ptrs(rope: Option<&Rope>, t: usize, d: usize) -> (*const f32, *const f32, i32) {
    match rope {
        None => (ptr::null(), ptr::null(), 0),
        Some(r) => {
            assert!(r.prefix <= t, "rope prefix");
            (opt_f32(Some(r.sin), (t - r.prefix) * d, "rope sin table"),
             opt_f32(Some(r.cos), (t - r.prefix) * d, "rope cos table"),
             i32_of(r.prefix, "prefix"))
        }
    }
}

fn upload(t: &HipTensor, src: *const c_void) {
    if t.byte_len() > 0 {
        hip_check(unsafe {
            ffi::hipMemcpy(t.mptr(), src, t.byte_len(), ffi::HIP_MEMCPY_HOST_TO_DEVICE)
        }, "hipMemcpy");
    }
}

fn download(t: &HipTensor, dst: *mut c_void) {
    if t.byte_len() > 0 {
        hip_check(unsafe {
            ffi::hipMemcpy(dst, t.cptr(), t.byte_len(), ffi::HIP_MEMCPY_DEVICE_TO_HOST)
        }, "hipMemcpy");
    }
}

/// Host-side RoPE tables (engine/rope.rs), bit-identical to the reference.
pub mod rope {
    use super::ffi;

    /// rope::periods (engine/rope.rs:8-10).
    pub fn periods() -> [f32; 16] {
        let mut p = [0f32; 16];
        unsafe { ffi::hs_rope_periods(p.as_mut_ptr()) };
        p
    }

    /// rope::tables (engine/rope.rs:18-43): (h_p*w_p, 64) sin and cos.
    pub fn tables(periods: &[f32; 16], h_p: usize, w_p: usize) -> (Vec<f32>, Vec<f32>) {
        let n = h_p * w_p * 64;
        let (mut sin, mut cos) = (vec![0f32; n], vec![0f32; n]);
        let st = unsafe {
            ffi::hs_rope_tables(periods.as_ptr(), h_p as i32, w_p as i32, sin.as_mut_ptr(),
                                cos.as_mut_ptr())
        };
        super::check(st, "rope::tables");
        (sin, cos)
    }
}
