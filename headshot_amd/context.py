"""``HipContext``: headshot-server's op-dispatch surface over libheadshot_hip.

Mirrors ``impl GpuContext`` (crates/headshot-server/src/engine/ops.rs,
engine/tensor.rs) for the per-layer op path: same method names, argument
meaning and error behaviour. Tensors are torch tensors in device memory
(torch supplies allocation and streams only; every op runs a HIP kernel of
libheadshot_hip through its C ABI on the current stream). Storage is
float32 or float16; norm weights, biases, gammas and RoPE tables must be
float32 (engine/ops.rs:5-8). Contract violations raise AssertionError, as the
reference's ``assert!`` panics.

Like the reference, every op except ``rope_apply`` and ``copy_rows`` returns
a new output tensor; the fused ops also accept ``out=`` to write into a
caller buffer (no allocation). After each op, ``last_launch`` holds a
callable that re-issues the same validated C call on the then-current
stream (for launch loops and graph capture without per-call Python checks).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib

F32 = torch.float32
F16 = torch.float16


def _dt(t: torch.Tensor) -> int:
    if t.dtype == F32:
        return _lib.HS_F32
    if t.dtype == F16:
        return _lib.HS_F16
    raise AssertionError(f"storage must be f32 or f16, got {t.dtype}")


class _Ptr(int):
    """A device address passed to the library, holding its tensor: a launch's
    re-issue thunk keeps the tensors of its own arguments alive (a replayed
    launch must never write into memory the caching allocator has handed
    out again). Nothing is shared between calls or threads."""


def _dev(t: torch.Tensor, what: str) -> int:
    assert t.is_cuda, f"{what} must live in device memory"
    assert t.is_contiguous(), f"{what} must be contiguous"
    p = _Ptr(t.data_ptr())
    p.tensor = t
    return p


def _param(t, n: int, what: str) -> int:
    assert t.dtype == F32, f"{what} must be f32"
    assert t.numel() == n, f"{what} len {t.numel()} != {n}"
    return _dev(t, what)


def _opt(t, n: int, what: str):
    return None if t is None else _param(t, n, what)


def _qkv_fused(dtype, d: int, n3: int, k: int) -> bool:
    """Shapes the fused q|k|v kernels cover: head dim 64, whole column tiles
    (256 in f16, 128 in f32) and whole k stages (64 in f16, 32 in f32)."""
    if d != 64:
        return False
    if dtype == F16:
        return n3 % 256 == 0 and k % 64 == 0
    return dtype == F32 and n3 % 128 == 0 and k % 32 == 0


class HipContext:
    """One device's op surface. ``device`` is a torch device (default cuda:0)."""

    def __init__(self, device: str | torch.device = "cuda"):
        self.lib = _lib.load()
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise AssertionError("HipContext needs a HIP device")
        if not torch.cuda.is_available():
            raise RuntimeError("no HIP device visible (torch.cuda.is_available() is False)")
        self.last_launch = None

    def _launch(self, name: str, fn, *args) -> None:
        held = tuple(a.tensor for a in args if isinstance(a, _Ptr))

        def call():
            _lib.check(fn(torch.cuda.current_stream().cuda_stream, *args), name)

        call.held = held
        call()
        self.last_launch = call

    # ------------------------------------------------------------------ tensors

    def empty_typed(self, shape, dtype: torch.dtype = F32) -> torch.Tensor:
        """engine/tensor.rs:132-141 (uninitialised device tensor)."""
        return torch.empty(tuple(shape), dtype=dtype, device=self.device)

    def empty(self, shape) -> torch.Tensor:
        return self.empty_typed(shape, F32)

    def tensor_from_f32(self, shape, data, dtype: torch.dtype = F32) -> torch.Tensor:
        """engine/tensor.rs:71-91: upload f32 data as ``dtype`` storage (f16 by
        round-to-nearest-even)."""
        arr = np.asarray(data, dtype=np.float32)
        assert arr.size == int(np.prod(shape)), "shape/data mismatch"
        host = torch.from_numpy(np.ascontiguousarray(arr).reshape(tuple(shape)))
        return host.to(device=self.device, dtype=dtype)

    def tensor_from_slice(self, shape, data) -> torch.Tensor:
        return self.tensor_from_f32(shape, data, F32)

    def download(self, t: torch.Tensor) -> np.ndarray:
        """engine/tensor.rs:162-198: flush, read back as f32."""
        torch.cuda.current_stream().synchronize()
        return t.detach().to("cpu").to(F32).numpy()

    def sync(self) -> None:
        torch.cuda.current_stream().synchronize()

    # ----------------------------------------------------------- reference ops

    def linear(self, x, weight, bias=None, out=None) -> torch.Tensor:
        """engine/ops.rs:81-128: ``out (m, n) = x (m, k) @ weight (n, k)^T [+ bias]``."""
        k = x.shape[-1]
        m = x.numel() // k if k else 0
        assert weight.dim() == 2 and weight.shape[1] == k, "weight k mismatch"
        assert weight.dtype == x.dtype, "weight/activation dtype"
        n = weight.shape[0]
        b = _opt(bias, n, "bias")
        if out is None:
            out = self.empty_typed((m, n), x.dtype)
        assert out.dtype == x.dtype and out.numel() == m * n, "out shape/dtype"
        self._launch("linear", self.lib.hs_linear, _dt(x), _dev(x, "x"), _dev(weight, "weight"),
                     b, _dev(out, "out"), m, n, k)
        return out

    def layernorm(self, x, weight, bias, eps: float = 1e-5, out=None) -> torch.Tensor:
        """engine/ops.rs:130-153 (eps is 1e-5 there; pass it explicitly here)."""
        dim = x.shape[-1]
        rows = x.numel() // dim if dim else 0
        w = _param(weight, dim, "norm weight")
        b = _param(bias, dim, "norm bias")
        if out is None:
            out = self.empty_typed(x.shape, x.dtype)
        assert out.dtype == x.dtype and out.numel() == x.numel(), "out shape/dtype"
        self._launch("layernorm", self.lib.hs_layernorm, _dt(x), _dev(x, "x"), w, b,
                     _dev(out, "out"), rows, dim, eps)
        return out

    def gelu(self, x, out=None) -> torch.Tensor:
        """engine/ops.rs:155-165."""
        if out is None:
            out = self.empty_typed(x.shape, x.dtype)
        assert out.dtype == x.dtype and out.numel() == x.numel(), "out shape/dtype"
        self._launch("gelu", self.lib.hs_gelu, _dt(x), _dev(x, "x"), _dev(out, "out"), x.numel())
        return out

    def residual_ls(self, res, x, gamma, out=None) -> torch.Tensor:
        """engine/ops.rs:167-183: ``res + gamma ⊙ x``."""
        assert res.numel() == x.numel(), "res/x length"
        assert res.dtype == x.dtype, "res/x dtype"
        assert gamma.dtype == F32, "gamma must be f32"
        dim = gamma.numel()
        assert dim > 0 and x.numel() % dim == 0, "gamma must tile x"
        if out is None:
            out = self.empty_typed(res.shape, x.dtype)
        assert out.dtype == x.dtype and out.numel() == x.numel(), "out shape/dtype"
        self._launch("residual_ls", self.lib.hs_residual_ls, _dt(x), _dev(res, "res"),
                     _dev(x, "x"), _dev(gamma, "gamma"), _dev(out, "out"), x.numel(), dim)
        return out

    def split_heads(self, x, s: int, t: int, h: int, d: int) -> torch.Tensor:
        """engine/ops.rs:185-200: (S·T, H·D) → (S, H, T, D)."""
        assert x.numel() == s * t * h * d, "split_heads size"
        out = self.empty_typed((s, h, t, d), x.dtype)
        self._launch("split_heads", self.lib.hs_split_heads, _dt(x), _dev(x, "x"),
                     _dev(out, "out"), s, t, h, d)
        return out

    def rope_apply(self, x, sin, cos, prefix: int) -> None:
        """engine/ops.rs:202-223: in place on (S, H, T, D); tables (T−prefix, D)."""
        assert x.dim() == 4, "rope_apply wants (S,H,T,D)"
        s, h, t, d = x.shape
        assert 0 <= prefix <= t, "prefix"
        assert sin.numel() == (t - prefix) * d, "table size"
        assert sin.dtype == F32 and cos.dtype == F32, "rope tables must be f32"
        assert cos.numel() == sin.numel(), "table size"
        self._launch("rope_apply", self.lib.hs_rope_apply, _dt(x), _dev(x, "x"),
                     _dev(sin, "sin"), _dev(cos, "cos"), s, h, t, d, prefix)

    def cast_to_f16(self, x) -> torch.Tensor:
        """engine/ops.rs:336-348."""
        assert x.dtype == F32, "cast_to_f16 wants f32"
        out = self.empty_typed(x.shape, F16)
        self._launch("cast_to_f16", self.lib.hs_cast_f32_to_f16, _dev(x, "x"), _dev(out, "out"),
                     x.numel())
        return out

    def copy_rows(self, src, src_row: int, dst, dst_row: int, n_rows: int) -> None:
        """engine/tensor.rs:146-160: rows of the last dimension."""
        assert src.dtype == dst.dtype, "copy_rows dtype"
        row_bytes = src.shape[-1] * src.element_size()
        assert row_bytes == dst.shape[-1] * dst.element_size(), "copy_rows row width"
        assert (src_row + n_rows) * row_bytes <= src.numel() * src.element_size(), "src rows"
        assert (dst_row + n_rows) * row_bytes <= dst.numel() * dst.element_size(), "dst rows"
        self._launch("copy_rows", self.lib.hs_copy_rows, _dev(src, "src"), src_row,
                     _dev(dst, "dst"), dst_row, n_rows, row_bytes)

    def tiled_add(self, x, table, out=None) -> torch.Tensor:
        """engine/ops.rs:374-389 (f32 only); ``out`` may be ``x``."""
        assert x.dtype == F32 and table.dtype == F32, "tiled_add is f32"
        assert table.numel() > 0 and x.numel() % table.numel() == 0, "table must tile x"
        if out is None:
            out = self.empty(x.shape)
        assert out.dtype == F32 and out.numel() == x.numel(), "out shape/dtype"
        self._launch("tiled_add", self.lib.hs_tiled_add, _dev(x, "x"), _dev(table, "table"),
                     _dev(out, "out"), x.numel(), table.numel())
        return out

    def concat_channels(self, a, b) -> torch.Tensor:
        """engine/ops.rs:302-318: a (rows, c1) ++ b (rows, c2) → (rows, c1+c2)."""
        c1, c2 = a.shape[-1], b.shape[-1]
        rows = math.prod(a.shape[:-1])
        assert math.prod(b.shape[:-1]) == rows, "row mismatch"
        assert a.dtype == b.dtype, "concat_channels dtype"
        out = self.empty_typed((rows, c1 + c2), a.dtype)
        self._launch("concat_channels", self.lib.hs_concat_channels, _dt(a), _dev(a, "a"),
                     _dev(b, "b"), _dev(out, "out"), rows, c1, c2)
        return out

    def cast_to_f32(self, x) -> torch.Tensor:
        """engine/ops.rs:321-334 (f16 → f32)."""
        assert x.dtype == F16, "cast_to_f32 wants f16"
        out = self.empty_typed(x.shape, F32)
        self._launch("cast_f16_to_f32", self.lib.hs_cast_f16_to_f32, _dev(x, "x"),
                     _dev(out, "out"), x.numel())
        return out

    def copy_row_blocks(self, src, src_row: int, src_stride: int, dst, dst_row: int,
                        dst_stride: int, n_blocks: int, rows_per_block: int) -> None:
        """``n_blocks`` copy_rows calls (engine/tensor.rs:146-160) in one launch:
        block j copies rows [src_row + j*src_stride, + rows_per_block) of src
        to [dst_row + j*dst_stride, ...) of dst (model/trunk.rs:103-116)."""
        assert src.dtype == dst.dtype, "copy_row_blocks dtype"
        row = src.shape[-1] * src.element_size()
        assert row == dst.shape[-1] * dst.element_size(), "copy_row_blocks row width"
        if n_blocks and rows_per_block:
            last_s = src_row + (n_blocks - 1) * src_stride + rows_per_block
            last_d = dst_row + (n_blocks - 1) * dst_stride + rows_per_block
            assert last_s * row <= src.numel() * src.element_size(), "src rows"
            assert last_d * row <= dst.numel() * dst.element_size(), "dst rows"
        self._launch("copy_row_blocks", self.lib.hs_copy_row_blocks, _dev(src, "src"), src_row,
                     src_stride, _dev(dst, "dst"), dst_row, dst_stride, n_blocks,
                     rows_per_block, row)

    def attention(self, q, k, v) -> torch.Tensor:
        """engine/ops.rs:225-253: non-causal attention over head-major
        (S, H, T, D) q, k, v; D 64 (f32/f16) or 128 (f32)."""
        assert q.dim() == 4, "attention wants (S,H,T,D)"
        s, h, t, d = q.shape
        assert tuple(k.shape) == tuple(q.shape), "attention: k shape"
        assert tuple(v.shape) == tuple(q.shape), "attention: v shape"
        assert q.dtype == k.dtype == v.dtype, "attention: dtype"
        out = self.empty_typed((s, h, t, d), q.dtype)
        self._launch("attention", self.lib.hs_attention, _dt(q), _dev(q, "q"), _dev(k, "k"),
                     _dev(v, "v"), _dev(out, "out"), s, h, t, d)
        return out

    def attn_merge(self, x) -> torch.Tensor:
        """engine/ops.rs:255-267: (S, H, T, D) → (S·T, H·D)."""
        assert x.dim() == 4, "attn_merge wants (S,H,T,D)"
        s, h, t, d = x.shape
        out = self.empty_typed((s * t, h * d), x.dtype)
        self._launch("attn_merge", self.lib.hs_attn_merge, _dt(x), _dev(x, "x"),
                     _dev(out, "out"), s, h, t, d)
        return out

    # --------------------------------------------------------------- fused ops

    def qknorm_rope(self, x_tok, s: int, t: int, h: int, d: int, norm=None, rope=None,
                    eps: float = 1e-5, out=None) -> torch.Tensor:
        """split_heads + QK-norm + RoPE (model/block.rs:130-146) in one pass.

        ``norm`` = (weight, bias) f32 (d) or None; ``rope`` = (sin, cos, prefix)
        with f32 tables (t − prefix, d) or None (global blocks)."""
        assert x_tok.numel() == s * t * h * d, "qknorm_rope size"
        nw = nb = sn = cs = None
        prefix = 0
        if norm is not None:
            nw = _param(norm[0], d, "qk-norm weight")
            nb = _param(norm[1], d, "qk-norm bias")
        if rope is not None:
            sin, cos, prefix = rope
            assert 0 <= prefix <= t, "prefix"
            sn = _param(sin, (t - prefix) * d, "rope sin table")
            cs = _param(cos, (t - prefix) * d, "rope cos table")
        if out is None:
            out = self.empty_typed((s, h, t, d), x_tok.dtype)
        assert out.dtype == x_tok.dtype and out.numel() == x_tok.numel(), "out shape/dtype"
        self._launch("qknorm_rope", self.lib.hs_qknorm_rope, _dt(x_tok), _dev(x_tok, "x"), nw, nb,
                     sn, cs, _dev(out, "out"), s, t, h, d, prefix, eps)
        return out

    def qknorm_rope_pair(self, q_tok, k_tok, s: int, t: int, h: int, d: int, qn=None, kn=None,
                         rope=None, eps: float = 1e-5, out_q=None, out_k=None):
        """``qknorm_rope`` on q (norm ``qn``) and on k (norm ``kn``) in one
        launch, bit-identical to two calls (model/block.rs:130-146). Both
        norms are given or neither. Returns (q_head, k_head)."""
        assert q_tok.numel() == s * t * h * d and k_tok.numel() == q_tok.numel(), "qk size"
        assert q_tok.dtype == k_tok.dtype, "q/k dtype"
        assert (qn is None) == (kn is None), "QK-norm for both q and k or for neither"
        qw = qb = kw = kb = sn = cs = None
        prefix = 0
        if qn is not None:
            qw, qb = _param(qn[0], d, "q-norm weight"), _param(qn[1], d, "q-norm bias")
            kw, kb = _param(kn[0], d, "k-norm weight"), _param(kn[1], d, "k-norm bias")
        if rope is not None:
            sin, cos, prefix = rope
            assert 0 <= prefix <= t, "prefix"
            sn = _param(sin, (t - prefix) * d, "rope sin table")
            cs = _param(cos, (t - prefix) * d, "rope cos table")
        outs = []
        for o in (out_q, out_k):
            if o is None:
                o = self.empty_typed((s, h, t, d), q_tok.dtype)
            assert o.dtype == q_tok.dtype and o.numel() == q_tok.numel(), "out shape/dtype"
            outs.append(o)
        self._launch("qknorm_rope_pair", self.lib.hs_qknorm_rope_pair, _dt(q_tok),
                     _dev(q_tok, "q"), _dev(k_tok, "k"), qw, qb, kw, kb, sn, cs,
                     _dev(outs[0], "out_q"), _dev(outs[1], "out_k"), s, t, h, d, prefix, eps)
        return outs[0], outs[1]

    def linear_qkv_heads(self, x, w_qkv, b_qkv, s: int, t: int, h: int, qn=None, kn=None,
                         rope=None, eps: float = 1e-5, out=None):
        """The attention input projection (model/block.rs:128-146) in one
        kernel: x (S*T, k) @ w_qkv^T + b_qkv with w_qkv (3*H*d, k) holding q |
        k | v on its output rows, split into head-major (S, H, T, d) q, k, v,
        QK-norm (``qn``, ``kn`` = (weight, bias) or None) and RoPE (``rope``
        = (sin, cos, prefix) or None) on q and k. Bit-identical to linear then
        qknorm_rope per third for 8, 16 or 32 heads (within one f16 ulp for
        other head counts); that sequence is what runs for shapes the fused
        kernel does not cover (f32, head dim other than 64). Returns (q, k, v)."""
        n3, k = w_qkv.shape
        assert n3 % (3 * h) == 0, "w_qkv rows must be 3 * H * d"
        d = n3 // (3 * h)
        assert x.numel() == s * t * k and x.dtype == w_qkv.dtype, "x shape/dtype"
        hd = h * d
        if not _qkv_fused(x.dtype, d, n3, k):
            outs = []
            for i, norm in enumerate((qn, kn, None)):
                b = None if b_qkv is None else b_qkv[i * hd:(i + 1) * hd]
                proj = self.linear(x, w_qkv[i * hd:(i + 1) * hd], b)
                outs.append(self.qknorm_rope(proj, s, t, h, d, norm=norm,
                                             rope=rope if i < 2 else None, eps=eps,
                                             out=None if out is None else out[i]))
            return tuple(outs)
        b = _opt(b_qkv, n3, "qkv bias")
        qw = qb = kw = kb = sn = cs = None
        prefix = 0
        if qn is not None:
            qw, qb = _param(qn[0], d, "q-norm weight"), _param(qn[1], d, "q-norm bias")
        if kn is not None:
            kw, kb = _param(kn[0], d, "k-norm weight"), _param(kn[1], d, "k-norm bias")
        if rope is not None:
            sin, cos, prefix = rope
            assert 0 <= prefix <= t, "prefix"
            sn = _param(sin, (t - prefix) * d, "rope sin table")
            cs = _param(cos, (t - prefix) * d, "rope cos table")
        if out is None:
            out = tuple(self.empty_typed((s, h, t, d), x.dtype) for _ in range(3))
        for o in out:
            assert o.dtype == x.dtype and o.numel() == s * t * hd, "out shape/dtype"
        self._launch("linear_qkv_heads", self.lib.hs_linear_qkv_heads, _dt(x), _dev(x, "x"),
                     _dev(w_qkv, "w_qkv"), b, qw, qb, kw, kb, sn, cs, _dev(out[0], "q out"),
                     _dev(out[1], "k out"), _dev(out[2], "v out"), s, t, h, d, k, prefix, eps)
        return tuple(out)

    def layernorm_stats(self, x, eps: float = 1e-5, out=None) -> torch.Tensor:
        """The statistics half of ``layernorm`` (engine/ops.rs:130-153): (rows,
        2) f32 holding each row's mean and rsqrt(var + eps), bit-identical to
        what ``layernorm`` normalises with."""
        dim = x.shape[-1]
        rows = x.numel() // dim if dim else 0
        if out is None:
            out = self.empty_typed((rows, 2), F32)
        assert out.dtype == F32 and out.numel() == 2 * rows, "out shape/dtype"
        self._launch("layernorm_stats", self.lib.hs_layernorm_stats, _dt(x), _dev(x, "x"),
                     _dev(out, "stats"), rows, dim, eps)
        return out

    def _ln_args(self, x, ln, weight, bias, workspace):
        """Operands of the ``linear_ln*`` calls: ``ln`` = (weight, bias) of the
        LayerNorm over x's last dim, ``weight`` (n, k) and ``bias`` (n) or
        None of the linear layer, ``workspace`` (m, 2) f32 or None."""
        k = x.shape[-1]
        m = x.numel() // k if k else 0
        assert weight.dim() == 2 and weight.shape[1] == k, "weight k mismatch"
        assert weight.dtype == x.dtype, "weight/activation dtype"
        n = weight.shape[0]
        lw, lb = _param(ln[0], k, "norm weight"), _param(ln[1], k, "norm bias")
        b = _opt(bias, n, "bias")
        if workspace is None:
            workspace = self.empty_typed((m, 2), F32)
        assert workspace.dtype == F32 and workspace.numel() >= 2 * m, "workspace shape/dtype"
        return m, n, k, lw, lb, b, _dev(workspace, "workspace")

    def linear_ln(self, x, ln, weight, bias=None, eps: float = 1e-5, out=None,
                  workspace=None) -> torch.Tensor:
        """layernorm(x, *ln) then linear(weight, bias) (model/block.rs:128-131)
        in one product: the normalised rows, rounded to the storage type as
        ``layernorm`` stores them, exist only on the way to the matrix cores.
        Bit-identical to ``linear(layernorm(x))``."""
        m, n, k, lw, lb, b, ws = self._ln_args(x, ln, weight, bias, workspace)
        if out is None:
            out = self.empty_typed((m, n), x.dtype)
        assert out.dtype == x.dtype and out.numel() == m * n, "out shape/dtype"
        self._launch("linear_ln", self.lib.hs_linear_ln, _dt(x), _dev(x, "x"), lw, lb,
                     _dev(weight, "weight"), b, ws, _dev(out, "out"), m, n, k, eps)
        return out

    def linear_ln_gelu(self, x, ln, weight, bias=None, eps: float = 1e-5, out=None,
                       workspace=None) -> torch.Tensor:
        """gelu(linear(layernorm(x))) (model/block.rs:153, 172-176: LN2, fc1,
        GELU) in one product, bit-identical to ``linear_gelu(layernorm(x))``
        under the conditions of ``linear_ln``."""
        m, n, k, lw, lb, b, ws = self._ln_args(x, ln, weight, bias, workspace)
        if out is None:
            out = self.empty_typed((m, n), x.dtype)
        assert out.dtype == x.dtype and out.numel() == m * n, "out shape/dtype"
        self._launch("linear_ln_gelu", self.lib.hs_linear_ln_gelu, _dt(x), _dev(x, "x"), lw, lb,
                     _dev(weight, "weight"), b, ws, _dev(out, "out"), m, n, k, eps)
        return out

    def linear_ln_qkv_heads(self, x, ln, w_qkv, b_qkv, s: int, t: int, h: int, qn=None,
                            kn=None, rope=None, eps: float = 1e-5, out=None, workspace=None):
        """LN1 + the q|k|v projection with split_heads, QK-norm and RoPE
        (model/block.rs:128-146) in one product: returns head-major (q, k,
        v), bit-identical to ``linear_qkv_heads(layernorm(x))``. ``eps``
        serves both norms. Shapes the fused kernel does not cover (f32, head
        dim other than 64) run ``layernorm`` then ``linear_qkv_heads``."""
        n3, k = w_qkv.shape
        assert n3 % (3 * h) == 0, "w_qkv rows must be 3 * H * d"
        d = n3 // (3 * h)
        assert x.numel() == s * t * k and x.dtype == w_qkv.dtype, "x shape/dtype"
        if not _qkv_fused(x.dtype, d, n3, k):
            xn = self.layernorm(x, ln[0], ln[1], eps=eps)
            return self.linear_qkv_heads(xn, w_qkv, b_qkv, s, t, h, qn=qn, kn=kn, rope=rope,
                                         eps=eps, out=out)
        m, _, _, lw, lb, b, ws = self._ln_args(x, ln, w_qkv, b_qkv, workspace)
        qw = qb = kw = kb = sn = cs = None
        prefix = 0
        if qn is not None:
            qw, qb = _param(qn[0], d, "q-norm weight"), _param(qn[1], d, "q-norm bias")
        if kn is not None:
            kw, kb = _param(kn[0], d, "k-norm weight"), _param(kn[1], d, "k-norm bias")
        if rope is not None:
            sin, cos, prefix = rope
            assert 0 <= prefix <= t, "prefix"
            sn = _param(sin, (t - prefix) * d, "rope sin table")
            cs = _param(cos, (t - prefix) * d, "rope cos table")
        if out is None:
            out = tuple(self.empty_typed((s, h, t, d), x.dtype) for _ in range(3))
        for o in out:
            assert o.dtype == x.dtype and o.numel() == s * t * h * d, "out shape/dtype"
        self._launch("linear_ln_qkv_heads", self.lib.hs_linear_ln_qkv_heads, _dt(x),
                     _dev(x, "x"), lw, lb, _dev(w_qkv, "w_qkv"), b, qw, qb, kw, kb, sn, cs, ws,
                     _dev(out[0], "q out"), _dev(out[1], "k out"), _dev(out[2], "v out"), s, t,
                     h, d, k, prefix, eps)
        return tuple(out)

    def linear_gelu(self, x, weight, bias=None, out=None) -> torch.Tensor:
        """linear(fc1, bias) + GELU (model/block.rs:172-176) in one kernel."""
        k = x.shape[-1]
        m = x.numel() // k if k else 0
        assert weight.dim() == 2 and weight.shape[1] == k, "weight k mismatch"
        assert weight.dtype == x.dtype, "weight/activation dtype"
        n = weight.shape[0]
        b = _opt(bias, n, "bias")
        if out is None:
            out = self.empty_typed((m, n), x.dtype)
        assert out.dtype == x.dtype and out.numel() == m * n, "out shape/dtype"
        self._launch("linear_gelu", self.lib.hs_linear_gelu, _dt(x), _dev(x, "x"),
                     _dev(weight, "weight"), b, _dev(out, "out"), m, n, k)
        return out

    def linear_ls_residual(self, x, weight, gamma, res, bias=None, out=None) -> torch.Tensor:
        """linear(proj | fc2, bias) + LayerScale + residual (model/block.rs:150-155):
        ``res + gamma * (x @ weight^T + bias)``; ``out`` may be ``res``."""
        k = x.shape[-1]
        m = x.numel() // k if k else 0
        assert weight.dim() == 2 and weight.shape[1] == k, "weight k mismatch"
        assert weight.dtype == x.dtype and res.dtype == x.dtype, "weight/res/activation dtype"
        n = weight.shape[0]
        assert res.numel() == m * n, "res shape"
        g = _param(gamma, n, "gamma")
        b = _opt(bias, n, "bias")
        if out is None:
            out = self.empty_typed((m, n), x.dtype)
        assert out.dtype == x.dtype and out.numel() == m * n, "out shape/dtype"
        self._launch("linear_ls_residual", self.lib.hs_linear_ls_residual, _dt(x), _dev(x, "x"),
                     _dev(weight, "weight"), b, g, _dev(res, "res"), _dev(out, "out"), m, n, k)
        return out

    def cache_build(self, frame_out, inter_out, out=None) -> torch.Tensor:
        """Cache::build (model/cache.rs:21-52) in one pass: concat_channels of
        the frame- and inter-block outputs, cast to f32 → (rows, c1+c2) f32."""
        c1, c2 = frame_out.shape[-1], inter_out.shape[-1]
        rows = math.prod(frame_out.shape[:-1])
        assert math.prod(inter_out.shape[:-1]) == rows, "row mismatch"
        assert frame_out.dtype == inter_out.dtype, "cache_build dtype"
        if out is None:
            out = self.empty_typed((rows, c1 + c2), F32)
        assert out.dtype == F32 and out.numel() == rows * (c1 + c2), "out shape/dtype"
        self._launch("cache_build", self.lib.hs_cache_build, _dt(frame_out),
                     _dev(frame_out, "frame_out"), _dev(inter_out, "inter_out"),
                     _dev(out, "out"), rows, c1, c2)
        return out

    def attention_merged(self, q, k, v, out=None) -> torch.Tensor:
        """attention + attn_merge (model/block.rs:148-149) in one pass:
        head-major (S, H, T, D) q, k, v → token-major (S·T, H·D)."""
        assert q.dim() == 4, "attention wants (S,H,T,D)"
        s, h, t, d = q.shape
        assert tuple(k.shape) == tuple(q.shape), "attention: k shape"
        assert tuple(v.shape) == tuple(q.shape), "attention: v shape"
        assert q.dtype == k.dtype == v.dtype, "attention: dtype"
        if out is None:
            out = self.empty_typed((s * t, h * d), q.dtype)
        assert out.dtype == q.dtype and out.numel() == q.numel(), "out shape/dtype"
        self._launch("attention_merged", self.lib.hs_attention_merged, _dt(q), _dev(q, "q"),
                     _dev(k, "k"), _dev(v, "v"), _dev(out, "out"), s, h, t, d)
        return out

    def bias_gelu(self, x, bias=None, out=None) -> torch.Tensor:
        """fc1 bias epilogue + GELU (model/block.rs:173-174)."""
        cols = x.shape[-1]
        rows = x.numel() // cols if cols else 0
        b = _opt(bias, cols, "fc1 bias")
        if out is None:
            out = self.empty_typed(x.shape, x.dtype)
        assert out.dtype == x.dtype and out.numel() == x.numel(), "out shape/dtype"
        self._launch("bias_gelu", self.lib.hs_bias_gelu, _dt(x), _dev(x, "x"), b,
                     _dev(out, "out"), rows, cols)
        return out

    def bias_ls_residual(self, res, x, gamma, bias=None, out=None) -> torch.Tensor:
        """proj/fc2 bias epilogue + LayerScale + residual (model/block.rs:150-155)."""
        assert res.numel() == x.numel() and res.dtype == x.dtype, "res/x shape or dtype"
        dim = x.shape[-1]
        rows = x.numel() // dim if dim else 0
        g = _param(gamma, dim, "gamma")
        b = _opt(bias, dim, "bias")
        if out is None:
            out = self.empty_typed(res.shape, x.dtype)
        assert out.dtype == x.dtype and out.numel() == x.numel(), "out shape/dtype"
        self._launch("bias_ls_residual", self.lib.hs_bias_ls_residual, _dt(x), _dev(res, "res"),
                     _dev(x, "x"), b, g, _dev(out, "out"), rows, dim)
        return out

    def bias_ls_residual_layernorm(self, res, x, gamma, bias, ln, eps: float = 1e-5, out=None,
                                   normed=None):
        """``bias_ls_residual`` then ``layernorm`` of its output in one pass
        (the pre-norm block's residual_ls -> layernorm pairs,
        model/block.rs:150-153, and a block's output into the next block's
        LN1): returns (out, normed), bit-identical to the two calls. ``ln``
        = (weight, bias) of the LayerNorm."""
        assert res.numel() == x.numel() and res.dtype == x.dtype, "res/x shape or dtype"
        dim = x.shape[-1]
        rows = x.numel() // dim if dim else 0
        g = _param(gamma, dim, "gamma")
        b = _opt(bias, dim, "bias")
        lw, lb = _param(ln[0], dim, "norm weight"), _param(ln[1], dim, "norm bias")
        if out is None:
            out = self.empty_typed(res.shape, x.dtype)
        if normed is None:
            normed = self.empty_typed(res.shape, x.dtype)
        for t in (out, normed):
            assert t.dtype == x.dtype and t.numel() == x.numel(), "out/normed shape/dtype"
        self._launch("bias_ls_residual_layernorm", self.lib.hs_bias_ls_residual_layernorm, _dt(x),
                     _dev(res, "res"), _dev(x, "x"), b, g, lw, lb, _dev(out, "out"),
                     _dev(normed, "normed"), rows, dim, eps)
        return out, normed

    def assemble_tokens(self, patches, s: int, p: int, cam, reg, patch_bias=None, pos=None,
                        out_dtype: torch.dtype = F16, n_var: int = 2, out=None) -> torch.Tensor:
        """Token assembly (model/trunk.rs:68-85): per frame
        ``[cam[v], reg[v·R .. v·R+R), patches + bias + pos]`` → (S·T, D)."""
        d = patches.shape[-1]
        assert patches.numel() == s * p * d, "patches shape"
        assert cam.dtype == out_dtype and cam.numel() == n_var * d, "camera token shape/dtype"
        r = reg.numel() // (n_var * d) if reg is not None else 0
        if reg is not None:
            assert reg.dtype == out_dtype and reg.numel() == n_var * r * d, "register token shape"
        b = _opt(patch_bias, d, "patch bias")
        ps = _opt(pos, p * d, "pos embed")
        t = 1 + r + p
        if out is None:
            out = self.empty_typed((s * t, d), out_dtype)
        assert out.dtype == out_dtype and out.numel() == s * t * d, "out shape/dtype"
        self._launch("assemble_tokens", self.lib.hs_assemble_tokens, _dt(out),
                     _dev(patches, "patches"), _dt(patches), b, ps, _dev(cam, "cam"),
                     None if reg is None else _dev(reg, "reg"), _dev(out, "out"), s, p, r, d,
                     n_var)
        return out
