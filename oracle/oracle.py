"""TEST INFRASTRUCTURE ONLY — numpy front end of the CPU oracle (hs_oracle.c).

The oracle restates headshot's per-layer WGSL kernels and host RoPE tables in
plain C (f32 arithmetic, no FMA contraction, f16 storage rounded to nearest
even where the reference stores). Only ``tests/``, ``__graft_entry__.smoke()``
and bench.py's ``cpu_baseline`` leg may import this module; the product path
(``headshot_amd``) never does.

Arrays are numpy ``float32`` or ``float16`` (storage dtype of the reference's
``Elem``). Norm weights, biases, LayerScale gammas and RoPE tables are always
``float32`` (crates/headshot-server/src/engine/ops.rs:5-8).

What pins each function independently of this code (tests/test_oracle.py):

=====================  ========================================================
function               pinned by
=====================  ========================================================
f16 conversion         numpy ``astype(float16)`` on random + edge-case floats
rope_periods           engine/rope.rs:61-67 values; correctly rounded 100**x
rope_tables            engine/rope.rs:70-90 closed forms; an independent numpy
                       restatement of the angle arithmetic with libm sinf/cosf
                       called through ctypes; correctly rounded sin/cos of the
                       same f32 angles; committed SHA-256 fixtures
rope_apply_cpu/apply   complex rotation (lo + i hi) * exp(i theta) in f64;
                       pair-norm preservation (engine/rope.rs:92-103)
layernorm              float64 torch.nn.functional.layer_norm; the reference
                       test layernorm_matches_cpu (tests/kernels.rs:100-126)
split_heads/merge      numpy reshape/transpose (exact); tests/kernels.rs:241-274
linear                 float64 numpy x @ w.T + b at f32 tolerance; small-
                       integer inputs (exact in every precision) bit-exact
concat/cast/cache      numpy concatenate + astype(float32), exact
attention              float64 full-matrix softmax as tests/kernels.rs:194-238
                       (1e-4); invariants: constant V rows, q = 0 gives the
                       mean of V, key permutation, T = 1 returns v
gelu                   f64 math.erf at 1e-5 (tests/kernels.rs:128-147)
residual_ls, bias,     numpy closed forms in float64 vs tolerance; f16
cast, tiled_add        rounding points checked against numpy float16
assemble_tokens        numpy concatenation (bit-exact for f32 patches)
=====================  ========================================================
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16 = 0, 1

_lib = None


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-B", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float


def _declare(L):
    sig = {
        "or_f32_to_f16": (ctypes.c_uint16, [_F]),
        "or_f16_to_f32": (_F, [ctypes.c_uint16]),
        "or_f32_to_f16_array": (None, [_P, _P, _I64]),
        "or_f16_to_f32_array": (None, [_P, _P, _I64]),
        "or_rope_periods": (None, [_P]),
        "or_rope_tables": (None, [_P, _I32, _I32, _P, _P]),
        "or_rope_apply_cpu": (None, [_P, _P, _P, _I64, _P]),
        "or_layernorm": (None, [ctypes.c_int, _P, _P, _P, _P, _I64, _I32, _F]),
        "or_split_heads": (None, [ctypes.c_int, _P, _P, _I32, _I32, _I32, _I32]),
        "or_attn_merge": (None, [ctypes.c_int, _P, _P, _I32, _I32, _I32, _I32]),
        "or_linear": (None, [ctypes.c_int, _P, _P, _P, _P, _I64, _I32, _I32, _P, _I64]),
        "or_concat_channels": (None, [ctypes.c_int, _P, _P, _P, _I64, _I32, _I32]),
        "or_cast_f16_to_f32": (None, [_P, _P, _I64]),
        "or_cache_build": (None, [ctypes.c_int, _P, _P, _P, _I64, _I32, _I32]),
        "or_attention": (None, [ctypes.c_int, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _I32]),
        "or_rope_apply": (None, [ctypes.c_int, _P, _P, _P, _I32, _I32, _I32, _I32, _I32]),
        "or_erf_as": (_F, [_F]),
        "or_gelu": (None, [ctypes.c_int, _P, _P, _I64]),
        "or_residual_ls": (None, [ctypes.c_int, _P, _P, _P, _P, _I64, _I32]),
        "or_add_bias": (None, [ctypes.c_int, _P, _P, _P, _I64, _I32]),
        "or_cast_f32_to_f16": (None, [_P, _P, _I64]),
        "or_tiled_add": (None, [_P, _P, _P, _I64, _I64]),
        "or_qknorm_rope": (None, [ctypes.c_int, _P, _P, _P, _P, _P, _P,
                                  _I32, _I32, _I32, _I32, _I32, _F]),
        "or_bias_gelu": (None, [ctypes.c_int, _P, _P, _P, _I64, _I32, ctypes.c_int]),
        "or_bias_ls_residual": (None, [ctypes.c_int, _P, _P, _P, _P, _P, _I64, _I32]),
        "or_assemble_tokens": (None, [ctypes.c_int, _P, ctypes.c_int, _P, _P, _P, _P, _P,
                                      _I32, _I32, _I32, _I32, _I32]),
        "or_block_ops": (None, [ctypes.c_int] + [_P] * 11 + [_I32] + [_P] * 10
                         + [_P] * 7 + [_I32] * 5 + [_F]),
        "or_num_threads": (ctypes.c_int, []),
        "or_set_num_threads": (None, [ctypes.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _dt(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise TypeError(f"oracle storage must be float32 or float16, got {a.dtype}")


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be C-contiguous"
    return a.ctypes.data


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


# --------------------------------------------------------------------------
# conversions


def to_f16(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.float16)
    lib().or_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


# --------------------------------------------------------------------------
# RoPE (engine/rope.rs)


def rope_periods() -> np.ndarray:
    out = np.empty(16, np.float32)
    lib().or_rope_periods(_ptr(out))
    return out


def rope_tables(periods: np.ndarray, h_p: int, w_p: int):
    periods = _f32(periods)
    assert periods.shape == (16,)
    p = h_p * w_p
    sin = np.empty((p, 64), np.float32)
    cos = np.empty((p, 64), np.float32)
    lib().or_rope_tables(_ptr(periods), h_p, w_p, _ptr(sin), _ptr(cos))
    return sin, cos


def rope_apply_cpu(x64: np.ndarray, sin: np.ndarray, cos: np.ndarray, table_row: int):
    x64 = _f32(x64)
    out = np.empty(64, np.float32)
    lib().or_rope_apply_cpu(_ptr(x64), _ptr(sin), _ptr(cos), table_row, _ptr(out))
    return out


# --------------------------------------------------------------------------
# single reference dispatches


def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x)
    dim = x.shape[-1]
    rows = x.size // dim if dim else 0
    w, b = _f32(w), _f32(b)
    assert w.shape == (dim,) and b.shape == (dim,)
    out = np.empty_like(x)
    lib().or_layernorm(_dt(x), _ptr(x), _ptr(w), _ptr(b), _ptr(out), rows, dim, eps)
    return out


def split_heads(x: np.ndarray, s: int, t: int, h: int, d: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    assert x.size == s * t * h * d
    out = np.empty((s, h, t, d), x.dtype)
    lib().or_split_heads(_dt(x), _ptr(x), _ptr(out), s, t, h, d)
    return out


def attn_merge(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    s, h, t, d = x.shape
    out = np.empty((s * t, h * d), x.dtype)
    lib().or_attn_merge(_dt(x), _ptr(x), _ptr(out), s, t, h, d)
    return out


def linear(x: np.ndarray, w: np.ndarray, bias=None, rows=None) -> np.ndarray:
    """linear.wesl: x (m, k) @ w (n, k)^T [+ bias], stored in x's dtype.
    ``rows`` (indices into x's rows) computes only those rows."""
    x, w = np.ascontiguousarray(x), np.ascontiguousarray(w)
    assert x.dtype == w.dtype
    k = x.shape[-1]
    m = x.size // k
    n = w.shape[0]
    assert w.shape[1] == k
    b = None if bias is None else _f32(bias)
    idx = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    nr = m if idx is None else idx.size
    out = np.empty((nr, n), x.dtype)
    lib().or_linear(_dt(x), _ptr(x), _ptr(w), _ptr(b), _ptr(out), m, n, k,
                    None if idx is None else _ptr(idx), nr)
    return out


def linear_gelu(x, w, bias=None, rows=None):
    """The reference sequence linear (stores Elem) -> gelu (block.rs:172-176)."""
    return gelu(linear(x, w, bias, rows))


def linear_ls_residual(x, w, gamma, res, bias=None, rows=None):
    """The reference sequence linear -> residual_ls (block.rs:150-155)."""
    y = linear(x, w, bias, rows)
    r = res if rows is None else np.ascontiguousarray(res[rows])
    return residual_ls(r, y, gamma)


def concat_channels(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """concat_channels.wesl: (rows, c1) ++ (rows, c2) → (rows, c1 + c2)."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    assert a.dtype == b.dtype
    c1, c2 = a.shape[-1], b.shape[-1]
    rows = int(np.prod(a.shape[:-1]))
    assert int(np.prod(b.shape[:-1])) == rows
    out = np.empty((rows, c1 + c2), a.dtype)
    lib().or_concat_channels(_dt(a), _ptr(a), _ptr(b), _ptr(out), rows, c1, c2)
    return out


def cast_to_f32(x: np.ndarray) -> np.ndarray:
    """cast_f16_to_f32.wesl."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    out = np.empty(x.shape, np.float32)
    lib().or_cast_f16_to_f32(_ptr(x), _ptr(out), x.size)
    return out


def cache_build(frame_out: np.ndarray, inter_out: np.ndarray) -> np.ndarray:
    """Cache::build (model/cache.rs:37-44) over all rows: f32 (rows, c1 + c2)."""
    a, b = np.ascontiguousarray(frame_out), np.ascontiguousarray(inter_out)
    assert a.dtype == b.dtype
    c1, c2 = a.shape[-1], b.shape[-1]
    rows = int(np.prod(a.shape[:-1]))
    assert int(np.prod(b.shape[:-1])) == rows
    out = np.empty((rows, c1 + c2), np.float32)
    lib().or_cache_build(_dt(a), _ptr(a), _ptr(b), _ptr(out), rows, c1, c2)
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_idx=None) -> np.ndarray:
    """attention.wesl over head-major (S, H, T, D). With ``q_idx`` (query
    indices) only those queries are computed: the result is (S, H, len, D)."""
    q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
    assert q.shape == k.shape == v.shape and q.dtype == k.dtype == v.dtype
    s, h, t, d = q.shape
    assert d % 4 == 0 and d <= 128
    idx = None if q_idx is None else np.ascontiguousarray(q_idx, dtype=np.int32)
    nq = t if idx is None else idx.size
    if idx is not None:
        assert idx.size == 0 or (idx.min() >= 0 and idx.max() < t)
    out = np.empty((s, h, nq, d), q.dtype)
    lib().or_attention(_dt(q), _ptr(q), _ptr(k), _ptr(v), _ptr(out), s, h, t, d,
                       None if idx is None else _ptr(idx), nq)
    return out


def rope_apply(x: np.ndarray, sin: np.ndarray, cos: np.ndarray, prefix: int) -> np.ndarray:
    """Returns the rotated copy of head-major ``x`` (S, H, T, D)."""
    out = np.array(x, copy=True, order="C")
    s, h, t, d = out.shape
    sin, cos = _f32(sin), _f32(cos)
    assert sin.size == (t - prefix) * d and cos.size == sin.size
    lib().or_rope_apply(_dt(out), _ptr(out), _ptr(sin), _ptr(cos), s, h, t, d, prefix)
    return out


def erf_as(v: float) -> float:
    return lib().or_erf_as(v)


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    out = np.empty_like(x)
    lib().or_gelu(_dt(x), _ptr(x), _ptr(out), x.size)
    return out


def residual_ls(res: np.ndarray, x: np.ndarray, gamma: np.ndarray) -> np.ndarray:
    res, x, gamma = np.ascontiguousarray(res), np.ascontiguousarray(x), _f32(gamma)
    assert res.size == x.size and res.dtype == x.dtype and x.size % gamma.size == 0
    out = np.empty_like(res)
    lib().or_residual_ls(_dt(x), _ptr(res), _ptr(x), _ptr(gamma), _ptr(out), x.size, gamma.size)
    return out


def add_bias(x: np.ndarray, bias: np.ndarray) -> np.ndarray:
    x, bias = np.ascontiguousarray(x), _f32(bias)
    cols = bias.size
    out = np.empty_like(x)
    lib().or_add_bias(_dt(x), _ptr(x), _ptr(bias), _ptr(out), x.size // cols, cols)
    return out


def cast_to_f16(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.float16)
    lib().or_cast_f32_to_f16(_ptr(x), _ptr(out), x.size)
    return out


def tiled_add(x: np.ndarray, table: np.ndarray) -> np.ndarray:
    x, table = _f32(x), _f32(table)
    assert x.size % table.size == 0
    out = np.empty_like(x)
    lib().or_tiled_add(_ptr(x), _ptr(table), _ptr(out), x.size, table.size)
    return out


# --------------------------------------------------------------------------
# composites: the reference's unfused sequence behind each fused operation


def qknorm_rope(x_tok, nw, nb, sin, cos, s, t, h, d, prefix, eps=1e-5):
    x_tok = np.ascontiguousarray(x_tok)
    assert x_tok.size == s * t * h * d
    out = np.empty((s, h, t, d), x_tok.dtype)
    nw = None if nw is None else _f32(nw)
    nb = None if nb is None else _f32(nb)
    sin = None if sin is None else _f32(sin)
    cos = None if cos is None else _f32(cos)
    lib().or_qknorm_rope(_dt(x_tok), _ptr(x_tok), _ptr(nw), _ptr(nb), _ptr(sin), _ptr(cos),
                         _ptr(out), s, t, h, d, prefix, eps)
    return out


def bias_gelu(x, bias, round_bias: bool = True):
    """round_bias: store x + bias in the storage dtype before GELU (the
    reference's GEMM epilogue); False keeps the sum in f32 (single rounding)."""
    x = np.ascontiguousarray(x)
    cols = x.shape[-1]
    bias = None if bias is None else _f32(bias)
    out = np.empty_like(x)
    lib().or_bias_gelu(_dt(x), _ptr(x), _ptr(bias), _ptr(out), x.size // cols, cols,
                       int(round_bias))
    return out


def bias_ls_residual(res, x, bias, gamma):
    res, x = np.ascontiguousarray(res), np.ascontiguousarray(x)
    dim = x.shape[-1]
    bias = None if bias is None else _f32(bias)
    gamma = _f32(gamma)
    out = np.empty_like(res)
    lib().or_bias_ls_residual(_dt(x), _ptr(res), _ptr(x), _ptr(bias), _ptr(gamma), _ptr(out),
                              x.size // dim, dim)
    return out


def assemble_tokens(patches, patch_bias, pos, cam, reg, s, p, r, out_dtype, n_var=2):
    patches = np.ascontiguousarray(patches)
    d = patches.shape[-1]
    cam = np.ascontiguousarray(cam, dtype=out_dtype)
    reg = np.ascontiguousarray(reg, dtype=out_dtype)
    patch_bias = None if patch_bias is None else _f32(patch_bias)
    pos = None if pos is None else _f32(pos)
    out = np.empty((s * (p + 1 + r), d), out_dtype)
    lib().or_assemble_tokens(_dt(out), _ptr(patches), _dt(patches), _ptr(patch_bias), _ptr(pos),
                             _ptr(cam), _ptr(reg), _ptr(out), s, p, r, d, n_var)
    return out


def block_ops(dt, x, ln1_w, ln1_b, q_raw, k_raw, qn_w, qn_b, kn_w, kn_b, sin, cos, prefix,
              proj_raw, proj_b, ls1, ln2_w, ln2_b, fc1_raw, fc1_b, fc2_raw, fc2_b, ls2,
              out, s, t, dim, heads, hidden, eps):
    """One block's per-layer ops in reference order; ``out`` is a dict of
    preallocated outputs: normed, q_head, k_head, x1, normed2, act, x_out."""
    lib().or_block_ops(
        dt, _ptr(x), _ptr(ln1_w), _ptr(ln1_b), _ptr(q_raw), _ptr(k_raw), _ptr(qn_w), _ptr(qn_b),
        _ptr(kn_w), _ptr(kn_b), _ptr(sin), _ptr(cos), prefix, _ptr(proj_raw), _ptr(proj_b),
        _ptr(ls1), _ptr(ln2_w), _ptr(ln2_b), _ptr(fc1_raw), _ptr(fc1_b), _ptr(fc2_raw),
        _ptr(fc2_b), _ptr(ls2), _ptr(out["normed"]), _ptr(out["q_head"]), _ptr(out["k_head"]),
        _ptr(out["x1"]), _ptr(out["normed2"]), _ptr(out["act"]), _ptr(out["x_out"]),
        s, t, dim, heads, hidden, eps)


def num_threads() -> int:
    return lib().or_num_threads()


def set_num_threads(n: int) -> None:
    lib().or_set_num_threads(n)


# --------------------------------------------------------------------------
# deterministic inputs (tests/kernels.rs:7-23, tests/f16_ops.rs:7-19)

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix_z(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        k = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + k * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def rng_vec(seed: int, n: int) -> np.ndarray:
    """``Rng(seed).vec(n)`` of tests/kernels.rs:7-23, bit for bit:
    ``(z >> 40) as f32 / 2^23 * 2 - 1`` (which spans [-1, 3))."""
    top = (_splitmix_z(seed, n) >> np.uint64(40)).astype(np.float32)
    v = top / np.float32(1 << 23)
    v = v * np.float32(2.0)
    return (v - np.float32(1.0)).astype(np.float32)


def rvec(seed: int, n: int) -> np.ndarray:
    """``rvec(seed, n)`` of tests/dense_kernels.rs:6-17, bit for bit:
    ``(z >> 40) as f32 / 2^24 * 2 - 1``, values in [-1, 1). That function
    stops before SplitMix64's last ``z ^ (z >> 31)``, which leaves the top
    24 bits unchanged, so the shared generator gives the same values."""
    top = (_splitmix_z(seed, n) >> np.uint64(40)).astype(np.float32)
    v = top / np.float32(1 << 24)
    v = v * np.float32(2.0)
    return (v - np.float32(1.0)).astype(np.float32)


def rvec_f16(seed: int, n: int) -> np.ndarray:
    """``rvec(seed, n)`` of tests/f16_ops.rs:7-19: f16-exact values in [-1, 1)."""
    return f16_to_f32(to_f16(rvec(seed, n)))


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Seeded N(mean, std) via SplitMix64 uniforms and Box-Muller, float32."""
    n = int(np.prod(shape)) if shape else 1
    m = (n + 1) // 2
    z = _splitmix_z(seed, 2 * m)
    u = ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    g = np.empty(2 * m, np.float64)
    g[0::2] = r * np.cos(2.0 * np.pi * u2)
    g[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (g[:n] * std + mean).astype(np.float32).reshape(shape)
