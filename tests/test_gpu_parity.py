"""HIP kernels vs the CPU oracle on identical seeded inputs (small shapes).

Bars: f32 within |a-e| <= 1e-5 + 1e-5|e|; f16 within 2e-3*max(1,|e|) and,
because the fused kernels reproduce the reference's storage rounding points,
within one f16 ulp everywhere; permutations, copies and RoPE passthrough
bit-exact.
"""
import numpy as np
import pytest
import torch

from headshot_amd import rope
from headshot_amd.parity import assert_bit_exact, assert_close, f16_close, ulp_diff_f16
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {torch.float32: np.float32, torch.float16: np.float16}
DTYPES = [torch.float32, torch.float16]


def host(a: np.ndarray, dtype) -> np.ndarray:
    """Storage-typed host copy (f16 by the oracle's RNE)."""
    return O.to_f16(a) if dtype == torch.float16 else np.ascontiguousarray(a, np.float32)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def back(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(got: np.ndarray, want: np.ndarray, what: str, max_ulp: int = 1,
          stages: int = 1):
    """f32: 1e-5 (abs + rel). f16: the 2e-3 gate, plus at most `max_ulp` f16
    ulps wherever |want| >= 1/64 (below that an f16 ulp, <= 2^-16, is close
    to the f32 noise of values that cancel to near zero). With two rounding
    stages (QK-norm stored as f16, then rotated) a 1-ulp flip of the stored
    norm output can move a cancelling rotation by more, so there at most
    0.1% of elements may exceed `max_ulp`."""
    assert got.dtype == want.dtype, f"{what}: dtype {got.dtype} vs {want.dtype}"
    if got.dtype == np.float32:
        assert_close(got, want, 1e-5, what)
    else:
        f16_close(got.astype(np.float32), want.astype(np.float32), what)
        u = ulp_diff_f16(got, want)
        big = np.abs(want.astype(np.float32)) >= 1.0 / 64
        bad = (u > max_ulp) & big
        allowed = 0 if stages == 1 else max(1, big.sum() // 1000)
        assert bad.sum() <= allowed, f"{what}: {int(bad.sum())} elements > {max_ulp} ulp"


# ---------------------------------------------------------------- layernorm

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim", [(1, 1024), (19, 1024), (257, 1024), (19, 300), (33, 64),
                                      (7, 512), (5, 2048), (3, 4096), (11, 100),
                                      # narrow rows: several per wave, ragged last group
                                      (1003, 64), (17, 128), (41, 32), (2, 64)])
def test_layernorm(ctx, dtype, rows, dim):
    x = host(O.normal(11, (rows, dim)), dtype)
    w = O.normal(12, (dim,), 1.0, 0.02)
    b = O.normal(13, (dim,), 0.0, 0.02)
    for eps in (1e-5, 1e-6):
        got = back(ctx.layernorm(dev(x), dev(w), dev(b), eps=eps))
        check(got, O.layernorm(x, w, b, eps), f"layernorm {dtype} {rows}x{dim} eps={eps}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_layernorm_in_place_and_empty(ctx, dtype):
    x = host(O.normal(14, (9, 1024)), dtype)
    w, b = O.normal(15, (1024,), 1.0, 0.02), O.normal(16, (1024,), 0.0, 0.02)
    t = dev(x)
    ctx.layernorm(t, dev(w), dev(b), eps=1e-6, out=t)
    check(back(t), O.layernorm(x, w, b, 1e-6), "layernorm in place")
    x64 = host(O.normal(17, (45, 64)), dtype)
    w64, b64 = O.normal(18, (64,), 1.0, 0.02), O.normal(19, (64,), 0.0, 0.02)
    t64 = dev(x64)
    ctx.layernorm(t64, dev(w64), dev(b64), eps=1e-6, out=t64)
    check(back(t64), O.layernorm(x64, w64, b64, 1e-6), "layernorm 64-wide in place")
    empty = torch.empty((0, 1024), dtype=dtype, device="cuda:0")
    assert ctx.layernorm(empty, dev(w), dev(b)).shape == (0, 1024)


# ------------------------------------------------------ qk-norm + rope (fused)

QK_CASES = [
    # s, t, h, d, prefix, grid (h_p, w_p)
    (2, 11, 16, 64, 5, (2, 3)),
    (2, 21, 16, 64, 5, (4, 4)),
    (3, 37, 8, 64, 17, (4, 5)),
    (3, 6, 32, 64, 2, (2, 2)),    # frames shorter than a token tile: tiles span frames
    (5, 7, 8, 64, 1, (2, 3)),
    (1, 9, 4, 64, 3, (2, 3)),
    (2, 11, 3, 64, 5, (2, 3)),    # H not a multiple of a load's heads: generic path
    (2, 10, 2, 32, 4, (2, 3)),    # head_dim 32: generic path (tables cut to 32 channels)
]


def _tables(t, prefix, grid, d):
    sin, cos = rope.tables(rope.periods(), *grid)
    assert sin.shape[0] == t - prefix
    if d != 64:
        sin, cos = np.ascontiguousarray(sin[:, :d]), np.ascontiguousarray(cos[:, :d])
    return sin, cos


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", QK_CASES)
@pytest.mark.parametrize("norm,use_rope", [(True, True), (True, False), (False, True),
                                           (False, False)])
def test_qknorm_rope(ctx, dtype, case, norm, use_rope):
    s, t, h, d, prefix, grid = case
    x = host(O.normal(21, (s * t, h * d)), dtype)
    nw, nb = O.normal(22, (d,), 1.0, 0.02), O.normal(23, (d,), 0.0, 0.02)
    sin, cos = _tables(t, prefix, grid, d)
    got = back(ctx.qknorm_rope(dev(x), s, t, h, d,
                               norm=(dev(nw), dev(nb)) if norm else None,
                               rope=(dev(sin), dev(cos), prefix) if use_rope else None, eps=1e-6))
    want = O.qknorm_rope(x, nw if norm else None, nb if norm else None,
                         sin if use_rope else None, cos if use_rope else None,
                         s, t, h, d, prefix, 1e-6)
    what = f"qknorm_rope {dtype} {case} norm={norm} rope={use_rope}"
    if not norm and not use_rope:
        assert_bit_exact(got, want, what)  # pure split_heads
        return
    check(got, want, what, stages=2 if (norm and use_rope) else 1)
    if use_rope and not norm:
        # prefix tokens pass through untouched
        xs = x.reshape(s, t, h, d).transpose(0, 2, 1, 3)
        assert_bit_exact(got[:, :, :prefix], np.ascontiguousarray(xs[:, :, :prefix]), what + " prefix")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", QK_CASES)
@pytest.mark.parametrize("norm,use_rope", [(True, True), (True, False), (False, True),
                                           (False, False)])
def test_qknorm_rope_pair(ctx, dtype, case, norm, use_rope):
    """q and k in one launch: bit-identical to two hs_qknorm_rope calls with
    their own norms (row kernel and generic fallback alike), and the oracle
    holds for k."""
    s, t, h, d, prefix, grid = case
    q = host(O.normal(31, (s * t, h * d)), dtype)
    k = host(O.normal(32, (s * t, h * d)), dtype)
    qn = (O.normal(33, (d,), 1.0, 0.02), O.normal(34, (d,), 0.0, 0.02))
    kn = (O.normal(35, (d,), 1.0, 0.02), O.normal(36, (d,), 0.0, 0.02))
    sin, cos = _tables(t, prefix, grid, d)
    rp = (dev(sin), dev(cos), prefix) if use_rope else None
    dq, dk = dev(q), dev(k)
    gq, gk = ctx.qknorm_rope_pair(dq, dk, s, t, h, d,
                                  qn=tuple(dev(a) for a in qn) if norm else None,
                                  kn=tuple(dev(a) for a in kn) if norm else None,
                                  rope=rp, eps=1e-6)
    wq = ctx.qknorm_rope(dq, s, t, h, d, norm=tuple(dev(a) for a in qn) if norm else None,
                         rope=rp, eps=1e-6)
    wk = ctx.qknorm_rope(dk, s, t, h, d, norm=tuple(dev(a) for a in kn) if norm else None,
                         rope=rp, eps=1e-6)
    what = f"qknorm_rope_pair {dtype} {case} norm={norm} rope={use_rope}"
    assert_bit_exact(back(gq), back(wq), what + " q")
    assert_bit_exact(back(gk), back(wk), what + " k")
    want = O.qknorm_rope(k, *(kn if norm else (None, None)), sin if use_rope else None,
                         cos if use_rope else None, s, t, h, d, prefix, 1e-6)
    check(back(gk), want, what + " k oracle", stages=2 if (norm and use_rope) else 1)


def test_qknorm_rope_pair_unaligned_and_shared_input(ctx):
    """Pointers off the 16-byte grid take the generic kernel for both halves;
    q and k may be the same buffer. Each half still equals its single call."""
    s, t, h, d, prefix, grid = 2, 11, 16, 64, 5, (2, 3)
    n = s * t * h * d
    buf = dev(host(O.normal(37, (n + 8,)), torch.float16))
    q = buf[1:1 + n].view(s * t, h * d)           # 2 bytes past a 16-byte boundary
    qn = tuple(dev(a) for a in (O.normal(38, (d,), 1.0, 0.02), O.normal(39, (d,), 0.0, 0.02)))
    kn = tuple(dev(a) for a in (O.normal(40, (d,), 1.0, 0.02), O.normal(41, (d,), 0.0, 0.02)))
    sin, cos = _tables(t, prefix, grid, d)
    rp = (dev(sin), dev(cos), prefix)
    gq, gk = ctx.qknorm_rope_pair(q, q, s, t, h, d, qn=qn, kn=kn, rope=rp, eps=1e-6)
    wq = ctx.qknorm_rope(q, s, t, h, d, norm=qn, rope=rp, eps=1e-6)
    wk = ctx.qknorm_rope(q, s, t, h, d, norm=kn, rope=rp, eps=1e-6)
    assert_bit_exact(back(gq), back(wq), "pair unaligned q")
    assert_bit_exact(back(gk), back(wk), "pair unaligned k")
    want = O.qknorm_rope(back(q), *(back(a) for a in kn), sin, cos, s, t, h, d, prefix, 1e-6)
    check(back(gk), want, "pair unaligned k oracle", stages=2)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("h", [8, 16, 32])
@pytest.mark.parametrize("norm,use_rope", [(True, True), (False, False)])
def test_qknorm_rope_long_sequence(ctx, dtype, h, norm, use_rope):
    """A sequence of 8286 tokens (91x91 grid, prefix 5): from 8192 tokens the
    row kernel gives each wave one load chunk of every row and runs the
    chunks one after another. The pair against the oracle and bit-exact
    against two single calls."""
    s, grid, prefix, d = 1, (91, 91), 5, 64
    t = grid[0] * grid[1] + prefix
    q = host(O.normal(41, (s * t, h * d)), dtype)
    k = host(O.normal(42, (s * t, h * d)), dtype)
    qn = (O.normal(43, (d,), 1.0, 0.02), O.normal(44, (d,), 0.0, 0.02))
    kn = (O.normal(45, (d,), 1.0, 0.02), O.normal(46, (d,), 0.0, 0.02))
    sin, cos = _tables(t, prefix, grid, d)
    rp = (dev(sin), dev(cos), prefix) if use_rope else None
    dq, dk = dev(q), dev(k)
    kw = dict(qn=tuple(dev(a) for a in qn) if norm else None,
              kn=tuple(dev(a) for a in kn) if norm else None)
    gq, gk = ctx.qknorm_rope_pair(dq, dk, s, t, h, d, rope=rp, eps=1e-6, **kw)
    what = f"qknorm_rope long {dtype} h={h} norm={norm} rope={use_rope}"
    assert_bit_exact(back(gq), back(ctx.qknorm_rope(dq, s, t, h, d, norm=kw["qn"], rope=rp,
                                                    eps=1e-6)), what + " q")
    want = O.qknorm_rope(k, *(kn if norm else (None, None)), sin if use_rope else None,
                         cos if use_rope else None, s, t, h, d, prefix, 1e-6)
    if not norm and not use_rope:
        assert_bit_exact(back(gk), want, what + " k")
    else:
        check(back(gk), want, what + " k oracle", stages=2)


@pytest.mark.parametrize("dtype", DTYPES)
def test_qknorm_rope_prefix_equals_t(ctx, dtype):
    s, t, h, d = 2, 5, 16, 64
    x = host(O.normal(24, (s * t, h * d)), dtype)
    nw, nb = O.normal(25, (d,), 1.0, 0.02), O.normal(26, (d,), 0.0, 0.02)
    dummy = torch.zeros(0, dtype=torch.float32, device="cuda:0")
    got = back(ctx.qknorm_rope(dev(x), s, t, h, d, norm=(dev(nw), dev(nb)),
                               rope=(dummy, dummy, t), eps=1e-5))
    want = O.qknorm_rope(x, nw, nb, None, None, s, t, h, d, t, 1e-5)
    check(got, want, "qknorm_rope prefix == T")


# ---------------------------------------------------------- split / rope ops

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 5, 4, 8), (2, 11, 16, 64), (1, 7, 3, 64), (3, 4, 5, 6)])
def test_split_heads(ctx, dtype, shape):
    s, t, h, d = shape
    x = host(O.normal(31, (s * t, h * d)), dtype)
    got = back(ctx.split_heads(dev(x), s, t, h, d))
    assert_bit_exact(got, np.ascontiguousarray(x.reshape(s, t, h, d).transpose(0, 2, 1, 3)),
                     f"split_heads {shape}")
    assert_bit_exact(got, O.split_heads(x, s, t, h, d), f"split_heads {shape} oracle")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [(2, 3, 11, 64, 5, (2, 3)), (2, 4, 21, 64, 5, (4, 4)),
                                  (1, 2, 23, 64, 17, (2, 3)), (2, 2, 7, 64, 7, (2, 3)),
                                  (3, 16, 137, 64, 17, (10, 12)),
                                  (2, 3, 11, 32, 5, (2, 3))])  # head_dim 32: generic kernel
def test_rope_apply(ctx, dtype, case):
    s, h, t, d, prefix, grid = case
    sin, cos = rope.tables(rope.periods(), *grid)
    if t - prefix != sin.shape[0]:
        sin, cos = sin[: t - prefix].copy(), cos[: t - prefix].copy()
    if d != sin.shape[1]:
        sin, cos = np.ascontiguousarray(sin[:, :d]), np.ascontiguousarray(cos[:, :d])
    x = host(O.normal(41, (s, h, t, d)), dtype)
    g = dev(x)
    ctx.rope_apply(g, dev(sin), dev(cos), prefix)
    got = back(g)
    want = O.rope_apply(x, sin, cos, prefix)
    check(got, want, f"rope_apply {case}")
    assert_bit_exact(got[:, :, :prefix], x[:, :, :prefix], "rope prefix passthrough")


# ------------------------------------------------------------- elementwise

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(37, 4096), (5, 1000), (3, 30), (64, 1024), (1, 8),
                                       (300, 3072), (1374, 4096), (97, 1000)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_bias_gelu(ctx, dtype, rows, cols, with_bias):
    """Shapes from one to several row visits per thread, grids rounded to
    the column period (3072 and 1000 columns), the scalar path (30)."""
    x = host(O.normal(51, (rows, cols)) * np.float32(2.0), dtype)
    b = O.normal(52, (cols,), 0.0, 0.02) if with_bias else None
    got = back(ctx.bias_gelu(dev(x), None if b is None else dev(b)))
    what = f"bias_gelu {dtype} {rows}x{cols} bias={with_bias}"
    # the fused op's own semantics (bias sum kept in f32): one ulp
    check(got, O.bias_gelu(x, b, round_bias=False), what)
    # the reference's dispatch sequence (its epilogue stores x + b first):
    # the parity gate
    ref = O.bias_gelu(x, b, round_bias=True)
    if got.dtype == np.float32:
        assert_close(got, ref, 1e-5, what + " vs reference sequence")
    else:
        f16_close(got.astype(np.float32), ref.astype(np.float32), what + " vs reference sequence")


@pytest.mark.parametrize("dtype", DTYPES)
def test_gelu_surface_and_in_place(ctx, dtype):
    for n in (1000, 999, 8, 3):
        x = host(O.normal(53 + n, (n,)) * np.float32(3.0), dtype)
        check(back(ctx.gelu(dev(x))), O.gelu(x), f"gelu n={n}")
    x = host(O.normal(54, (64, 4096)), dtype)
    b = O.normal(55, (4096,), 0.0, 0.02)
    t = dev(x)
    ctx.bias_gelu(t, dev(b), out=t)
    check(back(t), O.bias_gelu(x, b, round_bias=False), "bias_gelu in place")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim", [(37, 1024), (5, 300), (3, 30), (64, 4096), (2, 6)])
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("gamma_kind", ["init", "normal"])
def test_bias_ls_residual(ctx, dtype, rows, dim, with_bias, gamma_kind):
    res = host(O.normal(61, (rows, dim)), dtype)
    x = host(O.normal(62, (rows, dim)), dtype)
    b = O.normal(63, (dim,), 0.0, 0.02) if with_bias else None
    g = np.full(dim, 1e-5, np.float32) if gamma_kind == "init" else O.normal(64, (dim,))
    got = back(ctx.bias_ls_residual(dev(res), dev(x), dev(g), None if b is None else dev(b)))
    check(got, O.bias_ls_residual(res, x, b, g), f"bias_ls_residual {dtype} {rows}x{dim}")


@pytest.mark.parametrize("dtype,rows,dim", [(torch.float16, 70000, 1024), (torch.float32, 40000, 1024),
                                            (torch.float16, 20000, 4096), (torch.float16, 90000, 768),
                                            (torch.float32, 30000, 1200)])
def test_bias_ls_residual_large_grid(ctx, dtype, rows, dim):
    """Above 128 MiB per stream the launch gives each thread two visits
    instead of a fixed workgroup count per CU: the whole tensor (that grid)
    equals its two halves (each below the threshold, the other grid) bit for
    bit, and sampled rows match the oracle."""
    print(f"[bias_ls_residual large grid: {dtype} rows={rows} dim={dim}]", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows)
    res = torch.randn((rows, dim), device="cuda", generator=g).to(dtype)
    x = torch.randn((rows, dim), device="cuda", generator=g).to(dtype)
    gam = torch.randn(dim, device="cuda", generator=g)
    b = torch.randn(dim, device="cuda", generator=g) * 0.02
    whole = ctx.bias_ls_residual(res, x, gam, b)
    h = rows // 2
    halves = torch.cat([ctx.bias_ls_residual(res[:h], x[:h], gam, b),
                        ctx.bias_ls_residual(res[h:], x[h:], gam, b)])
    torch.cuda.synchronize()
    assert torch.equal(whole, halves)
    pick = torch.tensor([0, 1, h - 1, h, rows - 2, rows - 1], device="cuda")
    want = O.bias_ls_residual(back(res[pick]), back(x[pick]), back(b), back(gam))
    check(back(whole[pick]), want, f"bias_ls_residual large grid {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_residual_ls_surface_in_place(ctx, dtype):
    res = host(O.normal(65, (40, 1024)), dtype)
    x = host(O.normal(66, (40, 1024)), dtype)
    g = O.normal(67, (1024,))
    check(back(ctx.residual_ls(dev(res), dev(x), dev(g))), O.residual_ls(res, x, g), "residual_ls")
    t = dev(res)
    ctx.bias_ls_residual(t, dev(x), dev(g), out=t)
    check(back(t), O.residual_ls(res, x, g), "residual_ls in place on res")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim", [(37, 1024), (1, 1024), (1374, 1024), (9, 512), (5, 2048),
                                      (7, 256), (5, 300), (3, 64)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_bias_ls_residual_layernorm(ctx, dtype, rows, dim, with_bias):
    """LayerScale + residual, then the LayerNorm of its output, in one pass:
    bit-exact against hs_bias_ls_residual then hs_layernorm (the one-row
    kernel for 1, 2 or 4 chunks of 64 vectors, the two single ops for other
    widths), and within the bars of the oracle's two dispatches."""
    res = host(O.normal(71, (rows, dim)), dtype)
    x = host(O.normal(72, (rows, dim)), dtype)
    b = O.normal(73, (dim,), 0.0, 0.02) if with_bias else None
    g = O.normal(74, (dim,))  # gamma ~ N(0, 1): the residual branch is visible
    lw, lb = O.normal(75, (dim,), 1.0, 0.02), O.normal(76, (dim,), 0.0, 0.02)
    bd = None if b is None else dev(b)
    out, normed = ctx.bias_ls_residual_layernorm(dev(res), dev(x), dev(g), bd, (dev(lw), dev(lb)),
                                                 eps=1e-6)
    x1 = ctx.bias_ls_residual(dev(res), dev(x), dev(g), bd)
    n2 = ctx.layernorm(x1, dev(lw), dev(lb), eps=1e-6)
    what = f"bias_ls_residual_layernorm {dtype} {rows}x{dim}"
    assert_bit_exact(back(out), back(x1), what + " out")
    assert_bit_exact(back(normed), back(n2), what + " normed")
    want_x1 = O.bias_ls_residual(res, x, b, g)
    check(back(out), want_x1, what + " out vs oracle")
    # the LayerNorm stage on the stored out, then the whole chain (where a
    # 1-ulp difference in out can move a normalised value by more)
    check(back(normed), O.layernorm(back(out), lw, lb, 1e-6), what + " normed vs oracle")
    check(back(normed), O.layernorm(want_x1, lw, lb, 1e-6), what + " chain vs oracle", stages=2)


@pytest.mark.parametrize("dtype,rows", [(torch.float16, 70000), (torch.float32, 40000)])
def test_bias_ls_residual_layernorm_large(ctx, dtype, rows):
    """Above 128 MiB per stream the fused kernel streams all four tensors
    (non-temporal loads and stores): still bit-identical to the two single
    ops, which take their own large-tensor launch shapes."""
    print(f"[bias_ls_residual_layernorm large: {dtype} rows={rows}]", flush=True)
    dim = 1024
    g = torch.Generator(device="cuda").manual_seed(rows + 1)
    res = torch.randn((rows, dim), device="cuda", generator=g).to(dtype)
    x = torch.randn((rows, dim), device="cuda", generator=g).to(dtype)
    gam = torch.randn(dim, device="cuda", generator=g)
    b = torch.randn(dim, device="cuda", generator=g) * 0.02
    lw = 1.0 + 0.02 * torch.randn(dim, device="cuda", generator=g)
    lb = 0.02 * torch.randn(dim, device="cuda", generator=g)
    out, normed = ctx.bias_ls_residual_layernorm(res, x, gam, b, (lw, lb), eps=1e-6)
    x1 = ctx.bias_ls_residual(res, x, gam, b)
    n2 = ctx.layernorm(x1, lw, lb, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(out, x1)
    assert torch.equal(normed, n2)


@pytest.mark.parametrize("dtype", DTYPES)
def test_bias_ls_residual_layernorm_in_place(ctx, dtype):
    """out may be res (the residual stream updated in place)."""
    res = host(O.normal(77, (300, 1024)), dtype)
    x = host(O.normal(78, (300, 1024)), dtype)
    g = O.normal(79, (1024,))
    lw, lb = O.normal(80, (1024,), 1.0, 0.02), O.normal(81, (1024,), 0.0, 0.02)
    t = dev(res)
    _, normed = ctx.bias_ls_residual_layernorm(t, dev(x), dev(g), None, (dev(lw), dev(lb)),
                                               eps=1e-6, out=t)
    x1 = ctx.bias_ls_residual(dev(res), dev(x), dev(g), None)
    assert_bit_exact(back(t), back(x1), "in place out")
    assert_bit_exact(back(normed), back(ctx.layernorm(x1, dev(lw), dev(lb), eps=1e-6)),
                     "in place normed")


def test_cast_to_f16(ctx):
    for n in (1 << 16, 1001, 7, 3, 12293, (1 << 22) + 5):
        x = O.normal(71, (n,)) * np.float32(300.0)
        assert_bit_exact(back(ctx.cast_to_f16(dev(x))), O.cast_to_f16(x), f"cast n={n}")
    edge = np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, -7e4, 6.0e-8, 2.98e-8, 1e-10,
                     np.inf, -np.inf, 0.1, 1.0 / 3], np.float32)
    with np.errstate(over="ignore"):  # 65520 and -7e4 round to +-inf on purpose
        want = edge.astype(np.float16)
    assert_bit_exact(back(ctx.cast_to_f16(dev(edge))), want, "cast edges")


def test_tiled_add_table_stationary(ctx):
    """A table of >= 64K 16-byte vectors takes the vector kernel: odd and even
    repetition counts, several groups of four repetitions with a partial
    last one, and in place."""
    table = O.normal(84, (65536 * 4 + 8,))
    for reps in (1, 3, 4, 9):
        x = O.normal(85 + reps, (reps, table.size))
        assert_bit_exact(back(ctx.tiled_add(dev(x), dev(table))), O.tiled_add(x, table),
                         f"tiled_add x{reps}")
    t = dev(x)
    ctx.tiled_add(t, dev(table), out=t)
    assert_bit_exact(back(t), O.tiled_add(x, table), "tiled_add in place")


def test_tiled_add_and_copy_rows(ctx):
    x = O.normal(81, (6, 10, 4))
    table = O.normal(82, (10, 4))
    assert_bit_exact(back(ctx.tiled_add(dev(x), dev(table))), O.tiled_add(x, table), "tiled_add")
    src = dev(O.normal(83, (10, 24)))
    dst = torch.zeros((7, 24), dtype=torch.float32, device="cuda:0")
    ctx.copy_rows(src, 3, dst, 2, 4)
    want = np.zeros((7, 24), np.float32)
    want[2:6] = back(src)[3:7]
    assert_bit_exact(back(dst), want, "copy_rows")


# ----------------------------------------------------------------- assembly

@pytest.mark.parametrize("out_dtype", DTYPES)
@pytest.mark.parametrize("patch_dtype", DTYPES)
@pytest.mark.parametrize("s,grid,r,d,n_var", [(3, (2, 3), 4, 1024, 2), (2, (2, 3), 16, 256, 2),
                                              (2, (3, 2), 4, 96, 1), (1, (1, 4), 0, 512, 2),
                                              # several waves per patch position, the last
                                              # partial; several workgroup rounds per position
                                              (11, (2, 3), 4, 1024, 2), (37, (3, 3), 4, 256, 2),
                                              # rows of 2048: each wave takes two of a
                                              # row's eight 1 KiB chunks
                                              (5, (3, 4), 4, 2048, 2)])
@pytest.mark.parametrize("bias,pos", [(True, True), (False, False), (True, False)])
def test_assemble_tokens(ctx, out_dtype, patch_dtype, s, grid, r, d, n_var, bias, pos):
    p = grid[0] * grid[1]
    patches = host(O.normal(91, (s * p, d)), patch_dtype)
    nout = NP[out_dtype]
    cam = host(O.normal(92, (n_var, d)), out_dtype)
    reg = host(O.normal(93, (n_var * r, d)), out_dtype) if r else None
    pb = O.normal(94, (d,), 0.0, 0.02) if bias else None
    pe = O.normal(95, (p, d), 0.0, 0.02) if pos else None
    got = back(ctx.assemble_tokens(dev(patches), s, p, dev(cam), None if reg is None else dev(reg),
                                   patch_bias=None if pb is None else dev(pb),
                                   pos=None if pe is None else dev(pe), out_dtype=out_dtype,
                                   n_var=n_var))
    want = O.assemble_tokens(patches, pb, pe, cam, reg if reg is not None else np.zeros((0, d), nout),
                             s, p, r, nout, n_var)
    what = f"assemble {out_dtype}<-{patch_dtype} s={s} p={p} r={r} d={d}"
    assert_bit_exact(got, want, what)


# ------------------------------------------------------------ random sweep

@pytest.mark.parametrize("case", range(12))
def test_fused_ops_random_sweep(ctx, case):
    """Seeded random shapes for every fused per-layer op against the oracle,
    to the bars above: LayerNorm at random rows and widths; the QK-norm +
    RoPE pair at a random grid, prefix, frame count and head count (bit-exact
    against two single calls as well); bias + GELU and bias + LayerScale +
    residual at random shapes; token assembly at random frame counts, grids,
    register counts, widths and variant counts (bit-exact)."""
    rng = np.random.default_rng(700 + case)
    dtype = DTYPES[case % 2]
    tag = f"sweep case {case} {dtype}"

    rows = int(rng.integers(1, 3001))
    dim = int(rng.choice([64, 96, 128, 300, 512, 1024, 2048]))
    x = host(O.normal(701 + case, (rows, dim)), dtype)
    w, b = O.normal(702, (dim,), 1.0, 0.02), O.normal(703, (dim,), 0.0, 0.02)
    check(back(ctx.layernorm(dev(x), dev(w), dev(b), eps=1e-6)), O.layernorm(x, w, b, 1e-6),
          f"{tag} layernorm {rows}x{dim}")

    grid = (int(rng.integers(1, 9)), int(rng.integers(1, 9)))
    prefix = int(rng.integers(0, 18))
    s, h, d = int(rng.integers(1, 6)), int(rng.choice([4, 5, 8, 16, 32])), 64
    t = grid[0] * grid[1] + prefix
    q = host(O.normal(711 + case, (s * t, h * d)), dtype)
    k = host(O.normal(712 + case, (s * t, h * d)), dtype)
    qn = (O.normal(713, (d,), 1.0, 0.02), O.normal(714, (d,), 0.0, 0.02))
    kn = (O.normal(715, (d,), 1.0, 0.02), O.normal(716, (d,), 0.0, 0.02))
    sin, cos = _tables(t, prefix, grid, d)
    rp = (dev(sin), dev(cos), prefix)
    dq, dk = dev(q), dev(k)
    gq, gk = ctx.qknorm_rope_pair(dq, dk, s, t, h, d, qn=tuple(dev(a) for a in qn),
                                  kn=tuple(dev(a) for a in kn), rope=rp, eps=1e-6)
    what = f"{tag} qknorm_rope_pair s={s} t={t} h={h} grid={grid} prefix={prefix}"
    assert_bit_exact(back(gq), back(ctx.qknorm_rope(dq, s, t, h, d, norm=tuple(dev(a) for a in qn),
                                                    rope=rp, eps=1e-6)), what + " q")
    check(back(gk), O.qknorm_rope(k, *kn, sin, cos, s, t, h, d, prefix, 1e-6), what + " k oracle",
          stages=2)

    rows, cols = int(rng.integers(1, 2001)), int(rng.choice([8, 24, 1000, 1024, 4096]))
    x = host(O.normal(721 + case, (rows, cols)) * np.float32(2.0), dtype)
    bg = O.normal(722, (cols,), 0.0, 0.02)
    check(back(ctx.bias_gelu(dev(x), dev(bg))), O.bias_gelu(x, bg, round_bias=False),
          f"{tag} bias_gelu {rows}x{cols}")
    res = host(O.normal(723 + case, (rows, cols)), dtype)
    g = O.normal(724, (cols,))
    check(back(ctx.bias_ls_residual(dev(res), dev(x), dev(g), dev(bg))),
          O.bias_ls_residual(res, x, bg, g), f"{tag} bias_ls_residual {rows}x{cols}")

    s, grid = int(rng.integers(1, 7)), (int(rng.integers(1, 6)), int(rng.integers(1, 6)))
    r, d, n_var = int(rng.integers(0, 9)), int(rng.choice([96, 256, 1024])), int(rng.integers(1, 3))
    p = grid[0] * grid[1]
    patch_dtype = DTYPES[(case // 2) % 2]
    patches = host(O.normal(731 + case, (s * p, d)), patch_dtype)
    cam = host(O.normal(732, (n_var, d)), dtype)
    reg = host(O.normal(733, (n_var * r, d)), dtype) if r else None
    pb = O.normal(734, (d,), 0.0, 0.02) if case % 3 else None
    pe = O.normal(735, (p, d), 0.0, 0.02) if case % 4 else None
    got = back(ctx.assemble_tokens(dev(patches), s, p, dev(cam), None if reg is None else dev(reg),
                                   patch_bias=None if pb is None else dev(pb),
                                   pos=None if pe is None else dev(pe), out_dtype=dtype,
                                   n_var=n_var))
    want = O.assemble_tokens(patches, pb, pe, cam,
                             reg if reg is not None else np.zeros((0, d), NP[dtype]),
                             s, p, r, NP[dtype], n_var)
    assert_bit_exact(got, want, f"{tag} assemble s={s} p={p} r={r} d={d} n_var={n_var}")


# ------------------------------------------------------------ empty inputs

def test_every_op_accepts_empty_inputs(ctx):
    """Zero rows, tokens or frames through every op of the surface: each
    returns an empty result of the right shape and launches nothing that
    touches memory (no fault, HS_OK)."""
    f16, f32 = torch.float16, torch.float32
    d = "cuda:0"
    e = lambda *shape, dt=f16: torch.empty(shape, dtype=dt, device=d)  # noqa: E731
    ones = lambda n: torch.ones(n, dtype=f32, device=d)  # noqa: E731
    assert ctx.bias_gelu(e(0, 4096), ones(4096)).shape == (0, 4096)
    assert ctx.gelu(e(0, 64)).shape == (0, 64)
    assert ctx.bias_ls_residual(e(0, 1024), e(0, 1024), ones(1024), ones(1024)).shape == (0, 1024)
    assert ctx.residual_ls(e(0, 1024), e(0, 1024), ones(1024)).shape == (0, 1024)
    assert ctx.layernorm_stats(e(0, 1024), eps=1e-6).numel() == 0
    q = ctx.qknorm_rope(e(0, 1024), 0, 1374, 16, 64, norm=(ones(64), ones(64)))
    assert q.numel() == 0
    qh, kh = ctx.qknorm_rope_pair(e(0, 1024), e(0, 1024), 0, 1374, 16, 64)
    assert qh.numel() == 0 and kh.numel() == 0
    cam, reg = e(2, 1024), e(2 * 4, 1024)
    assert ctx.assemble_tokens(e(0, 1024, dt=f32), 0, 1369, cam, reg).shape == (0, 1024)
    for s, h, t in ((0, 16, 1374), (2, 16, 0)):
        assert ctx.attention(e(s, h, t, 64), e(s, h, t, 64), e(s, h, t, 64)).numel() == 0
        assert ctx.attention_merged(e(s, h, t, 64), e(s, h, t, 64), e(s, h, t, 64)).numel() == 0
    w = torch.zeros((256, 1024), dtype=f16, device=d)
    assert ctx.linear(e(0, 1024), w, ones(256)).shape == (0, 256)
    assert ctx.linear_gelu(e(0, 1024), w, ones(256)).shape == (0, 256)
    assert ctx.linear_ls_residual(e(0, 1024), w, ones(256), e(0, 256), ones(256)).shape == (0, 256)
    assert ctx.cache_build(e(0, 1024), e(0, 1024)).shape == (0, 2048)
    ln = (ones(1024), ones(1024))
    o, nrm = ctx.bias_ls_residual_layernorm(e(0, 1024), e(0, 1024), ones(1024), ones(1024), ln)
    assert o.shape == (0, 1024) and nrm.shape == (0, 1024)
    assert ctx.linear_ln(e(0, 1024), ln, w, ones(256)).shape == (0, 256)
    assert ctx.linear_ln_gelu(e(0, 1024), ln, w, ones(256)).shape == (0, 256)
    wqkv = torch.zeros((3072, 1024), dtype=f16, device=d)
    outs = ctx.linear_ln_qkv_heads(e(0, 1024), ln, wqkv, ones(3072), 0, 1374, 16,
                                   qn=(ones(64), ones(64)), kn=(ones(64), ones(64)))
    assert all(o.numel() == 0 for o in outs)
    # the allocation-free entry: zero rows return before its array is used
    from headshot_amd import _lib
    L = _lib.load()
    rc = L.hs_linear_ln_gelu_noalloc(torch.cuda.current_stream().cuda_stream, _lib.HS_F16,
                                     e(0, 1024).data_ptr(), ln[0].data_ptr(), ln[1].data_ptr(),
                                     w.data_ptr(), None, e(0, 256).data_ptr(), 0, 256, 1024, 1e-6)
    assert rc == _lib.HS_OK, L.hs_last_error().decode()
    torch.cuda.synchronize()


def test_every_op_f16_matches_f32(ctx):
    """The reference's every_op_f16_matches_f32 (tests/f16_ops.rs:36-123) on
    the HIP ops: each op's f16 variant against its f32 variant on the same
    f16-exact inputs in [-1, 1) (its rvec), with its max-abs tolerances:
    layernorm 2e-2, gelu 2e-3, residual_ls 2e-3, split_heads and attn_merge
    1e-6 (exact), rope_apply 2e-3, concat_channels 1e-6 (exact)."""
    s, h, t, d = 2, 4, 21, 64
    c, rows = h * d, s * t

    def both(a):
        return (torch.from_numpy(a.astype(np.float32)).to("cuda:0"),
                torch.from_numpy(a.astype(np.float16)).to("cuda:0"))

    def close(got16, got32, tol, what):
        a, b = back(got16).astype(np.float32), back(got32).astype(np.float32)
        assert np.count_nonzero(b) > 0, f"{what}: f32 output is all zero"
        assert np.count_nonzero(a) > 0, f"{what}: f16 output is all zero"
        err = np.abs(a - b).max()
        assert err < tol, f"{what}: max diff {err} >= {tol}"

    x32, x16 = both(O.rvec_f16(1, rows * c).reshape(rows, c))
    w = torch.from_numpy(O.rvec_f16(2, c)).to("cuda:0")
    b = torch.from_numpy(O.rvec_f16(3, c)).to("cuda:0")
    close(ctx.layernorm(x16, w, b), ctx.layernorm(x32, w, b), 2e-2, "layernorm")
    close(ctx.gelu(x16), ctx.gelu(x32), 2e-3, "gelu")
    r32, r16 = both(O.rvec_f16(4, rows * c).reshape(rows, c))
    g = torch.from_numpy(O.rvec_f16(5, c)).to("cuda:0")
    close(ctx.residual_ls(r16, x16, g), ctx.residual_ls(r32, x32, g), 2e-3, "residual_ls")
    q32, q16 = both(O.rvec_f16(6, rows * c).reshape(rows, c))
    hq32, hq16 = ctx.split_heads(q32, s, t, h, d), ctx.split_heads(q16, s, t, h, d)
    close(hq16, hq32, 1e-6, "split_heads")
    close(ctx.attn_merge(hq16), ctx.attn_merge(hq32), 1e-6, "attn_merge")
    sin, cos = rope.tables(rope.periods(), 4, 4)
    sin_t, cos_t = dev(sin), dev(cos)
    prefix = t - 16
    g32, g16 = both(O.rvec_f16(7, s * h * t * d).reshape(s, h, t, d))
    ctx.rope_apply(g32, sin_t, cos_t, prefix)
    ctx.rope_apply(g16, sin_t, cos_t, prefix)
    close(g16, g32, 2e-3, "rope_apply")
    a32, a16 = both(O.rvec_f16(8, rows * 8).reshape(rows, 8))
    c32, c16 = both(O.rvec_f16(9, rows * 24).reshape(rows, 24))
    close(ctx.concat_channels(a16, c16), ctx.concat_channels(a32, c32), 1e-6, "concat_channels")
