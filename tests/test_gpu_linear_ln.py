"""LayerNorm as the prologue of the linear layer after it (hs_layernorm_stats,
hs_linear_ln, hs_linear_ln_gelu, hs_linear_ln_qkv_heads): Block::forward's
LN1 -> q|k|v and LN2 -> fc1 -> GELU pairs (model/block.rs:128-146, 153,
172-176) in one product, whose x tiles are normalised and rounded to the
storage type in LDS, as the reference's layernorm stores its output
(shaders/layernorm.wesl:76), before the matrix cores read them.

Bars:
- bit-exact against this library's own unfused sequence (hs_layernorm, then
  hs_linear / hs_linear_gelu / hs_linear_qkv_heads), which the prologue
  reproduces operand for operand; this covers the matrix-core path at 1, 2,
  3 and 16 k stages (the pipeline's peeled last steps) and partial row
  tiles, and the generic path (f32, n not a multiple of 256);
- against the oracle's restatement of the reference's dispatches
  (layernorm, linear, gelu / split_heads + QK-norm + RoPE): f32 within 4e-5
  relative, f16 within the gate 2e-3 * max(1, |e|);
- the statistics: against float64 and bit-exact to what hs_layernorm
  normalises with.
"""
import numpy as np
import pytest
import torch

from headshot_amd import rope
from headshot_amd.parity import assert_bit_exact, assert_close, f16_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {torch.float32: np.float32, torch.float16: np.float16}


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def back(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(got, want, what):
    if got.dtype == np.float32:
        assert_close(got, want, 4e-5, what)
    else:
        f16_close(got.astype(np.float32), want.astype(np.float32), what)


def ln_operands(seed, m, n, k, dt, mean=0.0):
    """x ~ N(mean, 1) rows, LN gamma N(1, .02) / beta N(0, .02), w ~ N(0,
    1/k), bias N(0, .02), as the benchmark configurations draw them."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) + mean).astype(dt)
    g = (1.0 + 0.02 * rng.standard_normal(k)).astype(np.float32)
    be = (0.02 * rng.standard_normal(k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(dt)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    return x, g, be, w, b


def reference_ln_linear(x, g, be, w, b, eps):
    """layernorm (output stored in x's dtype) then linear: the oracle's
    restatement of the reference's two dispatches."""
    return O.linear(O.layernorm(x, g, be, eps), w, b)


@pytest.mark.parametrize("rows,dim", [(1, 1024), (19, 1024), (257, 1024), (300, 300), (64, 2048),
                                      (77, 64), (41, 128), (33, 192)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_layernorm_stats(ctx, rows, dim, dtype):
    rng = np.random.default_rng(rows + dim)
    x = (rng.standard_normal((rows, dim)) * 3 + 0.5).astype(NP[dtype])
    st = back(ctx.layernorm_stats(dev(x), eps=1e-6))
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1)
    inv = 1.0 / np.sqrt(x64.var(axis=1) + 1e-6)
    assert_close(st[:, 0], mu.astype(np.float32), 1e-5, "mean")
    assert_close(st[:, 1], inv.astype(np.float32), 1e-5, "rstd")
    # the same statistics hs_layernorm normalises with: unit weight, zero
    # bias, so each output is f16((x - mean) * rstd) of those statistics
    ones = torch.ones(dim, device="cuda:0")
    zeros = torch.zeros(dim, device="cuda:0")
    normed = back(ctx.layernorm(dev(x), ones, zeros, eps=1e-6))
    mine = ((x.astype(np.float32) - st[:, :1]) * st[:, 1:]).astype(NP[dtype])
    assert_bit_exact(normed, mine, f"stats of hs_layernorm {rows}x{dim}")


# (m, n, k): k = 64, 128, 192 run the f16 matrix-core pipeline with 1, 2
# and 3 stages (its peeled last steps alone), 1024 with 16; m = 1, 19, 257
# and 300 leave partial row tiles; n = 48 takes the generic kernel; f32
# takes the f32 matrix-core kernel in 64 x 128 tiles (n % 128 == 0).
SHAPES = [(1, 256, 1024), (19, 256, 1024), (257, 512, 1024), (300, 256, 64), (300, 256, 128),
          (300, 256, 192), (37, 48, 80), (1374, 1024, 1024), (600, 256, 2048)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("mean", [0.0, 4.0])
def test_linear_ln(ctx, m, n, k, dtype, mean):
    """mean 4 puts the rows' mean well above their spread."""
    x, g, be, w, b = ln_operands(m * 3 + n + k, m, n, k, NP[dtype], mean)
    xd, gd, bed, wd, bd = map(dev, (x, g, be, w, b))
    got = back(ctx.linear_ln(xd, (gd, bed), wd, bd, eps=1e-6))
    what = f"linear_ln {(m, n, k)} {dtype} mean {mean}"
    seq = back(ctx.linear(ctx.layernorm(xd, gd, bed, eps=1e-6), wd, bd))
    assert_bit_exact(got, seq, what + " against layernorm then linear")
    check(got, reference_ln_linear(x, g, be, w, b, 1e-6), what)


@pytest.mark.parametrize("m,n,k", [(300, 256, 1024), (37, 48, 80), (1374, 4096, 1024),
                                   (257, 512, 128)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_linear_ln_gelu(ctx, m, n, k, dtype):
    x, g, be, w, b = ln_operands(m + 7 * n + k, m, n, k, NP[dtype])
    xd, gd, bed, wd, bd = map(dev, (x, g, be, w, b))
    got = back(ctx.linear_ln_gelu(xd, (gd, bed), wd, bd, eps=1e-6))
    what = f"linear_ln_gelu {(m, n, k)} {dtype}"
    seq = back(ctx.linear_gelu(ctx.layernorm(xd, gd, bed, eps=1e-6), wd, bd))
    assert_bit_exact(got, seq, what + " against layernorm then linear_gelu")
    # the reference's sequence: the linear's storage rounding, then gelu
    check(got, O.gelu(reference_ln_linear(x, g, be, w, b, 1e-6)), what)


@pytest.mark.parametrize("m,n,k", [(8300, 1024, 256), (12345, 768, 96), (3000, 1024, 32),
                                   (700, 512, 2048)])
def test_linear_ln_f32_tile_shapes(ctx, m, n, k):
    """The f32 prologue in both tile shapes of the f32 matrix-core kernel:
    128 x 128 tiles (at least 512 of them: 8300 and 12345 rows, last row
    tiles of 108 and 57 rows) and 64 x 128 (3000 rows, one k stage), each
    bit-exact against layernorm then the product and within the f32 bar of
    the oracle's sequence."""
    x, g, be, w, b = ln_operands(m + n + 3 * k, m, n, k, np.float32, 2.0)
    xd, gd, bed, wd, bd = map(dev, (x, g, be, w, b))
    normed = ctx.layernorm(xd, gd, bed, eps=1e-6)
    got = back(ctx.linear_ln(xd, (gd, bed), wd, bd, eps=1e-6))
    assert_bit_exact(got, back(ctx.linear(normed, wd, bd)), f"f32 linear_ln {(m, n, k)}")
    got_g = back(ctx.linear_ln_gelu(xd, (gd, bed), wd, bd, eps=1e-6))
    assert_bit_exact(got_g, back(ctx.linear_gelu(normed, wd, bd)), f"f32 linear_ln_gelu {(m, n, k)}")
    rows = np.array([0, 1, 63, 64, 127, 128, m - 1])
    want = O.linear(O.layernorm(x, g, be, 1e-6)[rows], w, b)
    check(got[rows], want, f"f32 linear_ln {(m, n, k)} vs oracle")


def test_linear_ln_without_bias(ctx):
    x, g, be, w, _ = ln_operands(3, 513, 256, 1024, np.float16)
    xd, gd, bed, wd = map(dev, (x, g, be, w))
    got = back(ctx.linear_ln(xd, (gd, bed), wd, None, eps=1e-6))
    seq = back(ctx.linear(ctx.layernorm(xd, gd, bed, eps=1e-6), wd, None))
    assert_bit_exact(got, seq, "linear_ln without bias")


def qk_norms(d, seed=5):
    rng = np.random.default_rng(seed)
    return tuple(((1 + 0.02 * rng.standard_normal(d)).astype(np.float32),
                  (0.02 * rng.standard_normal(d)).astype(np.float32)) for _ in range(2))


@pytest.mark.parametrize("frames,grid,heads,rope_on", [(2, (37, 37), 16, True),
                                                       (1, (8, 8), 16, False),
                                                       (3, (4, 6), 8, True)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_linear_ln_qkv_heads(ctx, frames, grid, heads, rope_on, dtype):
    prefix = 5
    t = grid[0] * grid[1] + prefix
    d, dim = 64, heads * 64
    m = frames * t
    x, g, be, w, b = ln_operands(frames * 31 + heads, m, 3 * dim, dim, NP[dtype])
    qn, kn = qk_norms(d)
    sin, cos = rope.tables(rope.periods(), *grid)
    rp = (dev(sin), dev(cos), prefix) if rope_on else None
    xd, gd, bed, wd, bd = map(dev, (x, g, be, w, b))
    qnd, knd = tuple(map(dev, qn)), tuple(map(dev, kn))
    got = ctx.linear_ln_qkv_heads(xd, (gd, bed), wd, bd, frames, t, heads, qn=qnd, kn=knd,
                                  rope=rp, eps=1e-6)
    seq = ctx.linear_qkv_heads(ctx.layernorm(xd, gd, bed, eps=1e-6), wd, bd, frames, t, heads,
                               qn=qnd, kn=knd, rope=rp, eps=1e-6)
    proj = reference_ln_linear(x, g, be, w, b, 1e-6)
    for i, (norm, mine, theirs) in enumerate(zip((qn, kn, None), got, seq)):
        what = f"linear_ln_qkv_heads third {i}"
        assert_bit_exact(back(mine), back(theirs), what + " against layernorm then linear_qkv_heads")
        nw, nb = norm if norm is not None else (None, None)
        use_rope = rope_on and i < 2
        third = np.ascontiguousarray(proj[:, i * dim:(i + 1) * dim])
        want = O.qknorm_rope(third, nw, nb, sin if use_rope else None, cos if use_rope else None,
                             frames, t, heads, d, prefix if use_rope else 0, 1e-6)
        check(back(mine), want, what)


@pytest.mark.parametrize("name", ["qkv", "fc1"])
def test_linear_ln_full_size(ctx, name):
    """The trunk's LN1 -> q|k|v and LN2 -> fc1 + GELU at S=32 (43,968 rows):
    bit-exact against the library's unfused sequence, and within the f16
    gate of float32 torch on the reference's sequence (layernorm stored in
    f16, then the product)."""
    n, k = (3072, 1024) if name == "qkv" else (4096, 1024)
    m = 32 * 1374
    gen = torch.Generator(device="cpu").manual_seed(n + k + 1)
    x = torch.randn((m, k), generator=gen).half().to("cuda:0")
    g = (1 + 0.02 * torch.randn(k, generator=gen)).to("cuda:0")
    be = (0.02 * torch.randn(k, generator=gen)).to("cuda:0")
    w = (torch.randn((n, k), generator=gen) / k ** 0.5).half().to("cuda:0")
    b = (torch.randn(n, generator=gen) * 0.02).to("cuda:0")
    normed = torch.nn.functional.layer_norm(x.float(), (k,), g, be, eps=1e-6).half()
    ref = normed.float() @ w.float().t().contiguous() + b
    if name == "fc1":
        got = ctx.linear_ln_gelu(x, (g, be), w, b, eps=1e-6)
        seq = ctx.linear_gelu(ctx.layernorm(x, g, be, eps=1e-6), w, b)
        ref = torch.nn.functional.gelu(ref.half().float()).half()
    else:
        got = ctx.linear_ln(x, (g, be), w, b, eps=1e-6)
        seq = ctx.linear(ctx.layernorm(x, g, be, eps=1e-6), w, b)
        ref = ref.half()
    assert torch.equal(got.view(torch.int16), seq.view(torch.int16)), \
        f"full-size LN + {name}: {(got != seq).sum().item()} values differ from the unfused sequence"
    f16_close(back(got).astype(np.float32), back(ref).astype(np.float32), f"full-size LN + {name}")
