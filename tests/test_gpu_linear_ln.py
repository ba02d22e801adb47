"""The LayerNorm folded into the linear layer after it (hs_layernorm_stats,
hs_fold_layernorm, hs_linear_ln, hs_linear_ln_gelu, hs_linear_ln_qkv_heads)
against the reference's dispatch sequence in the oracle: layernorm (its
output rounded to the storage type), then linear with bias, then gelu or
split_heads + QK-norm + RoPE (model/block.rs:128-146, 153-176).

Bars: the statistics bit-exact to what hs_layernorm normalises with; the
folded weight bit-exact to dt(w * ln_w); f32 products within 1e-5 * (1 +
|e|) * 4 of the oracle (the summation order differs from its k order). f16
products (folded_close): the folded product rounds once on the folded
weight where the reference rounds the normalised row, an equally accurate
but different rounding pattern, so against the reference's sequence no
value may lie beyond twice the f16 gate 2e-3 * max(1, |e|) and at most
0.05% beyond the gate, and against the unrounded float64 result the folded
product may be no farther than the reference's own sequence (within 25%).
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


def folded_close(got, want, exact, what):
    """The bar for a folded product (f16): it rounds once on the folded
    weight where the reference rounds the normalised row, so the two are
    equally accurate but not the same rounding pattern. Against the
    reference's sequence: no value beyond twice the f16 gate and at most
    0.05% beyond it; against the unrounded float64 result: no farther than
    the reference's sequence itself (within 25%)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    exact = np.asarray(exact, np.float64)
    scaled = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    assert scaled.max() <= 4e-3, f"{what}: {scaled.max():.3g} beyond twice the f16 gate"
    assert (scaled > 2e-3).mean() <= 5e-4, f"{what}: {(scaled > 2e-3).mean():.3%} beyond the gate"
    err_fold = (np.abs(got - exact) / np.maximum(1.0, np.abs(exact))).max()
    err_ref = (np.abs(want - exact) / np.maximum(1.0, np.abs(exact))).max()
    assert err_fold <= 1.25 * err_ref + 1e-6, f"{what}: folded {err_fold:.3g} vs reference {err_ref:.3g}"


def exact_ln_linear(x, g, be, w, b, eps):
    """layernorm then linear in float64, without storage roundings."""
    x64 = x.astype(np.float64)
    mu, var = x64.mean(1, keepdims=True), x64.var(1, keepdims=True)
    return ((x64 - mu) / np.sqrt(var + eps) * g + be) @ w.astype(np.float64).T + b


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


@pytest.mark.parametrize("rows,dim", [(1, 1024), (19, 1024), (257, 1024), (300, 300), (64, 2048)])
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
    # the same statistics hs_layernorm normalises with: unit weight, zero bias
    ones = torch.ones(dim, device="cuda:0")
    zeros = torch.zeros(dim, device="cuda:0")
    normed = back(ctx.layernorm(dev(x), ones, zeros, eps=1e-6))
    mine = ((x.astype(np.float32) - st[:, :1]) * st[:, 1:]).astype(NP[dtype])
    assert_bit_exact(normed, mine, f"stats of hs_layernorm {rows}x{dim}")


@pytest.mark.parametrize("n,k", [(256, 1024), (48, 80), (3072, 1024)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fold_layernorm(ctx, n, k, dtype, with_bias):
    _, g, be, w, b = ln_operands(n + k, 1, n, k, NP[dtype])
    bias = b if with_bias else None
    f = ctx.fold_layernorm(dev(w), None if bias is None else dev(bias), dev(g), dev(be))
    w_fold = back(f.w_fold)
    assert_bit_exact(w_fold, (w.astype(np.float32) * g).astype(NP[dtype]), "w_fold")
    colsum = w_fold.astype(np.float64).sum(axis=1)
    shift = w.astype(np.float64) @ be.astype(np.float64) + (0.0 if bias is None else bias)
    assert_close(back(f.colsum), colsum.astype(np.float32), 1e-5, "colsum")
    assert_close(back(f.shift), shift.astype(np.float32), 1e-5, "shift")


def reference_ln_linear(x, g, be, w, b, eps):
    """layernorm (output stored in x's dtype) then linear: the oracle's
    restatement of the reference's two dispatches."""
    return O.linear(O.layernorm(x, g, be, eps), w, b)


@pytest.mark.parametrize("m,n,k", [(1, 256, 1024), (19, 256, 1024), (257, 512, 1024),
                                   (300, 256, 64), (37, 48, 80), (1374, 1024, 1024)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("mean", [0.0, 4.0])
def test_linear_ln_vs_reference_sequence(ctx, m, n, k, dtype, mean):
    """mean 4 puts the rows' mean well above their spread: the folded form
    subtracts mean * colsum from the raw product, so its cancellation shows
    here first."""
    x, g, be, w, b = ln_operands(m * 3 + n + k, m, n, k, NP[dtype], mean)
    f = ctx.fold_layernorm(dev(w), dev(b), dev(g), dev(be))
    got = back(ctx.linear_ln(dev(x), f, eps=1e-6))
    want = reference_ln_linear(x, g, be, w, b, 1e-6)
    what = f"linear_ln {(m, n, k)} {dtype} mean {mean}"
    if dtype == torch.float32:
        check(got, want, what)
    else:
        folded_close(got, want, exact_ln_linear(x, g, be, w, b, 1e-6), what)


@pytest.mark.parametrize("m,n,k", [(300, 256, 1024), (37, 48, 80), (1374, 4096, 1024)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_linear_ln_gelu_vs_reference_sequence(ctx, m, n, k, dtype):
    x, g, be, w, b = ln_operands(m + 7 * n + k, m, n, k, NP[dtype])
    f = ctx.fold_layernorm(dev(w), dev(b), dev(g), dev(be))
    got = back(ctx.linear_ln_gelu(dev(x), f, eps=1e-6))
    want = O.gelu(reference_ln_linear(x, g, be, w, b, 1e-6))
    what = f"linear_ln_gelu {(m, n, k)} {dtype}"
    if dtype == torch.float32:
        check(got, want, what)
    else:
        ex = exact_ln_linear(x, g, be, w, b, 1e-6)
        folded_close(got, want, ex * 0.5 * (1 + np.vectorize(__import__("math").erf)(ex / 2 ** 0.5)),
                     what)


@pytest.mark.parametrize("frames,grid,heads,rope_on", [(2, (37, 37), 16, True),
                                                       (1, (8, 8), 16, False),
                                                       (3, (4, 6), 8, True)])
def test_linear_ln_qkv_heads_vs_reference_sequence(ctx, frames, grid, heads, rope_on):
    prefix = 5
    t = grid[0] * grid[1] + prefix
    d, dim = 64, heads * 64
    m = frames * t
    x, g, be, w, b = ln_operands(frames * 31 + heads, m, 3 * dim, dim, np.float16)
    rng = np.random.default_rng(5)
    qn = ((1 + 0.02 * rng.standard_normal(d)).astype(np.float32),
          (0.02 * rng.standard_normal(d)).astype(np.float32))
    kn = ((1 + 0.02 * rng.standard_normal(d)).astype(np.float32),
          (0.02 * rng.standard_normal(d)).astype(np.float32))
    sin, cos = rope.tables(rope.periods(), *grid)
    rp = (dev(sin), dev(cos), prefix) if rope_on else None
    f = ctx.fold_layernorm(dev(w), dev(b), dev(g), dev(be))
    q, k, v = ctx.linear_ln_qkv_heads(dev(x), f, frames, t, heads, qn=tuple(map(dev, qn)),
                                      kn=tuple(map(dev, kn)), rope=rp, eps=1e-6)
    proj = reference_ln_linear(x, g, be, w, b, 1e-6)
    exact = exact_ln_linear(x, g, be, w, b, 1e-6)
    for i, (got, norm) in enumerate(((q, qn), (k, kn), (v, None))):
        nw, nb = norm if norm is not None else (None, None)
        use_rope = rope_on and i < 2

        def heads_of(p, dt):
            third = np.ascontiguousarray(p[:, i * dim:(i + 1) * dim]).astype(dt)
            return O.qknorm_rope(third, nw, nb, sin if use_rope else None,
                                 cos if use_rope else None, frames, t, heads, d,
                                 prefix if use_rope else 0, 1e-6)

        # QK-norm divides each head vector by its spread, which magnifies the
        # difference in rounding points; the unrounded reference is the
        # float64 projection normalised and rotated in f32 arithmetic
        folded_close(back(got), heads_of(proj, np.float16), heads_of(exact, np.float32),
                     f"linear_ln_qkv_heads third {i}")


@pytest.mark.parametrize("name", ["qkv", "fc1"])
def test_linear_ln_full_size(ctx, name):
    """The trunk's LN -> q|k|v and LN -> fc1 + GELU at S=32 (43,968 rows),
    against float32 torch of the reference sequence (layernorm stored in f16,
    then the product)."""
    n, k = (3072, 1024) if name == "qkv" else (4096, 1024)
    m = 32 * 1374
    gen = torch.Generator(device="cpu").manual_seed(n + k + 1)
    x = torch.randn((m, k), generator=gen).half().to("cuda:0")
    g = (1 + 0.02 * torch.randn(k, generator=gen)).to("cuda:0")
    be = (0.02 * torch.randn(k, generator=gen)).to("cuda:0")
    w = (torch.randn((n, k), generator=gen) / k ** 0.5).half().to("cuda:0")
    b = (torch.randn(n, generator=gen) * 0.02).to("cuda:0")
    f = ctx.fold_layernorm(w, b, g, be)
    normed = torch.nn.functional.layer_norm(x.float(), (k,), g, be, eps=1e-6).half()
    ref = normed.float() @ w.float().t().contiguous() + b
    x64 = x.double()
    ex = torch.nn.functional.layer_norm(x64, (k,), g.double(), be.double(), eps=1e-6)
    ex = ex @ w.double().t().contiguous() + b.double()
    if name == "fc1":
        got = ctx.linear_ln_gelu(x, f, eps=1e-6)
        ref = torch.nn.functional.gelu(ref.half().float()).half()
        ex = torch.nn.functional.gelu(ex)
    else:
        got = ctx.linear_ln(x, f, eps=1e-6)
        ref = ref.half()
    folded_close(back(got), back(ref), back(ex), f"full-size LN + {name}")
