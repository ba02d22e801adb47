"""Linear layers (hs_linear, hs_linear_gelu, hs_linear_ls_residual) against
the oracle (linear.wesl restated) and, at the trunk's full shapes, against a
float32 torch product on the device.

Bars: f32 within 1e-5 * (1 + |e|) * 4 of the oracle (the oracle sums in k
order; the kernel's order differs); f16 within 2e-3 * max(1, |e|);
small-integer inputs bit-exact (every product and partial sum is exact).
"""
import numpy as np
import pytest
import torch

from headshot_amd import _lib
from headshot_amd.parity import assert_bit_exact, assert_close, f16_close, ulp_diff_f16
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


def operands(seed, m, n, k, dt, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * scale).astype(dt)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(dt)
    b = (rng.standard_normal(n) * 0.02).astype(np.float32)
    return x, w, b


@pytest.mark.parametrize("m,n,k", [(1, 128, 32), (37, 128, 64), (256, 256, 1024), (300, 384, 96),
                                   (513, 128, 32), (37, 48, 80), (5, 100, 40)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("with_bias", [True, False])
def test_linear_vs_oracle(ctx, m, n, k, dtype, with_bias):
    x, w, b = operands(m * 7 + n + k, m, n, k, NP[dtype])
    bias = b if with_bias else None
    got = back(ctx.linear(dev(x), dev(w), None if bias is None else dev(bias)))
    check(got, O.linear(x, w, bias), f"linear {(m, n, k)} {dtype}")


@pytest.mark.parametrize("m,n,k", [(300, 256, 128), (37, 128, 1024)])
def test_linear_f16_integers_exact(ctx, m, n, k):
    rng = np.random.default_rng(m + n + k)
    x = rng.integers(-3, 4, (m, k)).astype(np.float16)
    w = rng.integers(-3, 4, (n, k)).astype(np.float16)
    got = back(ctx.linear(dev(x), dev(w)))
    assert_bit_exact(got, O.linear(x, w), "integer linear f16")


@pytest.mark.parametrize("m,n,k", [(300, 256, 128), (37, 48, 80)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_linear_gelu_vs_reference_sequence(ctx, m, n, k, dtype):
    x, w, b = operands(m + 3 * n + k, m, n, k, NP[dtype], scale=2.0)
    got = back(ctx.linear_gelu(dev(x), dev(w), dev(b)))
    check(got, O.linear_gelu(x, w, b), f"linear_gelu {(m, n, k)} {dtype}")


@pytest.mark.parametrize("m,n,k", [(300, 256, 128), (37, 48, 80)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("in_place", [False, True])
def test_linear_ls_residual_vs_reference_sequence(ctx, m, n, k, dtype, in_place):
    x, w, b = operands(m + 5 * n + k, m, n, k, NP[dtype])
    rng = np.random.default_rng(9)
    res = rng.standard_normal((m, n)).astype(NP[dtype])
    g = rng.standard_normal(n).astype(np.float32)
    r = dev(res)
    got = ctx.linear_ls_residual(dev(x), dev(w), dev(g), r, dev(b), out=r if in_place else None)
    check(back(got), O.linear_ls_residual(x, w, g, res, b), f"linear_ls_residual {(m, n, k)}")


# the trunk's GEMMs at S=32 (43968 rows), f16
FULL = {"qkv": (3072, 1024), "proj": (1024, 1024), "fc1": (4096, 1024), "fc2": (1024, 4096)}


@pytest.mark.parametrize("name", list(FULL))
def test_linear_full_size(ctx, name):
    n, k = FULL[name]
    m = 32 * 1374
    g = torch.Generator(device="cpu").manual_seed(n + k)
    x = torch.randn((m, k), generator=g).half().to("cuda:0")
    w = (torch.randn((n, k), generator=g) / k ** 0.5).half().to("cuda:0")
    b = (torch.randn(n, generator=g) * 0.02).to("cuda:0")
    ref = (x.float() @ w.float().t().contiguous()) + b
    if name == "fc1":
        got = ctx.linear_gelu(x, w, b)
        ref = torch.nn.functional.gelu(ref.half().float())  # reference sequence: stored, then GELU
    elif name in ("proj", "fc2"):
        res = torch.randn((m, n), generator=g).half().to("cuda:0")
        # LayerScale magnitudes (the trunk's are ~1e-5 .. 0.1): with |gamma|
        # near 1, a one-ulp difference in the stored linear output (the sum
        # order differs from torch's) would already reach the f16 gate.
        gam = (torch.randn(n, generator=g) * 0.1).to("cuda:0")
        got = ctx.linear_ls_residual(x, w, gam, res, b)
        ref = res.float() + gam * ref.half().float()
    else:
        got = ctx.linear(x, w, b)
    f16_close(back(got).astype(np.float32), back(ref), f"full-size {name}")
    rows = np.array([0, 1, 255, 256, 20000, m - 1])
    xs, ws = back(x), back(w)
    if name == "qkv":
        check(back(got)[rows], O.linear(xs, ws, back(b), rows), f"full-size {name} vs oracle")


@pytest.mark.parametrize("case", range(16))
def test_linear_epilogues_random_sweep(ctx, case):
    """Seeded random shapes on the matrix-core path (n a multiple of 256, k
    of 64) and off it, each epilogue against float32 torch of the
    reference's sequence: bias; bias then GELU of the stored (f16) value;
    bias then LayerScale + residual of the stored value. m from 1 to 3000
    covers every remainder of the 256-row tile."""
    rng = np.random.default_rng(500 + case)
    m = int(rng.integers(1, 3001))
    fast = case % 4 != 3
    n = int(rng.choice([256, 512, 768, 1024])) if fast else int(rng.integers(1, 300))
    k = int(rng.choice([64, 128, 192, 512, 1024])) if fast else int(rng.integers(1, 200))
    g = torch.Generator(device="cpu").manual_seed(500 + case)
    x = torch.randn((m, k), generator=g).half().to("cuda:0")
    w = (torch.randn((n, k), generator=g) / k ** 0.5).half().to("cuda:0")
    b = (torch.randn(n, generator=g) * 0.02).to("cuda:0")
    stored = ((x.float() @ w.float().t().contiguous()) + b).half().float()
    what = f"sweep case {case}: m={m} n={n} k={k}"
    f16_close(back(ctx.linear(x, w, b)).astype(np.float32), back(stored), what + " bias")
    f16_close(back(ctx.linear_gelu(x, w, b)).astype(np.float32),
              back(torch.nn.functional.gelu(stored)), what + " gelu")
    res = torch.randn((m, n), generator=g).half().to("cuda:0")
    gam = (torch.randn(n, generator=g) * 0.1).to("cuda:0")
    f16_close(back(ctx.linear_ls_residual(x, w, gam, res, b)).astype(np.float32),
              back(res.float() + gam * stored), what + " layerscale")


# f32 shapes on the f32 matrix-core kernel (n % 128 == 0, k % 32 == 0): 64
# x 128 tiles below 512 tiles of 128 x 128, 128 x 128 tiles from there.
# Narrow: a last row tile of 56 rows; of 19 rows; one k stage (k = 32) with
# a last row tile of one row; an odd stage count; a single column tile (n =
# 128) with 2 stages (the smaller shapes of the tests above with n % 128 ==
# 0 and k % 32 == 0 run on it too). 128 x 128: a last row tile of 57 rows
# and 3 stages; one stage and a last row tile of one row; an odd stage
# count and n = 1024. Long k on few tiles: 16 x 8 tiles at k = 2048; 5 x 2
# tiles at k = 2080 (65 stages).
F32_MATRIX = [(3000, 2048, 64), (6163, 1024, 96), (6145, 1024, 32), (24577, 256, 160),
              (2815, 128, 64), (12345, 768, 96), (8193, 1024, 32), (8300, 1024, 160),
              (1000, 1024, 2048), (301, 256, 2080)]


@pytest.mark.parametrize("m,n,k", F32_MATRIX)
def test_linear_f32_matrix_core_epilogues(ctx, m, n, k):
    x, w, b = operands(m + 11 * n + k, m, n, k, np.float32, scale=2.0)
    rng = np.random.default_rng(m + k)
    res = rng.standard_normal((m, n)).astype(np.float32)
    g = (rng.standard_normal(n) * 0.5).astype(np.float32)
    y = O.linear(x, w, b)
    xd, wd, bd = dev(x), dev(w), dev(b)
    check(back(ctx.linear(xd, wd, bd)), y, f"f32 linear {(m, n, k)}")
    check(back(ctx.linear(xd, wd)), O.linear(x, w), f"f32 linear without bias {(m, n, k)}")
    check(back(ctx.linear_gelu(xd, wd, bd)), O.gelu(y), f"f32 linear_gelu {(m, n, k)}")
    want = O.residual_ls(res, y, g)
    check(back(ctx.linear_ls_residual(xd, wd, dev(g), dev(res), bd)), want,
          f"f32 linear_ls_residual {(m, n, k)}")
    r = dev(res)
    ctx.linear_ls_residual(xd, wd, dev(g), r, bd, out=r)
    check(back(r), want, f"f32 linear_ls_residual in place {(m, n, k)}")


@pytest.mark.parametrize("case", range(12))
def test_linear_f32_random_sweep(ctx, case):
    """Seeded random f32 shapes on the f32 matrix-core kernel, each epilogue
    against a float64 product on the device; m from 1 to 3000 covers every
    remainder of the 128-row tile."""
    rng = np.random.default_rng(900 + case)
    m = int(rng.integers(1, 3001))
    n = int(rng.choice([128, 256, 384, 640, 1024]))
    k = int(rng.choice([32, 64, 96, 160, 512, 1024]))
    g = torch.Generator(device="cpu").manual_seed(900 + case)
    x = torch.randn((m, k), generator=g).to("cuda:0")
    w = (torch.randn((n, k), generator=g) / k ** 0.5).to("cuda:0")
    b = (torch.randn(n, generator=g) * 0.02).to("cuda:0")
    res = torch.randn((m, n), generator=g).to("cuda:0")
    gam = torch.randn(n, generator=g).to("cuda:0")
    y = x.double() @ w.double().t().contiguous() + b.double()
    what = f"f32 sweep case {case}: m={m} n={n} k={k}"
    check(back(ctx.linear(x, w, b)), back(y), what + " bias")
    check(back(ctx.linear_gelu(x, w, b)), back(torch.nn.functional.gelu(y)), what + " gelu")
    check(back(ctx.linear_ls_residual(x, w, gam, res, b)), back(res.double() + gam.double() * y),
          what + " layerscale")


def test_linear_f32_integers_exact(ctx):
    """Small-integer f32 operands on the f32 matrix-core kernel: every
    product and partial sum is an integer below 2^24, so any summation order
    gives the oracle's value exactly."""
    m, n, k = 6000, 1024, 256
    rng = np.random.default_rng(77)
    x = rng.integers(-3, 4, (m, k)).astype(np.float32)
    w = rng.integers(-3, 4, (n, k)).astype(np.float32)
    assert_bit_exact(back(ctx.linear(dev(x), dev(w))), O.linear(x, w), "integer linear f32")


@pytest.mark.parametrize("name", ["qkv", "fc1", "fc2"])
def test_linear_f32_full_size(ctx, name):
    """The trunk's f32 products at S=32 (43968 rows) on the f32 matrix-core
    kernel against a float64 product on the device, and sampled rows
    against the oracle."""
    n, k = FULL[name]
    n = n // 3 if name == "qkv" else n  # the f32 q|k|v runs one product per third
    m = 32 * 1374
    g = torch.Generator(device="cpu").manual_seed(n + k + 1)
    x = torch.randn((m, k), generator=g).to("cuda:0")
    w = (torch.randn((n, k), generator=g) / k ** 0.5).to("cuda:0")
    b = (torch.randn(n, generator=g) * 0.02).to("cuda:0")
    ref = x.double() @ w.double().t().contiguous() + b.double()
    if name == "fc1":
        got = ctx.linear_gelu(x, w, b)
        ref = torch.nn.functional.gelu(ref)
    elif name == "fc2":
        res = torch.randn((m, n), generator=g).to("cuda:0")
        gam = (torch.randn(n, generator=g) * 0.1).to("cuda:0")
        got = ctx.linear_ls_residual(x, w, gam, res, b)
        ref = res.double() + gam.double() * ref
    else:
        got = ctx.linear(x, w, b)
    torch.cuda.synchronize()
    err = ((got.double() - ref).abs() / (ref.abs() + 1)).max().item()
    assert err < 4e-5, f"f32 full-size {name}: max relative error {err}"
    rows = np.array([0, 1, 255, 256, 20000, m - 1])
    xs, ws, bs = back(x), back(w), back(b)
    y = O.linear(xs, ws, bs, rows)
    if name == "fc1":
        want = O.gelu(y)
    elif name == "fc2":
        want = O.residual_ls(back(res)[rows], y, back(gam))
    else:
        want = y
    check(back(got)[rows], want, f"f32 full-size {name} vs oracle")
    del ref


def test_linear_contract(ctx):
    x = torch.zeros((4, 32), dtype=torch.float16, device="cuda:0")
    with pytest.raises(AssertionError):
        ctx.linear(x, torch.zeros((128, 16), dtype=torch.float16, device="cuda:0"))
    with pytest.raises(AssertionError):
        ctx.linear(x, torch.zeros((128, 32), dtype=torch.float32, device="cuda:0"))
    w = torch.zeros((128, 32), dtype=torch.float16, device="cuda:0")
    with pytest.raises(_lib.HsContractError):
        _lib.check(ctx.lib.hs_linear_ls_residual(torch.cuda.current_stream().cuda_stream, _lib.HS_F16,
                                                 x.data_ptr(), w.data_ptr(), None, None,
                                                 x.data_ptr(), x.data_ptr(), 4, 128, 32),
                   "linear_ls_residual")


# ---------------------------------------------------- fused q|k|v projection

def qkv_sequence(ctx, x, w, b, s, t, h, qn, kn, rope, eps):
    """The unfused sequence: linear per third, then qknorm_rope (q, k) or the
    plain head split (v)."""
    hd = h * 64
    outs = []
    for i, norm in enumerate((qn, kn, None)):
        proj = ctx.linear(x, w[i * hd:(i + 1) * hd], None if b is None else b[i * hd:(i + 1) * hd])
        outs.append(ctx.qknorm_rope(proj, s, t, h, 64, norm=norm, rope=rope if i < 2 else None,
                                    eps=eps))
    return outs


def qkv_case(seed, s, t, h, k, norm, prefix):
    from headshot_amd import rope as rp
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((s * t, k), generator=g).half().to("cuda:0")
    w = (torch.randn((3 * h * 64, k), generator=g) / k ** 0.5).half().to("cuda:0")
    b = (torch.randn(3 * h * 64, generator=g) * 0.02).to("cuda:0")
    nrm = lambda: ((1 + 0.1 * torch.randn(64, generator=g)).to("cuda:0"),  # noqa: E731
                   (0.1 * torch.randn(64, generator=g)).to("cuda:0"))
    qn, kn = (nrm(), nrm()) if norm else (None, None)
    rope = None
    if prefix is not None:
        sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), 1, t - prefix))
        rope = (sin, cos, prefix)
    return x, w, b, qn, kn, rope


# (s, t, h, k, QK-norm, RoPE prefix or None); t = 3 and 1 are shorter than
# the epilogue's 8-row step (its token counter wraps within a step)
QKV_CASES = [(2, 41, 16, 256, True, 5), (1, 300, 16, 1024, True, None), (3, 20, 8, 64, False, 17),
             (50, 3, 8, 128, True, 1), (1, 1, 8, 64, True, None), (5, 77, 32, 192, False, None),
             (7, 30, 4, 128, True, 3), (4, 9, 12, 64, True, None)]


@pytest.mark.parametrize("s,t,h,k,norm,prefix", QKV_CASES)
def test_linear_qkv_heads_is_the_sequence(ctx, s, t, h, k, norm, prefix):
    """hs_linear_qkv_heads against hs_linear + hs_qknorm_rope per third:
    bit-exact where hs_qknorm_rope runs its row kernel (8, 16 or 32 heads:
    the same head-vector code), within one f16 ulp where it runs its generic
    kernel (other head counts: another reduction order); q against the
    oracle's reference sequence (linear.wesl, split_heads, layernorm,
    rope_apply) within the f16 gate."""
    x, w, b, qn, kn, rope = qkv_case(s * 1000 + t, s, t, h, k, norm, prefix)
    got = ctx.linear_qkv_heads(x, w, b, s, t, h, qn=qn, kn=kn, rope=rope, eps=1e-5)
    want = qkv_sequence(ctx, x, w, b, s, t, h, qn, kn, rope, 1e-5)
    for name, a, e in zip("qkv", got, want):
        assert tuple(a.shape) == (s, h, t, 64)
        what = f"{name} {(s, t, h, k, norm, prefix)}"
        if h in (8, 16, 32) or name == "v":
            assert_bit_exact(back(a), back(e), what)
        else:
            assert ulp_diff_f16(back(a), back(e)).max() <= 1, what
    qproj = O.linear(back(x), back(w[:h * 64]), back(b[:h * 64]))
    tabs = (None, None, 0) if rope is None else (back(rope[0]), back(rope[1]), prefix)
    qo = O.qknorm_rope(qproj, *(tuple(back(a) for a in qn) if qn else (None, None)),
                       tabs[0], tabs[1], s, t, h, 64, tabs[2], 1e-5)
    f16_close(back(got[0]).astype(np.float32), qo.astype(np.float32), "q vs oracle")


def test_linear_qkv_heads_full_size_frame(ctx):
    """The S=32 frame block's projection (43,968 tokens, 37x37 grid, prefix
    5, 16 heads, dim 1024) bit-exact against the unfused sequence."""
    from headshot_amd import rope as rp
    s, t, h, k = 32, 1374, 16, 1024
    g = torch.Generator(device="cpu").manual_seed(77)
    x = torch.randn((s * t, k), generator=g).half().to("cuda:0")
    w = (torch.randn((3 * h * 64, k), generator=g) / k ** 0.5).half().to("cuda:0")
    b = (torch.randn(3 * h * 64, generator=g) * 0.02).to("cuda:0")
    qn = (torch.ones(64, device="cuda:0") * 1.1, torch.full((64,), 0.05, device="cuda:0"))
    kn = (torch.ones(64, device="cuda:0") * 0.9, torch.full((64,), -0.05, device="cuda:0"))
    sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), 37, 37))
    got = ctx.linear_qkv_heads(x, w, b, s, t, h, qn=qn, kn=kn, rope=(sin, cos, 5), eps=1e-6)
    want = qkv_sequence(ctx, x, w, b, s, t, h, qn, kn, (sin, cos, 5), 1e-6)
    for name, a, e in zip("qkv", got, want):
        assert torch.equal(a, e), f"full-size {name}"


@pytest.mark.parametrize("s,t,h,k,norm,prefix", QKV_CASES)
def test_linear_qkv_heads_f32_is_the_sequence(ctx, s, t, h, k, norm, prefix):
    """The f32 q|k|v epilogue (f32 matrix-core kernel) against hs_linear +
    hs_qknorm_rope per third: bit-exact where hs_qknorm_rope runs its row
    kernel (8, 16 or 32 heads: the same head-vector code in the same lane
    layout), within 1e-6 relative where it runs its generic kernel (another
    reduction order); q against the oracle's reference sequence within the
    f32 bar."""
    x, w, b, qn, kn, rope = qkv_case(s * 1000 + t + 1, s, t, h, k, norm, prefix)
    x, w = x.float(), w.float()
    got = ctx.linear_qkv_heads(x, w, b, s, t, h, qn=qn, kn=kn, rope=rope, eps=1e-5)
    want = qkv_sequence(ctx, x, w, b, s, t, h, qn, kn, rope, 1e-5)
    for name, a, e in zip("qkv", got, want):
        assert tuple(a.shape) == (s, h, t, 64) and a.dtype == torch.float32
        what = f"f32 {name} {(s, t, h, k, norm, prefix)}"
        if h in (8, 16, 32) or name == "v":
            assert_bit_exact(back(a), back(e), what)
        else:
            assert_close(back(a), back(e), 1e-6, what)
    qproj = O.linear(back(x), back(w[:h * 64]), back(b[:h * 64]))
    tabs = (None, None, 0) if rope is None else (back(rope[0]), back(rope[1]), prefix)
    qo = O.qknorm_rope(qproj, *(tuple(back(a) for a in qn) if qn else (None, None)),
                       tabs[0], tabs[1], s, t, h, 64, tabs[2], 1e-5)
    check(back(got[0]), qo, "f32 q vs oracle")


def test_linear_qkv_heads_f32_block_shape(ctx):
    """The S=2 f32 frame block's projection (2 x 1374 tokens, 37x37 grid,
    prefix 5, 16 heads, dim 1024: 64 x 128 tiles) and the same at 8 frames
    (128 x 128 tiles), bit-exact against the unfused sequence."""
    from headshot_amd import rope as rp
    sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), 37, 37))
    for s in (2, 8):
        x, w, b, qn, kn, _ = qkv_case(77 + s, s, 1374, 16, 1024, True, None)
        x, w = x.float(), w.float()
        got = ctx.linear_qkv_heads(x, w, b, s, 1374, 16, qn=qn, kn=kn, rope=(sin, cos, 5), eps=1e-6)
        want = qkv_sequence(ctx, x, w, b, s, 1374, 16, qn, kn, (sin, cos, 5), 1e-6)
        for name, a, e in zip("qkv", got, want):
            assert_bit_exact(back(a), back(e), f"f32 {name} at S={s}")


def test_linear_qkv_heads_fallback_f32(ctx):
    """f32 shapes the fused kernel does not cover (3 * H * 64 not a multiple
    of 128: H odd) run the unfused sequence; the C entry point refuses them."""
    x, w, b, qn, kn, rope = qkv_case(3, 2, 41, 3, 64, True, 5)
    x, w = x.float(), w.float()
    got = ctx.linear_qkv_heads(x, w, b, 2, 41, 3, qn=qn, kn=kn, rope=rope)
    want = qkv_sequence(ctx, x, w, b, 2, 41, 3, qn, kn, rope, 1e-5)
    for a, e in zip(got, want):
        assert torch.equal(a, e)
    with pytest.raises(_lib.HsError):
        _lib.check(ctx.lib.hs_linear_qkv_heads(
            torch.cuda.current_stream().cuda_stream, _lib.HS_F32, x.data_ptr(), w.data_ptr(),
            None, None, None, None, None, None, None, got[0].data_ptr(), got[1].data_ptr(),
            got[2].data_ptr(), 2, 41, 3, 64, 64, 0, 1e-5), "linear_qkv_heads")
