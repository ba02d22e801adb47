"""Attention (hs_attention, hs_attention_merged) and the head merge
(hs_attn_merge) against the oracle on the reference's own test shapes, at
tile edges, and at full size against a float32 torch reference on the device.

Bars:
- f32: within 1e-5 (abs + rel) of the oracle, and 1e-4 absolute of the
  float64 naive softmax as tests/kernels.rs:232-235.
- f16: within 2e-3*max(1,|e|) of the oracle's f16 result (f32 math on the
  same f16 inputs, output rounded). The matrix-core path rounds the softmax
  weights to f16 for the P.V product; this bound covers that.
- f16 vs f32 on the same values: 5e-3 relative (tests/kernels.rs:377-401).
- attn_merge bit-exact; attention_merged bit-exact against
  attn_merge(attention(...)).
"""
import numpy as np
import pytest
import torch

from headshot_amd import _lib
from headshot_amd.parity import assert_bit_exact, assert_close, f16_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {torch.float32: np.float32, torch.float16: np.float16}
DTYPES = [torch.float32, torch.float16]


def host(a: np.ndarray, dtype) -> np.ndarray:
    return O.to_f16(a) if dtype == torch.float16 else np.ascontiguousarray(a, np.float32)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def back(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(got: np.ndarray, want: np.ndarray, what: str):
    assert got.dtype == want.dtype, f"{what}: dtype {got.dtype} vs {want.dtype}"
    if got.dtype == np.float32:
        assert_close(got, want, 1e-5, what)
    else:
        f16_close(got.astype(np.float32), want.astype(np.float32), what)


def naive64(q, k, v):
    """tests/kernels.rs:207-231 in float64."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    s = np.matmul(q, np.swapaxes(k, -1, -2)) / np.sqrt(q.shape[-1])
    p = np.exp(s - s.max(-1, keepdims=True))
    return np.matmul(p / p.sum(-1, keepdims=True), v)


def torch_attention32(q, k, v, q_rows=None):
    """float32 reference on the device; q_rows selects queries (dim 2)."""
    q32, k32, v32 = (x.float() for x in (q, k, v))
    if q_rows is not None:
        q32 = q32[:, :, q_rows].contiguous()
    scale = 1.0 / float(np.sqrt(q.shape[-1]))
    s = torch.matmul(q32, k32.transpose(-1, -2).contiguous()) * scale
    return torch.matmul(torch.softmax(s, dim=-1), v32)


def rand_qkv(seed, shape, dtype):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return [torch.randn(shape, generator=g).to(dtype).to("cuda:0") for _ in range(3)]


# ------------------------------------------------------ the reference's cases

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("t", [17, 64, 150])
def test_attention_reference_cases(ctx, dtype, t):
    """tests/kernels.rs:185-238: (s, h, d) = (2, 3, 64), q, k, v from Rng(5 + t)."""
    s, h, d = 2, 3, 64
    stream = O.rng_vec(5 + t, 3 * s * h * t * d).reshape(3, s, h, t, d)
    q, k, v = (host(stream[i], dtype) for i in range(3))
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), f"attention t={t} {dtype}")
    if dtype == torch.float32:
        assert np.abs(got - naive64(q, k, v)).max() < 1e-4


def test_attention_f16_matches_f32(ctx):
    """tests/kernels.rs:377-401: (1, 2, 33, 64), Rng(9), 5e-3."""
    s, h, t, d = 1, 2, 33, 64
    stream = O.rng_vec(9, 3 * s * h * t * d).reshape(3, s, h, t, d)
    f32 = back(ctx.attention(*(dev(stream[i]) for i in range(3))))
    f16 = back(ctx.attention(*(dev(O.to_f16(stream[i])) for i in range(3))))
    assert_close(f16.astype(np.float32), f32, 5e-3, "attention f16 vs f32")


# ------------------------------------------------------------- tile edges

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("t", [1, 2, 31, 63, 65, 127, 128, 129, 257])
@pytest.mark.parametrize("s,h", [(1, 1), (3, 5), (2, 13)])
def test_attention_edges(ctx, dtype, t, s, h):
    rng = np.random.default_rng(1000 * t + 10 * s + h)
    q, k, v = (host(rng.standard_normal((s, h, t, 64)), dtype) for _ in range(3))
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), f"attention t={t} s={s} h={h} {dtype}")


@pytest.mark.parametrize("scale", [0.25, 4.0])
def test_attention_f16_score_range(ctx, scale):
    """Flat (scale 0.25) and peaked (scale 4: scores of std 16) softmax."""
    rng = np.random.default_rng(77)
    s, h, t = 2, 4, 300
    q = O.to_f16(scale * rng.standard_normal((s, h, t, 64)))
    k = O.to_f16(rng.standard_normal((s, h, t, 64)))
    v = O.to_f16(rng.standard_normal((s, h, t, 64)))
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), f"attention score scale {scale}")


@pytest.mark.parametrize("case", ["ramp", "spike", "mixed"])
def test_attention_f16_reference_moves(ctx, case):
    """Scores that rise from tile to tile, so that later 64-key tiles take the
    max path (a tile's weights against the kept reference would overflow
    f16): "ramp" raises every tile's scores by ~18 (log2 units), "spike" puts
    one dominant key in the last tile, "mixed" gives half the queries of each
    wave a rising and half a falling ramp (the max path then runs for the
    whole wave while half its queries keep their reference)."""
    rng = np.random.default_rng(5)
    s, h, t = 1, 2, 300
    q = np.zeros((s, h, t, 64))
    k = 0.5 * rng.standard_normal((s, h, t, 64))
    v = rng.standard_normal((s, h, t, 64))
    q[..., 0] = 8.0  # score = k[..., 0] (q.k / 8)
    if case == "spike":
        k[..., 0] += 2.0 * rng.standard_normal((s, h, t))
        k[:, :, t - 3, 0] = 120.0
    else:
        k[..., 0] += 12.5 * (np.arange(t) // 64)  # 12.5 * log2(e) = 18 per tile
        if case == "mixed":
            q[:, :, 1::2, 0] = -8.0  # odd queries: scores fall tile to tile
    q, k, v = O.to_f16(q), O.to_f16(k), O.to_f16(v)
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), f"attention reference moves ({case})")


@pytest.mark.parametrize("v_scale", [1.0, 1000.0])
def test_attention_f16_row_sum_rounding_worst_case(ctx, v_scale):
    """The f16 matrix-core kernel sums each lane's weights in groups of four
    keys (the keys of one 32-key block that agree mod 8) by two levels of
    f16 additions, then in f32. Its worst case: one weight of 1 per group
    and three that f16 drops, one (just under half an f16 ulp of 1) at the
    first level beside the 1 and two (together just under it) at the
    second. Every group then loses ~1.97 * 2^-11 of its 1 + 1.97 * 2^-11,
    so l is low by ~9.6e-4 relative, and with V constant the output is high
    by as much (the numerator adds the same f16 weights in f32). Bound: at
    most 2^-10 from the two rounding levels plus 2^-11 from the output's
    f16 rounding, relative, which is also inside the f16 gate."""
    s_, h, t, d = 1, 2, 512, 64
    k = np.zeros((s_, h, t, d), np.float32)
    m32 = np.arange(t) % 32
    # scores q.k / 8 = a * 8 / 8 = a: weights exp(a) against the max 0
    a = np.where(m32 < 8, 0.0, np.where((m32 >= 16) & (m32 < 24), -7.6328125, -8.3359375))
    k[..., 0] = a
    q = np.zeros((s_, h, t, d), np.float32)
    q[..., 0] = 8.0
    v = np.full((s_, h, t, d), v_scale, np.float32)
    qh, kh, vh = (O.to_f16(x) for x in (q, k, v))
    w = np.exp2(np.float64(a) * np.log2(np.e))
    lost = w[(m32 >= 8)].reshape(-1)  # every non-dominant weight is dropped by the f16 sums
    assert np.all(w[(m32 >= 16) & (m32 < 24)] < 2.0 ** -11), "first-level weight below half an ulp"
    assert np.all(2 * w[(m32 >= 8) & (m32 < 16)] < 2.0 ** -11), "second-level pair below half an ulp"
    got = back(ctx.attention(dev(qh), dev(kh), dev(vh))).astype(np.float64)
    want = naive64(qh, kh, vh)
    rel = np.abs(got - want) / np.abs(want)
    # the construction reaches the bound's order: l low by ~lost / total
    assert rel.max() > 0.5 * lost.sum() / w.sum(), "the worst case did not show"
    assert rel.max() <= 2.0 ** -10 + 2.0 ** -11, f"row-sum rounding {rel.max():.3g} beyond its bound"
    f16_close(got.astype(np.float32), want.astype(np.float32), "row-sum worst case")


@pytest.mark.parametrize("case", range(24))
def test_attention_f16_random_sweep(ctx, case):
    """Seeded random shapes and score statistics against float32 torch: T
    from 1 to 3000 (partial tiles of every size), 1-4 sequences x 1-5
    heads, score scales from flat to peaked, and in half the cases a drift
    that raises or lowers the scores along the keys by a random amount per
    64-key tile, so that the max path runs at random tiles and not only at
    the first."""
    rng = np.random.default_rng(1000 + case)
    s, h = int(rng.integers(1, 5)), int(rng.integers(1, 6))
    t = int(rng.integers(1, 3001))
    scale = float(rng.choice([0.1, 0.5, 1.0, 2.0, 4.0]))
    q = scale * rng.standard_normal((s, h, t, 64))
    k = rng.standard_normal((s, h, t, 64))
    v = rng.standard_normal((s, h, t, 64))
    if case % 2:
        # every query leans on one direction u; key j moves along u by a
        # random walk over the tiles, so its scores move by ~2 * drift
        u = rng.standard_normal(64)
        u /= np.linalg.norm(u)
        q = q + 2.0 * u
        drift = rng.normal(0.0, 6.0, -(-t // 64)).cumsum()
        k = k + (4.0 * drift[np.arange(t) // 64])[None, None, :, None] * u
    q, k, v = (dev(O.to_f16(a)) for a in (q, k, v))
    got = back(ctx.attention(q, k, v)).astype(np.float32)
    ref = back(torch_attention32(q, k, v))
    f16_close(got, ref, f"attention sweep case {case}: s={s} h={h} t={t} scale={scale}")


@pytest.mark.parametrize("t", [257, 300, 511])
def test_attention_partial_tile_launch(ctx, t):
    """32 sequences x 16 heads with a partial last 256-query tile: the tile
    runs as its own launch with the waves past T idle (t = 257 leaves one
    live query in it), plain and merged outputs against float32 torch."""
    s, h = 32, 16
    q, k, v = rand_qkv(t, (s, h, t, 64), torch.float16)
    got = ctx.attention(q, k, v)
    f16_close(back(got).astype(np.float32), back(torch_attention32(q, k, v)),
              f"partial-tile launch t={t}")
    assert_bit_exact(back(ctx.attention_merged(q, k, v)), back(ctx.attn_merge(got)),
                     f"partial-tile launch merged t={t}")


# ------------------------------------------- f32 head_dim 64 (matrix cores)

@pytest.mark.parametrize("scale", [0.25, 4.0])
def test_attention_f32_score_range(ctx, scale):
    """Flat (scale 0.25) and peaked (scale 4: scores of std 16) softmax in
    f32, against the oracle and the float64 softmax."""
    rng = np.random.default_rng(78)
    s, h, t = 2, 4, 300
    q = (scale * rng.standard_normal((s, h, t, 64))).astype(np.float32)
    k, v = (rng.standard_normal((s, h, t, 64)).astype(np.float32) for _ in range(2))
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), f"f32 attention score scale {scale}")
    assert np.abs(got - naive64(q, k, v)).max() < 1e-4


@pytest.mark.parametrize("case", ["ramp", "falling", "spike"])
def test_attention_f32_running_max(ctx, case):
    """Scores that rise from one 64-key tile to the next by ~18 (log2
    units), so every tile rescales what came before; that fall, so the first
    tile's max holds; and one dominant key in the last tile."""
    rng = np.random.default_rng(6)
    s, h, t = 1, 2, 300
    q = np.zeros((s, h, t, 64))
    k = 0.5 * rng.standard_normal((s, h, t, 64))
    v = rng.standard_normal((s, h, t, 64))
    q[..., 0] = 8.0  # score = k[..., 0] (q.k / 8)
    if case == "spike":
        k[:, :, t - 3, 0] = 120.0
    else:
        k[..., 0] += (12.5 if case == "ramp" else -12.5) * (np.arange(t) // 64)
    q, k, v = (a.astype(np.float32) for a in (q, k, v))
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), f"f32 attention running max ({case})")
    assert np.abs(got - naive64(q, k, v)).max() < 1e-4


def test_attention_f32_unaligned_takes_generic(ctx):
    """Inputs 4 bytes off 16-byte alignment take the generic kernel: the
    same results within the f32 bar."""
    rng = np.random.default_rng(79)
    s, h, t = 1, 3, 100
    q, k, v = (rng.standard_normal((s, h, t, 64)).astype(np.float32) for _ in range(3))
    want = O.attention(q, k, v)
    bufs = [torch.zeros(a.size + 1, dtype=torch.float32, device="cuda:0") for a in (q, k, v)]
    views = []
    for b_, a in zip(bufs, (q, k, v)):
        b_[1:].copy_(torch.from_numpy(a.reshape(-1)))
        views.append(b_[1:].view(s, h, t, 64))
    assert views[0].data_ptr() % 16 != 0
    check(back(ctx.attention(*views)), want, "f32 attention, unaligned inputs")


@pytest.mark.parametrize("s,t", [(2, 1374), (1, 2748), (16, 782)])
def test_attention_f32_block_shapes(ctx, s, t):
    """The f32 block's frame and global attention at S=2 (2 x 1374 tokens)
    and the 21x37 frame (782 tokens), 16 heads: every query against a
    float64 softmax on the device, sampled queries against the oracle,
    and the merged output bit-exact against the merge of the plain one."""
    q, k, v = rand_qkv(s * 10000 + t, (s, 16, t, 64), torch.float32)
    got = ctx.attention(q, k, v)
    sc = torch.matmul(q.double(), k.double().transpose(-1, -2).contiguous()) / 8.0
    ref = torch.matmul(torch.softmax(sc, dim=-1), v.double())
    err = (got.double() - ref).abs().max().item()
    assert err < 1e-4, f"f32 attention ({s}, 16, {t}): max error {err} against float64"
    rows = np.array([0, 1, 31, 32, 127, 128, t - 1])
    qs, ks, vs = back(q), back(k), back(v)
    check(back(got)[:, :, rows], O.attention(qs, ks, vs, rows), f"f32 attention ({s}, 16, {t}) vs oracle")
    assert_bit_exact(back(ctx.attention_merged(q, k, v)), back(ctx.attn_merge(got)),
                     f"f32 attention merged ({s}, 16, {t})")
    del sc, ref


def test_attention_d128_f32(ctx):
    """The camera head's head_dim 128 (f32 only, engine/ops.rs:233-238)."""
    rng = np.random.default_rng(128)
    q, k, v = (rng.standard_normal((1, 2, 40, 128)).astype(np.float32) for _ in range(3))
    got = back(ctx.attention(dev(q), dev(k), dev(v)))
    check(got, O.attention(q, k, v), "attention d128")
    assert np.abs(got - naive64(q, k, v)).max() < 1e-4


def test_attention_unsupported_shapes(ctx):
    x16 = torch.zeros((1, 1, 8, 128), dtype=torch.float16, device="cuda:0")
    with pytest.raises(_lib.HsError) as e:
        ctx.attention(x16, x16, x16)
    assert e.value.status == _lib.HS_EUNSUPPORTED
    x32 = torch.zeros((1, 1, 8, 32), dtype=torch.float32, device="cuda:0")
    with pytest.raises(_lib.HsError):
        ctx.attention(x32, x32, x32)
    with pytest.raises(AssertionError):
        ctx.attention(x32, x32, torch.zeros((1, 1, 9, 32), device="cuda:0"))


# ------------------------------------------------------------------ merge

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("s,h,t,d", [(2, 4, 5, 8), (2, 16, 37, 64), (1, 3, 11, 6), (3, 2, 7, 128),
                                     (1, 8, 13, 64), (3, 16, 131, 64)])
def test_attn_merge_exact(ctx, dtype, s, h, t, d):
    """Covers the token-per-wave kernel at 64, 128 and 256 vectors per token
    (odd token counts leave a half-filled wave) and the flat kernel."""
    rng = np.random.default_rng(s * 1000 + t)
    x = host(rng.standard_normal((s, h, t, d)), dtype)
    got = back(ctx.attn_merge(dev(x)))
    want = np.ascontiguousarray(x.transpose(0, 2, 1, 3).reshape(s * t, h * d))
    assert_bit_exact(got, want, f"attn_merge {dtype} {(s, h, t, d)}")
    assert_bit_exact(got, O.attn_merge(x), "attn_merge vs oracle")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("s,h,t", [(2, 3, 150), (3, 5, 65)])
def test_attention_merged_is_merge_of_attention(ctx, dtype, s, h, t):
    q, k, v = rand_qkv(s + h + t, (s, h, t, 64), dtype)
    a = ctx.attn_merge(ctx.attention(q, k, v))
    m = ctx.attention_merged(q, k, v)
    assert_bit_exact(back(m), back(a), f"attention_merged {dtype}")


# -------------------------------------------------------------- full size

def test_attention_frame_blocks_full_size(ctx):
    """Frame attention of the S=32 aggregator: (32, 16, 1374, 64) f16, every
    output against float32 torch on the same f16 inputs; two sequences
    against the oracle; the merged variant bit-exact."""
    s, h, t = 32, 16, 1374
    q, k, v = rand_qkv(32, (s, h, t, 64), torch.float16)
    got = ctx.attention(q, k, v)
    ref = torch_attention32(q, k, v)
    f16_close(back(got).astype(np.float32), back(ref), "frame attention vs torch f32")
    qs, ks, vs = (back(x)[[0, 31]][:, [0, 15]] for x in (q, k, v))
    sub = np.ascontiguousarray(back(got)[[0, 31]][:, [0, 15]])
    check(sub, O.attention(np.ascontiguousarray(qs), np.ascontiguousarray(ks),
                           np.ascontiguousarray(vs)), "frame attention vs oracle")
    merged = ctx.attention_merged(q, k, v)
    assert_bit_exact(back(merged), back(ctx.attn_merge(got)), "frame attention merged")


def test_attention_global_blocks_sampled(ctx):
    """Global attention of the S=32 aggregator: one sequence of 32*1374 =
    43968 tokens, 16 heads. Sampled queries against float32 torch and the
    oracle; constant V rows reproduce that row everywhere."""
    s, h, t = 1, 16, 32 * 1374
    q, k, v = rand_qkv(43968, (s, h, t, 64), torch.float16)
    got = back(ctx.attention(q, k, v))
    rows = torch.from_numpy(np.random.default_rng(5).choice(t, 256, replace=False)).to("cuda:0")
    ref = back(torch_attention32(q, k, v, rows))
    r = rows.cpu().numpy()
    f16_close(got[:, :, r].astype(np.float32), ref, "global attention vs torch f32")
    idx = np.sort(r[:6]).astype(np.int32)
    want = O.attention(back(q), back(k), back(v), q_idx=idx)
    check(np.ascontiguousarray(got[:, :, idx]), want, "global attention vs oracle")
    vc = v[:, :, :1].expand(s, h, t, 64).contiguous()
    out = back(ctx.attention(q, k, vc)).astype(np.float32)
    f16_close(out, np.broadcast_to(back(vc).astype(np.float32), out.shape), "constant V")
