"""The reference's own kernel tests (crates/headshot-server/tests/kernels.rs)
with their inputs, shapes and tolerances, run on the HIP ops: the Rng of
tests/kernels.rs:7-23 (SplitMix64, bit for bit), each case against the
closed form or CPU routine that test uses.

- residual_add (:45-61): a + b over 1000 values, 1e-6 (here as
  residual_ls with gamma = 1, exact in f32);
- layernorm_matches_cpu (:100-126): 19 rows of 300, eps 1e-5, 1e-4
  against a float64 LayerNorm;
- gelu_matches_erf (:128-147): x = -8 .. 8 in steps of 0.2 against the
  float64 erf form, 1e-5, and gelu(0) = 0, gelu(+-10) = 10 / 0;
- rope_apply_matches_cpu (:149-182): (2, 3, 11, 64), prefix 5, 2 x 3 grid,
  each vector against rope::apply_cpu (the oracle's restatement), 1e-5;
- linear_matches_cpu (:63-98): (m, k, n) = (37, 53, 29) f32, with and
  without bias, 1e-4 against float64 sums;
- linear_f16_and_wmma_match_cpu (:313-375): (37, 96, 128) f16 with bias,
  1e-2, and n = 48 without bias, 2e-3, against float64 sums of the
  f16-rounded inputs stored as f16;
- split_heads_merge_roundtrip (:241-274): (2, 5, 4, 8), exact;
- the concat part of im2col_and_concat (:300-310): (3, 2) ++ (3, 3), exact;
- tiled_add_broadcasts (tests/dense_kernels.rs:50-63): (3, 40) + a table
  of 40 broadcast over rows, inputs from that file's rvec (:6-17), 1e-6
  (one f32 add per element, so exact).
"""
import math

import numpy as np
import pytest
import torch

from headshot_amd.parity import assert_bit_exact, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def back(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_residual_add(ctx):
    v = O.rng_vec(1, 2000)
    a, b = v[:1000], v[1000:]
    got = back(ctx.residual_ls(dev(a), dev(b), torch.ones(1000, device="cuda:0")))
    assert_close(got, a + b, 1e-6, "residual_add")
    assert_bit_exact(got, a + b, "residual_add (gamma 1 is exact)")


def test_layernorm_matches_cpu(ctx):
    rows, dim = 19, 300
    v = O.rng_vec(3, rows * dim + 2 * dim)
    x = v[: rows * dim].reshape(rows, dim)
    w, b = v[rows * dim: rows * dim + dim], v[rows * dim + dim:]
    got = back(ctx.layernorm(dev(x), dev(w), dev(b), eps=1e-5))
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=1, keepdims=True)
    want = (x64 - mu) / np.sqrt(var + 1e-5) * w + b
    assert np.abs(got - want).max() < 1e-4


def test_gelu_matches_erf(ctx):
    xs = np.array([i * 0.2 for i in range(-40, 41)], np.float32)
    got = back(ctx.gelu(dev(xs)))
    for x, g in zip(xs, got):
        exact = 0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0)))
        assert abs(float(g) - exact) < 1e-5, (x, g, exact)
    edges = back(ctx.gelu(dev(np.array([0.0, 10.0, -10.0], np.float32))))
    assert edges[0] == 0.0 and abs(edges[1] - 10.0) < 1e-6 and abs(edges[2]) < 1e-6


def test_rope_apply_matches_cpu(ctx):
    s, h, t, d, prefix = 2, 3, 11, 64, 5
    sin, cos = O.rope_tables(O.rope_periods(), 2, 3)
    x = O.rng_vec(4, s * h * t * d).reshape(s, h, t, d)
    g = dev(x)
    ctx.rope_apply(g, dev(sin), dev(cos), prefix)
    got = back(g)
    for si in range(s):
        for hi in range(h):
            for ti in range(t):
                if ti < prefix:
                    assert_bit_exact(got[si, hi, ti], x[si, hi, ti], "prefix untouched")
                else:
                    want = O.rope_apply_cpu(x[si, hi, ti], sin, cos, ti - prefix)
                    assert np.abs(got[si, hi, ti] - want).max() < 1e-5, (si, hi, ti)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_split_heads_merge_roundtrip(ctx, dtype):
    s, t, h, d = 2, 5, 4, 8
    x = O.rng_vec(6, s * t * h * d).reshape(s * t, h * d)
    if dtype == torch.float16:
        x = O.to_f16(x)
    q = ctx.split_heads(dev(x), s, t, h, d)
    assert_bit_exact(back(q), np.ascontiguousarray(x.reshape(s, t, h, d).transpose(0, 2, 1, 3)),
                     "split_heads")
    assert_bit_exact(back(ctx.attn_merge(q)), x, "attn_merge")


def test_concat_channels(ctx):
    v = O.rng_vec(7, 15)
    a, b = v[:6], v[6:]
    got = back(ctx.concat_channels(dev(a.reshape(3, 2)), dev(b.reshape(3, 3)))).ravel()
    want = np.array([a[0], a[1], b[0], b[1], b[2], a[2], a[3], b[3], b[4], b[5], a[4], a[5],
                     b[6], b[7], b[8]], np.float32)
    assert_bit_exact(got, want, "concat")


def test_linear_matches_cpu(ctx):
    m, k, n = 37, 53, 29  # deliberately not multiples of any tile
    v = O.rng_vec(2, m * k + n * k + n)
    x = v[: m * k].reshape(m, k)
    w = v[m * k: m * k + n * k].reshape(n, k)
    b = v[m * k + n * k:]
    want = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32) + b
    assert_close(back(ctx.linear(dev(x), dev(w), dev(b))), want, 1e-4, "linear")
    assert_close(back(ctx.linear(dev(x), dev(w), None)), want - b, 1e-4, "linear no bias")


def test_linear_f16_matches_cpu(ctx):
    m, k, n = 37, 96, 128
    v = O.rng_vec(8, m * k + n * k + n)
    x = O.to_f16(v[: m * k].reshape(m, k))
    w = O.to_f16(v[m * k: m * k + n * k].reshape(n, k))
    b = v[m * k + n * k:]
    acc = x.astype(np.float64) @ w.astype(np.float64).T
    want = (acc.astype(np.float32) + b).astype(np.float16).astype(np.float32)
    got = back(ctx.linear(dev(x), dev(w), dev(b))).astype(np.float32)
    assert_close(got, want, 1e-2, "linear f16")
    n2 = 48
    want2 = acc[:, :n2].astype(np.float32).astype(np.float16).astype(np.float32)
    got2 = back(ctx.linear(dev(x), dev(np.ascontiguousarray(w[:n2])), None)).astype(np.float32)
    assert_close(got2, want2, 2e-3, "linear f16 n=48")


def test_tiled_add_broadcasts(ctx):
    n, block = 3, 40
    x, t = O.rvec(2, n * block), O.rvec(3, block)
    got = back(ctx.tiled_add(dev(x.reshape(n, block)), dev(t))).reshape(-1)
    want = x + t[np.arange(n * block) % block]
    assert_close(got, want, 1e-6, "tiled_add")
    assert_bit_exact(got, want, "tiled_add (one f32 add)")
