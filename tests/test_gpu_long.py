"""The largest workload: S=200 frames flattened to one global sequence of
274,800 tokens, f16, no RoPE, through the attention,
linear-layer and cache-build kernels at its real shapes.

Bars as for the smaller sizes: f16 outputs within 2e-3 * max(1, |e|) of a
float32 torch restatement on the device (every output for the linear layers,
sampled queries for attention) and of the oracle on sampled rows; the cache
build and the register gather / scatter bit-exact at full size.
"""
import numpy as np
import pytest
import torch

from headshot_amd.parity import assert_bit_exact, f16_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROWS = 200 * 1374
H, D = 16, 64


def back(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def randn(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda:0") * scale).half()


def max_scaled_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    """max |got - ref| / max(1, |ref|), computed on the device in row chunks."""
    worst = 0.0
    for i in range(0, got.shape[0], 32768):
        g, r = got[i:i + 32768].float(), ref[i:i + 32768].float()
        worst = max(worst, ((g - r).abs() / r.abs().clamp(min=1.0)).max().item())
    return worst


def test_attention_s200(ctx):
    """Global attention over 274,800 tokens, 16 heads of 64, written
    token-major: 64 sampled queries against float32 torch, 2 against the
    oracle, and constant V rows reproduced at every query."""
    print(f"[s200 attention: t={ROWS}]", flush=True)
    q, k, v = (randn((1, H, ROWS, D), 300 + i) for i in range(3))
    got = ctx.attention_merged(q, k, v).view(ROWS, H, D)
    rows = np.sort(np.random.default_rng(3).choice(ROWS, 64, replace=False))
    ri = torch.from_numpy(rows).to("cuda:0")
    s = torch.matmul(q[0][:, ri].float(), k[0].float().transpose(-1, -2).contiguous()) / 8.0
    ref = torch.matmul(torch.softmax(s, dim=-1), v[0].float())          # (H, 64, D)
    f16_close(back(got[ri].permute(1, 0, 2)).astype(np.float32), back(ref),
              "s200 attention vs torch f32")
    idx = rows[[5, 40]].astype(np.int32)
    want = O.attention(back(q), back(k), back(v), q_idx=idx)            # (1, H, 2, D)
    f16_close(back(got[torch.from_numpy(idx).long().to("cuda:0")].permute(1, 0, 2)).astype(np.float32),
              want[0].astype(np.float32), "s200 attention vs oracle")
    vc = v[:, :, :1].expand(1, H, ROWS, D).contiguous()
    out = ctx.attention_merged(q, k, vc).view(ROWS, H, D)
    err = (out.float() - vc[0, :, 0].float().unsqueeze(0)).abs().max().item()
    assert err <= 2e-3 * max(1.0, vc.float().abs().max().item()), f"constant V: {err}"


@pytest.mark.parametrize("name", ["fc1", "fc2"])
def test_linear_s200(ctx, name):
    """fc1 + bias + GELU (274,800 x 1024 -> 4096) and fc2 + bias + LayerScale
    + residual (274,800 x 4096 -> 1024): every output against float32 torch
    of the reference sequence (the linear's output stored as f16, then the
    epilogue), 4 rows against the oracle."""
    n, k = (4096, 1024) if name == "fc1" else (1024, 4096)
    print(f"[s200 {name}: m={ROWS} n={n} k={k}]", flush=True)
    x = randn((ROWS, k), 11 + n)
    w = randn((n, k), 12 + n, 1.0 / k ** 0.5)
    b = (randn((n,), 13 + n).float() * 0.02)
    y = (x.float() @ w.float().t().contiguous() + b).half().float()
    if name == "fc1":
        got = ctx.linear_gelu(x, w, b)
        ref = torch.nn.functional.gelu(y)
    else:
        res = randn((ROWS, n), 14 + n)
        gam = randn((n,), 15 + n).float() * 0.1
        got = ctx.linear_ls_residual(x, w, gam, res, b)
        ref = res.float() + gam * y
    del y
    err = max_scaled_err(got, ref)
    assert err <= 2e-3, f"s200 {name} vs torch f32: max scaled error {err:.3g}"
    rows = np.array([0, 70001, 199999, ROWS - 1])
    ri = torch.from_numpy(rows).to("cuda:0")
    xs, ws, bs = back(x[ri]), back(w), back(b)
    if name == "fc1":
        want = O.linear_gelu(xs, ws, bs)
    else:
        want = O.linear_ls_residual(xs, ws, back(gam), back(res[ri]), bs)
    f16_close(back(got[ri]).astype(np.float32), want.astype(np.float32), f"s200 {name} vs oracle")


def test_cache_build_s200(ctx):
    """The head-input cache at 274,800 rows, (rows, 2048) f32: bit-exact
    against the concatenation of the widened halves."""
    a, b = randn((ROWS, 1024), 21), randn((ROWS, 1024), 22)
    got = ctx.cache_build(a, b)
    assert torch.equal(got[:, :1024], a.float()) and torch.equal(got[:, 1024:], b.float())


def test_register_gather_scatter_200_frames(ctx):
    """The trunk's register-layer gather and scatter over 200 frames of
    1386 tokens (17 prefix + 37 x 37 patches), bit-exact against the
    per-frame copies."""
    n, t, p = 200, 1386, 17
    x = randn((n * t, 1024), 31)
    reg = torch.empty((n * p, 1024), dtype=torch.float16, device="cuda:0")
    ctx.copy_row_blocks(x, 0, t, reg, 0, p, n, p)
    want = x.view(n, t, 1024)[:, :p].reshape(n * p, 1024)
    assert_bit_exact(back(reg), back(want), "gather")
    y = randn((n * p, 1024), 32)
    ctx.copy_row_blocks(y, 0, p, x, 0, t, n, p)
    xv = x.view(n, t, 1024)
    assert torch.equal(xv[:, :p].reshape(n * p, 1024), y)
    assert torch.equal(xv[:, p:], randn((n * t, 1024), 31).view(n, t, 1024)[:, p:])
