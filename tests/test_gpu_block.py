"""A whole aggregator block on HIP (headshot_amd.aggregator.block_forward:
LN, the q/k/v linears, QK-norm + RoPE, attention, the proj/fc1/fc2 linears
with their epilogues fused) against the reference's unfused dispatch
sequence through the same library (block_forward_reference, model/
block.rs:118-193), and against a float32 torch restatement of the block.

Bars: fused vs the reference sequence within the f16 gate 2e-3 * max(1,
|e|) (they differ only where the fused ops skip or reorder a storage
rounding); against float32 torch within 1e-2 * max(1, |e|), the f16
storage roundings of a dozen dispatches accumulating.
"""
import numpy as np
import pytest
import torch

from headshot_amd import rope as rp
from headshot_amd.aggregator import BlockWeights, block_forward, block_forward_reference
from headshot_amd.parity import f16_close

pytestmark = pytest.mark.gpu

DIM, HEADS, HIDDEN, PREFIX = 1024, 16, 4096, 5


def back(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def torch_block(wts, x, s, t, rope, eps):
    """float32 restatement of Block::forward on the same (f16) values."""
    f = lambda a: a.float()  # noqa: E731
    p = wts.p
    ln = lambda a, wb: torch.nn.functional.layer_norm(a, (a.shape[-1],), f(wb[0]), f(wb[1]), eps)  # noqa: E731
    x = f(x)
    normed = ln(x, p.ln1)

    def heads(w_, b_):
        y = normed @ f(w_).t().contiguous() + b_
        return y.view(s, t, HEADS, 64).permute(0, 2, 1, 3).contiguous()

    q, k, v = heads(wts.q_w, wts.q_b), heads(wts.k_w, wts.k_b), heads(wts.v_w, wts.v_b)
    if p.qn is not None:
        q, k = ln(q, p.qn), ln(k, p.kn)
    if rope is not None:
        sin, cos, pre = rope
        def rot(a):
            lo, hi = a[..., pre:, :32], a[..., pre:, 32:]
            out = a.clone()
            out[..., pre:, :32] = lo * cos[:, :32] - hi * sin[:, :32]
            out[..., pre:, 32:] = hi * cos[:, 32:] + lo * sin[:, 32:]
            return out
        q, k = rot(q), rot(k)
    sc = torch.matmul(q, k.transpose(-1, -2).contiguous()) / 8.0
    attn = torch.matmul(torch.softmax(sc, dim=-1), v)
    merged = attn.permute(0, 2, 1, 3).reshape(s * t, DIM)
    x1 = x + p.ls1 * (merged @ f(wts.proj_w).t().contiguous() + p.proj_b)
    normed2 = ln(x1, p.ln2)
    h = torch.nn.functional.gelu(normed2 @ f(wts.fc1_w).t().contiguous() + p.fc1_b)
    return x1 + p.ls2 * (h @ f(wts.fc2_w).t().contiguous() + p.fc2_b)


@pytest.mark.parametrize("kind", ["frame", "global"])
def test_block_small(ctx, kind):
    g = torch.Generator(device="cpu").manual_seed(5)
    if kind == "frame":
        s, grid = 2, (5, 29)
        t = PREFIX + grid[0] * grid[1]
        sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), *grid))
        rope = (sin, cos, PREFIX)
    else:
        s, t, rope = 1, 300, None
    wts = BlockWeights.random(DIM, HIDDEN, 64, torch.float16, "cuda:0",
                              torch.Generator(device="cuda:0").manual_seed(5), ls_init=0.1)
    x = torch.randn((s * t, DIM), generator=g).half().to("cuda:0")
    fused = back(block_forward(ctx, wts, x, s, t, rope=rope))
    seq = back(block_forward_reference(ctx, wts, x, s, t, rope=rope))
    f16_close(fused, seq, f"block {kind} fused vs reference sequence")
    ref = back(torch_block(wts, x, s, t, rope, 1e-6))
    err = np.abs(fused - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 1e-2, f"block {kind} vs float32: max scaled error {err.max():.3g}"


@pytest.mark.parametrize("kind", ["frame", "global"])
def test_block_f32_s2(ctx, kind):
    """The reference's f32 path at S=2 x 1374 (37x37 grid, prefix 5): a
    whole block in f32 (f32 linear layers and attention on the matrix cores)
    against the reference's unfused sequence through the same library
    (within 1e-5 * max(1, |e|): only summation orders differ) and against
    the float32 torch restatement (within 1e-4 * max(1, |e|), the
    reference's f32 gate)."""
    g = torch.Generator(device="cpu").manual_seed(8)
    grid = (37, 37)
    t = PREFIX + grid[0] * grid[1]
    if kind == "frame":
        s = 2
        sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), *grid))
        rope = (sin, cos, PREFIX)
    else:
        s, t, rope = 1, 2 * t, None
    wts = BlockWeights.random(DIM, HIDDEN, 64, torch.float32, "cuda:0",
                              torch.Generator(device="cuda:0").manual_seed(8), ls_init=0.1)
    x = torch.randn((s * t, DIM), generator=g).to("cuda:0")
    fused = back(block_forward(ctx, wts, x, s, t, rope=rope))
    seq = back(block_forward_reference(ctx, wts, x, s, t, rope=rope))
    err = np.abs(fused - seq) / np.maximum(1.0, np.abs(seq))
    assert err.max() <= 1e-5, f"f32 block {kind} fused vs reference sequence: {err.max():.3g}"
    ref = back(torch_block(wts, x, s, t, rope, 1e-6))
    err = np.abs(fused - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 1e-4, f"f32 block {kind} vs float32 torch: max scaled error {err.max():.3g}"


def test_block_full_size_frame(ctx):
    """A frame block at S=32 (32 x 1374 tokens, 37x37 grid, prefix 5)."""
    g = torch.Generator(device="cpu").manual_seed(6)
    s, grid = 32, (37, 37)
    t = PREFIX + grid[0] * grid[1]
    sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), *grid))
    wts = BlockWeights.random(DIM, HIDDEN, 64, torch.float16, "cuda:0",
                              torch.Generator(device="cuda:0").manual_seed(6), ls_init=0.1)
    x = torch.randn((s * t, DIM), generator=g).half().to("cuda:0")
    fused = back(block_forward(ctx, wts, x, s, t, rope=(sin, cos, PREFIX)))
    seq = back(block_forward_reference(ctx, wts, x, s, t, rope=(sin, cos, PREFIX)))
    f16_close(fused, seq, "full-size frame block fused vs reference sequence")


@pytest.mark.parametrize("kind", ["frame", "global"])
def test_block_ln_prologue(ctx, kind):
    """The block with each LayerNorm as the prologue of the product after it
    (fuse_ln) is bit-identical to the block with the LayerNorm passes, frame
    block at S=2 and global block at T=300."""
    g = torch.Generator(device="cpu").manual_seed(15)
    if kind == "frame":
        s, grid = 2, (5, 29)
        t = PREFIX + grid[0] * grid[1]
        sin, cos = (torch.from_numpy(a).to("cuda:0") for a in rp.tables(rp.periods(), *grid))
        rope = (sin, cos, PREFIX)
    else:
        s, t, rope = 1, 300, None
    wts = BlockWeights.random(DIM, HIDDEN, 64, torch.float16, "cuda:0",
                              torch.Generator(device="cuda:0").manual_seed(15), ls_init=0.1)
    x = torch.randn((s * t, DIM), generator=g).half().to("cuda:0")
    fused = block_forward(ctx, wts, x, s, t, rope=rope, fuse_ln=True)
    unfused = block_forward(ctx, wts, x, s, t, rope=rope, fuse_ln=False)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16)), \
        f"block {kind}: {(fused != unfused).sum().item()} values differ with the LayerNorm prologue"
