"""The fused per-layer ops at the benchmark configurations' real shapes.

Each configuration runs one frame block (QK-norm + 2D RoPE) and/or one
global block (QK-norm, no RoPE) of the aggregator through HipContext and
compares every output with the oracle running the reference's unfused
dispatch sequence on the same inputs: at full size where the oracle takes
seconds, on sampled token rows (plus size-independent invariants) at the
274,800-token length. Also: HIP-graph replays of a pass against eager
launches.

Bars: f32 |a-e| <= 1e-5 + 1e-5|e|; f16 |a-e| <= 2e-3 * max(1, |e|);
permutations, copies and RoPE tables bit-exact.
"""
import hashlib
import json
import os
import zlib

import numpy as np
import pytest
import torch

from headshot_amd import rope
from headshot_amd.aggregator import BlockIO, BlockParams, FusedOpPass, run_block_ops
from headshot_amd.parity import Gate, assert_bit_exact, assert_close, compare, f16_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
DIM, HEADS, HD, HIDDEN = 1024, 16, 64, 4096


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def gate(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    if got.dtype == np.float32:
        assert_close(got, want, 1e-5, what)
    else:
        f16_close(got.astype(np.float32), want.astype(np.float32), what)


def make_block(ctx, rows, dtype, seed, ls_init=1e-5):
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    n = lambda *s: torch.randn(s, generator=g, device="cuda:0").to(dtype)  # noqa: E731
    io = BlockIO.empty_like_inputs(n(rows, DIM), n(rows, DIM), n(rows, DIM), n(rows, DIM),
                                   n(rows, HIDDEN), n(rows, DIM))
    p = BlockParams.random(DIM, HIDDEN, HD, "cuda:0", g, ls_init=ls_init)
    return io, p


def oracle_block(io, p, s, t, rope_tabs, eps, dt):
    """O.block_ops on host copies: the reference's dispatch sequence."""
    h = host
    out = {k: np.empty_like(h(getattr(io, k))) for k in
           ("normed", "q_head", "k_head", "x1", "normed2", "act", "x_out")}
    sin, cos, prefix = rope_tabs if rope_tabs is not None else (None, None, 0)
    P = {k: (tuple(h(x) for x in v) if isinstance(v, tuple) else h(v)) for k, v in vars(p).items()}
    O.block_ops(dt, h(io.x), *P["ln1"], h(io.q_raw), h(io.k_raw), *P["qn"], *P["kn"],
                None if sin is None else h(sin), None if cos is None else h(cos), prefix,
                h(io.proj_raw), P["proj_b"], P["ls1"], *P["ln2"], h(io.fc1_raw), P["fc1_b"],
                h(io.fc2_raw), P["fc2_b"], P["ls2"], out, s, t, DIM, HEADS, HIDDEN, eps)
    return out


def check_block(io, ref, what):
    for k in ("normed", "q_head", "k_head", "x1", "normed2", "act", "x_out"):
        got = host(getattr(io, k)).reshape(ref[k].shape)
        gate(got, ref[k], f"{what} {k}")
        Gate.F16_TRUNK.check(f"{what} {k}", compare(got.astype(np.float32), ref[k].astype(np.float32)))


def tables(grid):
    sin, cos = rope.tables(rope.periods(), *grid)
    return torch.from_numpy(sin).cuda(), torch.from_numpy(cos).cuda()


@pytest.mark.parametrize("cfg", [
    # name, frames, grid, dtype, kinds
    ("f32 S=2 37x37", 2, (37, 37), torch.float32, ("frame", "global")),
    ("f16 S=8 37x37", 8, (37, 37), torch.float16, ("frame",)),
    ("f16 S=32 37x37", 32, (37, 37), torch.float16, ("frame", "global")),
    ("f32 S=16 21x37", 16, (21, 37), torch.float32, ("frame", "global")),
    ("f16 S=16 21x37", 16, (21, 37), torch.float16, ("frame", "global")),
])
def test_block_ops_full_size(ctx, cfg):
    name, frames, grid, dtype, kinds = cfg
    t = grid[0] * grid[1] + 5
    rows = frames * t
    O.set_num_threads(min(16, os.cpu_count() or 1))
    dt = O.F16 if dtype == torch.float16 else O.F32
    sin, cos = tables(grid)
    for kind in kinds:
        io, p = make_block(ctx, rows, dtype, seed=zlib.crc32(f"{name} {kind}".encode()) % 1000)
        if kind == "frame":
            s, tt, rp = frames, t, (sin, cos, 5)
        else:
            s, tt, rp = 1, rows, None
        print(f"[{name} {kind} block: rows={rows}]", flush=True)
        run_block_ops(ctx, p, io, s, tt, HEADS, HD, rope=rp, eps=1e-6)
        check_block(io, oracle_block(io, p, s, tt, rp, 1e-6, dt), f"{name} {kind}")


def test_layerscale_sensitivity(ctx):
    """LayerScale 1e-5 hides the residual branch in f16 (out == res almost
    everywhere); gamma ~ N(0,1) makes the branch visible."""
    rows = 4 * 1374
    io, p = make_block(ctx, rows, torch.float16, seed=7, ls_init=None)
    sin, cos = tables((37, 37))
    run_block_ops(ctx, p, io, 4, 1374, HEADS, HD, rope=(sin, cos, 5), eps=1e-6)
    ref = oracle_block(io, p, 4, 1374, (sin, cos, 5), 1e-6, O.F16)
    check_block(io, ref, "gamma~N(0,1)")
    assert not np.array_equal(host(io.x1), host(io.x)), "residual branch must be visible"


def test_trunk_prefix_17(ctx):
    """VGGT-Omega trunk frame blocks: 1 camera + 16 register tokens unrotated."""
    grid, prefix, frames = (16, 16), 17, 3
    t = grid[0] * grid[1] + prefix
    x = torch.randn(frames * t, DIM, device="cuda:0").half()
    nw = torch.randn(HD, device="cuda:0") * 0.02 + 1
    nb = torch.randn(HD, device="cuda:0") * 0.02
    sin, cos = tables(grid)
    got = host(ctx.qknorm_rope(x, frames, t, HEADS, HD, norm=(nw, nb), rope=(sin, cos, prefix)))
    want = O.qknorm_rope(host(x), host(nw), host(nb), host(sin), host(cos), frames, t, HEADS, HD,
                         prefix, 1e-5)
    gate(got, want, "prefix 17")


def test_non_square_tables_bit_exact_and_used(ctx):
    """The non-square 21x37 grid: the tables equal the golden fixture and the
    kernel's rotation uses row t - prefix of them."""
    g = json.load(open(os.path.join(HERE, "golden", "rope_tables.json")))["grids"]["21x37"]
    sin, cos = rope.tables(rope.periods(), 21, 37)
    assert hashlib.sha256(sin.tobytes()).hexdigest() == g["sin_sha256"]
    assert hashlib.sha256(cos.tobytes()).hexdigest() == g["cos_sha256"]
    t = 777 + 5
    x = torch.randn(2 * t, DIM, device="cuda:0")
    got = host(ctx.qknorm_rope(x, 2, t, HEADS, HD, rope=(torch.from_numpy(sin).cuda(),
                                                         torch.from_numpy(cos).cuda(), 5)))
    xs = host(x).reshape(2, t, HEADS, HD)
    for tok in (5, 6, 400, t - 1):
        want = O.rope_apply_cpu(xs[1, tok, 3], sin, cos, tok - 5)
        assert_close(got[1, 3, tok], want, 1e-5, f"token {tok}")
    assert_bit_exact(got[:, :, :5], np.ascontiguousarray(xs[:, :5].transpose(0, 2, 1, 3)), "prefix")


@pytest.mark.parametrize("frames,p", [(32, 1369), (16, 777)], ids=["s32_37x37", "s16_21x37"])
def test_assembly_full_size(ctx, frames, p):
    """The assembly at S=32 x 37 x 37 and S=16 x 21 x 37 patches: f32 patches
    + bias + pos-embed -> f16 tokens, with camera/register variants for frame
    0 and the rest; bit-exact."""
    r = 4
    g = torch.Generator(device="cuda:0")
    g.manual_seed(3 + p)
    patches = torch.randn(frames * p, DIM, generator=g, device="cuda:0")
    pos = torch.randn(p, DIM, generator=g, device="cuda:0") * 0.02
    pb = torch.randn(DIM, generator=g, device="cuda:0") * 0.02
    cam = torch.randn(2, DIM, generator=g, device="cuda:0").half()
    reg = torch.randn(2 * r, DIM, generator=g, device="cuda:0").half()
    got = host(ctx.assemble_tokens(patches, frames, p, cam, reg, patch_bias=pb, pos=pos))
    want = O.assemble_tokens(host(patches), host(pb), host(pos), host(cam), host(reg), frames, p,
                             r, np.float16)
    assert_bit_exact(got, want, f"assembly S={frames} P={p}")


def test_assembly_dino_layout_full_size(ctx):
    """The DINO stage's assembly (model/dino.rs:76-93): per frame [cls,
    storage x 4, patches + patch-embed bias], one token variant for every
    frame (n_var 1), f32 in and out, at D=1024 on 16 frames of the
    non-square 21 x 37 = 777-patch grid; bit-exact."""
    frames, p, r = 16, 777, 4
    g = torch.Generator(device="cuda:0")
    g.manual_seed(21)
    patches = torch.randn(frames * p, DIM, generator=g, device="cuda:0")
    pb = torch.randn(DIM, generator=g, device="cuda:0") * 0.02
    cls = torch.randn(1, DIM, generator=g, device="cuda:0")
    storage = torch.randn(r, DIM, generator=g, device="cuda:0")
    print(f"[dino assembly: frames={frames} p={p} n_var=1 f32]", flush=True)
    got = host(ctx.assemble_tokens(patches, frames, p, cls, storage, patch_bias=pb, pos=None,
                                   out_dtype=torch.float32, n_var=1))
    want = O.assemble_tokens(host(patches), host(pb), None, host(cls), host(storage), frames, p,
                             r, np.float32, n_var=1)
    assert_bit_exact(got, want, "dino assembly S=16 x 777")
    # every frame carries the same cls and storage rows, then its own patches
    t = 1 + r + p
    g3 = got.reshape(frames, t, DIM)
    assert_bit_exact(g3[:, 0], np.broadcast_to(host(cls), (frames, DIM)), "cls rows")
    assert_bit_exact(g3[:, 1:1 + r], np.broadcast_to(host(storage), (frames, r, DIM)), "storage")


def test_s200_frame_layout_rope(ctx):
    """The S=200 qk-norm + RoPE2D leg: S=200 frames x 1374 tokens in the
    frame-block layout (37 x 37 tables, prefix 5), q and k in one launch.
    Oracle on 4 whole frames (5,496 tokens); at full size RoPE preserves
    every pair norm of the normalised vectors and the 5 prefix tokens pass
    through bit-exact."""
    frames, t, prefix = 200, 1374, 5
    rows = frames * t
    g = torch.Generator(device="cuda:0")
    g.manual_seed(33)
    q = torch.randn(rows, DIM, generator=g, device="cuda:0").half()
    k = torch.randn(rows, DIM, generator=g, device="cuda:0").half()
    qn = (torch.randn(HD, generator=g, device="cuda:0") * 0.02 + 1,
          torch.randn(HD, generator=g, device="cuda:0") * 0.02)
    kn = (torch.randn(HD, generator=g, device="cuda:0") * 0.02 + 1,
          torch.randn(HD, generator=g, device="cuda:0") * 0.02)
    sin, cos = tables((37, 37))
    print(f"[s200 frame layout: rows={rows}]", flush=True)
    qh, kh = ctx.qknorm_rope_pair(q, k, frames, t, HEADS, HD, qn=qn, kn=kn,
                                  rope=(sin, cos, prefix), eps=1e-6)
    O.set_num_threads(min(16, os.cpu_count() or 1))
    for name, src, nrm, got in (("q", q, qn, qh), ("k", k, kn, kh)):
        for f in (0, 57, 123, 199):
            x_f = host(src[f * t:(f + 1) * t])
            want = O.qknorm_rope(x_f, host(nrm[0]), host(nrm[1]), host(sin), host(cos), 1, t,
                                 HEADS, HD, prefix, 1e-6)
            gate(host(got[f]), want[0], f"s200 {name} frame {f}")
    # full size: the same normalisation without RoPE ...
    qa, ka = ctx.qknorm_rope_pair(q, k, frames, t, HEADS, HD, qn=qn, kn=kn, rope=None, eps=1e-6)
    for name, rot, plain in (("q", qh, qa), ("k", kh, ka)):
        r32, p32 = rot.float(), plain.float()
        nr = torch.hypot(r32[..., :32], r32[..., 32:])
        np_ = torch.hypot(p32[..., :32], p32[..., 32:])
        # rotating an f16 pair and rounding each component to f16 again
        # moves its norm by at most 2^-11 of the norm (half an f16 ulp per
        # component), plus f32 rounding
        err = ((nr - np_).abs() / np_.clamp_min(1.0)).max().item()
        assert err < 1e-3, f"s200 {name} pair norms moved by {err}"
        assert torch.equal(rot[:, :, :prefix], plain[:, :, :prefix]), f"{name} prefix passthrough"
        del r32, p32, nr, np_


def test_global_block_long_sequence(ctx):
    """S=200 frames flattened to one 274,800-token sequence through
    the global-block ops (no RoPE). Oracle on 512 sampled token rows; the
    split is checked bit-exact at full size; LN invariants at full size."""
    rows = 200 * 1374
    dtype = torch.float16
    io, p = make_block(ctx, rows, dtype, seed=11)
    print(f"[s200 global block: rows={rows}]", flush=True)
    run_block_ops(ctx, p, io, 1, rows, HEADS, HD, rope=None, eps=1e-6)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    idx = np.sort(rng.choice(rows, 512, replace=False))
    ii = torch.from_numpy(idx).cuda()
    sel = lambda t: host(t.index_select(0, ii))  # noqa: E731
    P = {k: (tuple(host(x) for x in v) if isinstance(v, tuple) else host(v))
         for k, v in vars(p).items()}
    x, x1 = sel(io.x), sel(io.x1)
    gate(sel(io.normed), O.layernorm(x, *P["ln1"], 1e-6), "LN1")
    gate(x1, O.bias_ls_residual(x, sel(io.proj_raw), P["proj_b"], P["ls1"]), "LS1")
    gate(sel(io.normed2), O.layernorm(x1, *P["ln2"], 1e-6), "LN2")
    gate(sel(io.act), O.bias_gelu(sel(io.fc1_raw), P["fc1_b"]), "GELU")
    gate(sel(io.x_out), O.bias_ls_residual(x1, sel(io.fc2_raw), P["fc2_b"], P["ls2"]), "LS2")
    qh = io.q_head.view(1, HEADS, rows, HD)
    got_q = host(qh[0][:, ii])                                   # (H, n, 64)
    want_q = O.qknorm_rope(sel(io.q_raw), *P["qn"], None, None, 1, len(idx), HEADS, HD, 0, 1e-6)
    gate(got_q, want_q[0], "QK-norm")
    # full-size invariants: pure split is an exact permutation ...
    split = ctx.qknorm_rope(io.q_raw, 1, rows, HEADS, HD)
    perm = io.q_raw.view(1, rows, HEADS, HD).permute(0, 2, 1, 3).contiguous()
    assert torch.equal(split.view_as(perm), perm)
    # ... and LN with unit weight / zero bias has per-row mean 0, variance 1
    ones, zeros = torch.ones(DIM, device="cuda:0"), torch.zeros(DIM, device="cuda:0")
    y = ctx.layernorm(io.x, ones, zeros, eps=1e-6).float()
    assert y.mean(dim=1).abs().max().item() < 2e-3
    assert (y.var(dim=1, unbiased=False) - 1).abs().max().item() < 5e-3


def test_rope_preserves_pair_norms_full_size(ctx):
    frames, grid = 32, (37, 37)
    t = 1374
    x = torch.randn(frames * t, DIM, device="cuda:0")
    sin, cos = tables(grid)
    nw = torch.randn(HD, device="cuda:0") * 0.02 + 1
    nb = torch.randn(HD, device="cuda:0") * 0.02
    a = ctx.qknorm_rope(x, frames, t, HEADS, HD, norm=(nw, nb), rope=None)
    b = ctx.qknorm_rope(x, frames, t, HEADS, HD, norm=(nw, nb), rope=(sin, cos, 5))
    na = torch.hypot(a[..., :32], a[..., 32:])
    nb_ = torch.hypot(b[..., :32], b[..., 32:])
    assert (na - nb_).abs().max().item() < 1e-5 * max(1.0, na.abs().max().item())
    assert torch.equal(a[:, :, :5], b[:, :, :5]), "prefix tokens must pass through"


@pytest.mark.parametrize("frames,grid,dtype", [(2, (37, 37), torch.float16),
                                               (2, (21, 37), torch.float32)])
def test_fused_pass_equals_six_op_pass(ctx, frames, grid, dtype):
    """The pass with every LayerScale + residual fused with the LayerNorm
    after it (LS1 with LN2, LS2 with the next block's LN1) against the same
    pass with the six single ops per block, same seed: bit-identical block
    outputs and LayerNorm outputs."""
    a = FusedOpPass(ctx, frames, grid=grid, n_frame=3, n_global=3, dtype=dtype, fuse=True)
    b = FusedOpPass(ctx, frames, grid=grid, n_frame=3, n_global=3, dtype=dtype, fuse=False)
    assert len(a.seq) == 1 + 4 * 6 + 1 and len(b.seq) == 1 + 6 * 6
    a.run()
    b.run()
    torch.cuda.synchronize()
    for k in ("normed", "normed2", "act", "x1", "q_head", "k_head"):
        assert_bit_exact(host(getattr(a.io, k)), host(getattr(b.io, k)), f"fused pass {k}")
    assert_bit_exact(host(a.out), host(b.out), "fused pass output")


@pytest.mark.parametrize("fuse", [False, True])
def test_graph_replay_matches_eager(ctx, fuse):
    """The pass (six ops per block, or four with LayerScale + LayerNorm
    fused) captured in a HIP graph, replayed three times with eager work and
    synchronisation between replays; every replay equals eager launches."""
    fp = FusedOpPass(ctx, frames=2, grid=(4, 4), n_frame=2, n_global=2, fuse=fuse)
    fp.run()
    torch.cuda.synchronize()
    eager = {k: host(getattr(fp.io, k)).copy() for k in ("q_head", "k_head", "act", "normed2")}
    eager["out"] = host(fp.out).copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fp.run()
    for i in range(3):
        junk = torch.randn(1 << 20, device="cuda:0")
        fp.io.act.zero_()
        fp.out.zero_()
        torch.cuda.synchronize()
        del junk
        graph.replay()
        torch.cuda.synchronize()
        for k in ("q_head", "k_head", "act", "normed2"):
            assert_bit_exact(host(getattr(fp.io, k)), eager[k], f"replay {i} {k}")
        assert_bit_exact(host(fp.out), eager["out"], f"replay {i} out")
