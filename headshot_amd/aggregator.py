"""The aggregator's per-layer op sequence on HipContext.

``BlockParams`` holds one pre-norm block's f32 parameters and
``run_block_ops`` issues that block's fused per-layer ops in the order of
``Block::forward`` (crates/headshot-server/src/model/block.rs:118-159) with
the GEMMs and attention left to the caller: their raw outputs come in as
tensors, and the biases of proj/fc1/fc2 are applied by the fused ops.

``FusedOpPass`` lays out every buffer of one aggregator pass (token
assembly, model/trunk.rs:68-85, then alternating frame and global blocks,
model/trunk.rs:92-143) and records the launch sequence as re-issuable C-ABI
calls, so the whole pass can be replayed or captured in a HIP graph.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import rope as _rope
from .context import HipContext

DIM, HEADS, HEAD_DIM, HIDDEN = 1024, 16, 64, 4096


@dataclass
class BlockParams:
    ln1: tuple            # (weight, bias) f32 (dim)
    ln2: tuple
    qn: tuple | None      # QK-norm (weight, bias) f32 (head_dim), None = no QK-norm
    kn: tuple | None
    proj_b: torch.Tensor  # f32 (dim)
    ls1: torch.Tensor     # LayerScale gamma f32 (dim)
    fc1_b: torch.Tensor   # f32 (hidden)
    fc2_b: torch.Tensor   # f32 (dim)
    ls2: torch.Tensor

    @staticmethod
    def random(dim: int, hidden: int, head_dim: int, device, generator, qk_norm: bool = True,
               ls_init: float | None = 1e-5) -> "BlockParams":
        """Random init as the benchmark workloads draw it: LN gamma ~N(1,.02), beta and
        biases ~N(0,.02), LayerScale = ls_init (or ~N(0,1) when None)."""
        def n(shape, mean=0.0, std=1.0):
            return torch.randn(shape, generator=generator, device=device) * std + mean

        def ls():
            return torch.full((dim,), ls_init, device=device) if ls_init is not None else n(dim)

        qn = (n(head_dim, 1.0, 0.02), n(head_dim, 0.0, 0.02)) if qk_norm else None
        kn = (n(head_dim, 1.0, 0.02), n(head_dim, 0.0, 0.02)) if qk_norm else None
        return BlockParams(ln1=(n(dim, 1.0, 0.02), n(dim, 0.0, 0.02)),
                           ln2=(n(dim, 1.0, 0.02), n(dim, 0.0, 0.02)), qn=qn, kn=kn,
                           proj_b=n(dim, 0.0, 0.02), ls1=ls(), fc1_b=n(hidden, 0.0, 0.02),
                           fc2_b=n(dim, 0.0, 0.02), ls2=ls())


@dataclass
class BlockIO:
    """Per-block buffers: inputs x and the raw GEMM outputs, plus outputs."""
    x: torch.Tensor          # (S*T, dim) residual stream in
    q_raw: torch.Tensor      # (S*T, H*hd) q projection (qkv bias already added)
    k_raw: torch.Tensor
    proj_raw: torch.Tensor   # (S*T, dim) attention projection without bias
    fc1_raw: torch.Tensor    # (S*T, hidden) fc1 output without bias
    fc2_raw: torch.Tensor    # (S*T, dim) fc2 output without bias
    normed: torch.Tensor     # LN1 output
    q_head: torch.Tensor     # (S, H, T, hd)
    k_head: torch.Tensor
    x1: torch.Tensor         # residual after attention
    normed2: torch.Tensor    # LN2 output
    act: torch.Tensor        # GELU output
    x_out: torch.Tensor      # block output

    @staticmethod
    def empty_like_inputs(x, q_raw, k_raw, proj_raw, fc1_raw, fc2_raw) -> "BlockIO":
        e = torch.empty_like
        return BlockIO(x, q_raw, k_raw, proj_raw, fc1_raw, fc2_raw, e(x), e(q_raw), e(k_raw),
                       e(x), e(x), e(fc1_raw), e(x))


def run_block_ops(ctx: HipContext, p: BlockParams, io: BlockIO, s: int, t: int, heads: int,
                  head_dim: int, rope=None, eps: float = 1e-5, record=None, fuse: bool = False,
                  ln1_done: bool = False, next_ln1=None) -> None:
    """One block's per-layer ops (model/block.rs:128-155 minus GEMMs and
    attention). ``rope`` = (sin, cos, prefix) for frame blocks, None for
    global blocks (which the trunk runs as one sequence, s=1, t=S*T).
    ``record(op_name)`` is called after each launch (for launch recording).

    With ``fuse`` each LayerScale + residual and the LayerNorm of its output
    run as one launch (``bias_ls_residual_layernorm``, bit-identical to the
    two): LS1 with LN2, and, when ``next_ln1`` (the next block's LN1 weight
    and bias) is given, LS2 with the next block's LN1 into ``io.normed``;
    ``ln1_done`` skips this block's LN1, done so by the block before."""
    rec = record or (lambda op: None)
    if not ln1_done:
        ctx.layernorm(io.x, *p.ln1, eps=eps, out=io.normed)
        rec("layernorm")
    # always: with neither QK-norm nor RoPE this is the plain split_heads
    # the reference runs unconditionally (model/block.rs:130-133)
    ctx.qknorm_rope_pair(io.q_raw, io.k_raw, s, t, heads, head_dim, qn=p.qn, kn=p.kn,
                         rope=rope, eps=eps, out_q=io.q_head, out_k=io.k_head)
    rec("qknorm_rope")
    if fuse:
        ctx.bias_ls_residual_layernorm(io.x, io.proj_raw, p.ls1, p.proj_b, p.ln2, eps=eps,
                                       out=io.x1, normed=io.normed2)
        rec("bias_ls_residual_layernorm")
    else:
        ctx.bias_ls_residual(io.x, io.proj_raw, p.ls1, p.proj_b, out=io.x1)
        rec("bias_ls_residual")
        ctx.layernorm(io.x1, *p.ln2, eps=eps, out=io.normed2)
        rec("layernorm")
    ctx.bias_gelu(io.fc1_raw, p.fc1_b, out=io.act)
    rec("bias_gelu")
    if fuse and next_ln1 is not None:
        ctx.bias_ls_residual_layernorm(io.x1, io.fc2_raw, p.ls2, p.fc2_b, next_ln1, eps=eps,
                                       out=io.x_out, normed=io.normed)
        rec("bias_ls_residual_layernorm")
    else:
        ctx.bias_ls_residual(io.x1, io.fc2_raw, p.ls2, p.fc2_b, out=io.x_out)
        rec("bias_ls_residual")


class FusedOpPass:
    """All buffers and the launch sequence of one aggregator fused-op pass:
    assembly, then ``n_frame`` frame blocks (QK-norm + RoPE, ``prefix``
    unrotated tokens) alternating with ``n_global`` global blocks (QK-norm,
    no RoPE). Inputs are synthetic: seeded N(0,1) activations and GEMM
    outputs, random-init parameters (``BlockParams.random``). With
    ``distinct_inputs`` every block reads raw GEMM outputs of its own (as
    in the trunk, where each block's products are new data); otherwise all
    blocks share one set. With ``fuse`` (``run_block_ops``) every
    LayerScale + residual is one launch with the LayerNorm after it: LS1
    with LN2, LS2 with the next block's LN1 (the first block's LN1 and the
    last block's LS2 stay single ops)."""

    def __init__(self, ctx: HipContext, frames: int, grid=(37, 37), n_reg: int = 4,
                 n_frame: int = 24, n_global: int = 24, dtype=torch.float16, eps: float = 1e-6,
                 dim: int = DIM, heads: int = HEADS, hidden: int = HIDDEN, seed: int = 42,
                 distinct_inputs: bool = False, fuse: bool = False):
        self.ctx, self.frames, self.dtype, self.eps = ctx, frames, dtype, eps
        self.fuse = fuse
        self.dim, self.heads, self.hidden = dim, heads, hidden
        self.head_dim = dim // heads
        dev = ctx.device
        self.p = grid[0] * grid[1]
        self.n_reg = n_reg
        self.prefix = 1 + n_reg
        self.t = self.p + self.prefix
        self.rows = rows = frames * self.t
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def normal(shape, mean=0.0, std=1.0, dt=torch.float32):
            return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std
                    + mean).to(dt)

        self.patches = normal((frames * self.p, dim))          # f32 stage input
        self.pos = normal((self.p, dim), 0.0, 0.02)
        self.patch_bias = normal((dim,), 0.0, 0.02)
        self.cam = normal((2, dim), dt=dtype)
        self.reg = normal((2 * n_reg, dim), dt=dtype)
        def raw_outputs():
            """q, k (qkv bias added), proj, fc1, fc2 products of one block."""
            return (normal((rows, dim), dt=dtype), normal((rows, dim), dt=dtype),
                    normal((rows, dim), dt=dtype), normal((rows, hidden), dt=dtype),
                    normal((rows, dim), dt=dtype))

        kinds = []
        for i in range(max(n_frame, n_global)):
            if i < n_frame:
                kinds.append("frame")
            if i < n_global:
                kinds.append("global")
        self.kinds = kinds
        raws = [raw_outputs()] * len(kinds) if not distinct_inputs else [raw_outputs() for _ in kinds]
        self.raws = raws
        x0 = torch.empty((rows, dim), device=dev, dtype=dtype)
        x_b = torch.empty_like(x0)
        io = BlockIO.empty_like_inputs(x0, *raws[0][:3], raws[0][3], raws[0][4])
        io.x_out = x_b
        self.io = io
        self.x = [x0, x_b]
        sin, cos = _rope.tables(_rope.periods(), *grid)
        self.sin = torch.from_numpy(sin).to(dev)
        self.cos = torch.from_numpy(cos).to(dev)
        self.blocks = [BlockParams.random(dim, hidden, self.head_dim, dev, g) for _ in kinds]
        self.seq = self._record()

    def _record(self):
        """Run the pass once through HipContext (validating every call) and
        keep each launch as a re-issuable raw call: [(op, thunk)]."""
        c = self.ctx
        seq = []

        def rec(op):
            seq.append((op, c.last_launch))

        io = self.io
        c.assemble_tokens(self.patches, self.frames, self.p, self.cam, self.reg,
                          patch_bias=self.patch_bias, pos=self.pos, out_dtype=self.dtype,
                          out=self.x[0])
        rec("assemble")
        x = self.x[0]
        n = len(self.blocks)
        for i, (kind, p, raw) in enumerate(zip(self.kinds, self.blocks, self.raws)):
            io.q_raw, io.k_raw, io.proj_raw, io.fc1_raw, io.fc2_raw = raw
            io.x = x
            io.x_out = self.x[1] if x is self.x[0] else self.x[0]
            if kind == "frame":
                s, t, rp = self.frames, self.t, (self.sin, self.cos, self.prefix)
            else:
                s, t, rp = 1, self.rows, None
            nxt = self.blocks[i + 1].ln1 if self.fuse and i + 1 < n else None
            run_block_ops(c, p, io, s, t, self.heads, self.head_dim, rope=rp, eps=self.eps,
                          record=rec, fuse=self.fuse, ln1_done=self.fuse and i > 0, next_ln1=nxt)
            x = io.x_out
        self.out = x
        return seq

    def run(self) -> None:
        for _, thunk in self.seq:
            thunk()

    def launches(self) -> dict:
        counts = {}
        for op, _ in self.seq:
            counts[op] = counts.get(op, 0) + 1
        return counts


# ---------------------------------------------------------------------------
# a whole block on HipContext: GEMMs and attention included


@dataclass
class BlockWeights:
    """One block's weights (model/block.rs:60-110): the linear weights in
    the storage dtype, everything else f32 (``p``). The attention input
    projection stays fused as the checkpoint stores it, q | k | v on the
    output rows of ``qkv_w``; ``q_w`` .. ``v_b`` are its row slices (views)."""
    p: BlockParams
    qkv_w: torch.Tensor   # (3 dim, dim) storage dtype; rows = output features
    qkv_b: torch.Tensor   # f32 (3 dim)
    proj_w: torch.Tensor  # (dim, dim)
    fc1_w: torch.Tensor   # (hidden, dim)
    fc2_w: torch.Tensor   # (dim, hidden)

    def _third(self, t, i):
        dim = self.qkv_w.shape[1]
        return t[i * dim:(i + 1) * dim]

    q_w = property(lambda self: self._third(self.qkv_w, 0))
    k_w = property(lambda self: self._third(self.qkv_w, 1))
    v_w = property(lambda self: self._third(self.qkv_w, 2))
    q_b = property(lambda self: self._third(self.qkv_b, 0))
    k_b = property(lambda self: self._third(self.qkv_b, 1))
    v_b = property(lambda self: self._third(self.qkv_b, 2))

    @staticmethod
    def random(dim: int, hidden: int, head_dim: int, dtype, device, generator,
               qk_norm: bool = True, ls_init: float | None = 1e-5) -> "BlockWeights":
        """Random init: linear weights ~N(0, 1/fan_in), biases ~N(0, .02),
        the rest as BlockParams.random."""
        def w(n, k):
            return (torch.randn((n, k), generator=generator, device=device) / k ** 0.5).to(dtype)

        def b(n):
            return torch.randn(n, generator=generator, device=device) * 0.02

        p = BlockParams.random(dim, hidden, head_dim, device, generator, qk_norm, ls_init)
        qkv_w = torch.cat([w(dim, dim) for _ in range(3)])
        qkv_b = torch.cat([b(dim) for _ in range(3)])
        return BlockWeights(p, qkv_w, qkv_b, w(dim, dim), w(hidden, dim), w(dim, hidden))

    @staticmethod
    def load(weights, prefix: str, qk_norm: bool, precision, device) -> "BlockWeights":
        """``{prefix}.{norm1, attn.qkv, ...}`` from a converted checkpoint
        (model/block.rs:60-110): linear weights at ``precision``, norms,
        biases and gammas f32. The qkv projection, stored as q | k | v
        stacked on its output rows, stays one (3 dim, dim) weight (the
        reference splits it into three GEMMs to stay under wgpu's buffer
        size cap; here one fused launch computes all three)."""
        from .weights import upload_at, upload_f32

        f32t = lambda s: upload_f32(weights, f"{prefix}.{s}", device)  # noqa: E731
        gemm = lambda s: upload_at(weights, f"{prefix}.{s}", precision, device)  # noqa: E731
        dim = weights.tensor(f"{prefix}.norm1.weight").shape[0]
        qkv_w, qkv_b = gemm("attn.qkv.weight"), f32t("attn.qkv.bias")
        assert tuple(qkv_w.shape) == (3 * dim, dim), f"{prefix}: qkv weight shape"
        qn = (f32t("attn.q_norm.weight"), f32t("attn.q_norm.bias")) if qk_norm else None
        kn = (f32t("attn.k_norm.weight"), f32t("attn.k_norm.bias")) if qk_norm else None
        p = BlockParams(ln1=(f32t("norm1.weight"), f32t("norm1.bias")),
                        ln2=(f32t("norm2.weight"), f32t("norm2.bias")), qn=qn, kn=kn,
                        proj_b=f32t("attn.proj.bias"), ls1=f32t("ls1.gamma"),
                        fc1_b=f32t("mlp.fc1.bias"), fc2_b=f32t("mlp.fc2.bias"),
                        ls2=f32t("ls2.gamma"))
        return BlockWeights(p, qkv_w, qkv_b, gemm("attn.proj.weight"), gemm("mlp.fc1.weight"),
                            gemm("mlp.fc2.weight"))


def block_forward(ctx: HipContext, wts: BlockWeights, x, s: int, t: int, heads: int = HEADS,
                  rope=None, eps: float = 1e-6, fuse_ln: bool = False):
    """Block::forward (model/block.rs:118-193) with every op on HIP and the
    epilogues fused: LN1 -> the q|k|v linear with split_heads, QK-norm and
    RoPE in its epilogue -> attention written token-major -> proj +
    LayerScale + residual -> LN2 -> fc1 + GELU -> fc2 + LayerScale +
    residual. ``rope`` = (sin, cos, prefix) or None (global blocks). With
    ``fuse_ln`` each LayerNorm runs as the prologue of the product after it
    (``linear_ln_qkv_heads``, ``linear_ln_gelu``): a row-statistics pass
    replaces the LayerNorm pass and the normalised rows never reach memory.
    The result is bit-identical either way; the LayerNorm pass is the
    default because it is faster (every 256-column tile of the product
    normalises the same x rows again, 12-16 times the pass's arithmetic).
    Returns the block output (S*T, dim)."""
    p = wts.p
    if fuse_ln:
        q, k, v = ctx.linear_ln_qkv_heads(x, p.ln1, wts.qkv_w, wts.qkv_b, s, t, heads, qn=p.qn,
                                          kn=p.kn, rope=rope, eps=eps)
    else:
        normed = ctx.layernorm(x, *p.ln1, eps=eps)
        q, k, v = ctx.linear_qkv_heads(normed, wts.qkv_w, wts.qkv_b, s, t, heads, qn=p.qn,
                                       kn=p.kn, rope=rope, eps=eps)
    attn = ctx.attention_merged(q, k, v)
    x1 = ctx.linear_ls_residual(attn, wts.proj_w, p.ls1, x, p.proj_b)
    if fuse_ln:
        act = ctx.linear_ln_gelu(x1, p.ln2, wts.fc1_w, p.fc1_b, eps=eps)
    else:
        normed2 = ctx.layernorm(x1, *p.ln2, eps=eps)
        act = ctx.linear_gelu(normed2, wts.fc1_w, p.fc1_b)
    return ctx.linear_ls_residual(act, wts.fc2_w, p.ls2, x1, p.fc2_b)


def block_forward_reference(ctx: HipContext, wts: BlockWeights, x, s: int, t: int,
                            heads: int = HEADS, rope=None, eps: float = 1e-6):
    """The reference's unfused dispatch sequence (model/block.rs:118-193)
    through the same library's single ops: linear (with bias) -> split_heads
    -> layernorm(q|k) -> rope_apply -> attention -> attn_merge -> linear ->
    residual_ls -> layernorm -> linear -> gelu -> linear -> residual_ls."""
    p = wts.p
    dim = x.shape[-1]
    hd = dim // heads
    normed = ctx.layernorm(x, *p.ln1, eps=eps)
    q, k, v = (ctx.split_heads(ctx.linear(normed, w_, b_), s, t, heads, hd)
               for w_, b_ in ((wts.q_w, wts.q_b), (wts.k_w, wts.k_b), (wts.v_w, wts.v_b)))
    if p.qn is not None:
        q = ctx.layernorm(q, *p.qn, eps=eps)
        k = ctx.layernorm(k, *p.kn, eps=eps)
    if rope is not None:
        ctx.rope_apply(q, *rope)
        ctx.rope_apply(k, *rope)
    merged = ctx.attn_merge(ctx.attention(q, k, v))
    x1 = ctx.residual_ls(x, ctx.linear(merged, wts.proj_w, p.proj_b), p.ls1)
    normed2 = ctx.layernorm(x1, *p.ln2, eps=eps)
    mlp = ctx.linear(ctx.gelu(ctx.linear(normed2, wts.fc1_w, p.fc1_b)), wts.fc2_w, p.fc2_b)
    return ctx.residual_ls(x1, mlp, p.ls2)
