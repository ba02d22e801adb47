"""The aggregator trunk on HIP (crates/headshot-server/src/model/trunk.rs).

``Trunk.load`` reads the trunk's parameters from a converted checkpoint
(trunk.rs:28-47): camera and register tokens at the engine precision, the
RoPE periods, and ``depth`` frame / inter-frame block pairs with QK-norm.
``Trunk.forward`` runs DINO patch tokens through it (trunk.rs:49-146):

- token assembly per frame, ``[camera[v], register[v] x 16, patches]`` with
  v = 0 for frame 0 and 1 otherwise, the f32 patches rounded to the trunk's
  precision on the way (one ``hs_assemble_tokens`` launch);
- per layer k, a frame block (S sequences of T tokens, RoPE on the patch
  tokens), then an inter-frame block: at the register-attention layers over
  the 17 prefix tokens of every frame, gathered into one sequence and
  scattered back (``hs_copy_row_blocks``, one launch each way); at the
  others over all N*T tokens as one sequence, without RoPE;
- at the cached layers, the head-input cache: the frame- and inter-block
  outputs concatenated channel-wise and widened to f32 (``hs_cache_build``).

Every block runs ``block_forward`` (linears with fused epilogues, fused
QK-norm + RoPE, matrix-core attention written token-major). With
``fused=False`` the same trunk runs the reference's dispatch sequence
through this library's single ops instead (``block_forward_reference``,
one ``copy_rows`` per frame, concat then cast), the comparison path of the
parity tests.
"""
from __future__ import annotations

import torch

from . import rope as _rope
from .aggregator import BlockWeights, block_forward, block_forward_reference
from .context import HipContext

PREFIX = 17   # 1 camera + 16 register tokens per frame (trunk.rs:15)
N_REG = 16
DIM = 1024    # trunk.rs:16
HEADS = 16    # trunk.rs:33
EPS = 1e-5    # the reference LayerNorm's eps (engine/ops.rs:139)
REGISTER_ATTENTION_LAYERS = (2, 6, 9, 14, 20)  # crates/headshot-shared/src/model.rs:25
CACHED_LAYERS = (4, 11, 17, 23)                 # crates/headshot-shared/src/model.rs:28


class Trunk:
    def __init__(self, camera_token, register_token, frame_blocks, inter_blocks, periods,
                 precision):
        self.camera_token = camera_token      # (2, DIM): variant 0 = frame 0, 1 = the rest
        self.register_token = register_token  # (2 * 16, DIM)
        self.frame_blocks = frame_blocks
        self.inter_blocks = inter_blocks
        self.periods = periods                # (16,) f32, host
        self.precision = precision

    @property
    def depth(self) -> int:
        return len(self.frame_blocks)

    @staticmethod
    def load(weights, precision, device, depth: int = 24) -> "Trunk":
        """trunk.rs:28-47. ``depth`` < 24 loads the first block pairs only
        (a partial checkpoint, e.g. in tests)."""
        from .weights import read_f32, upload_at

        def blocks(name):
            return [BlockWeights.load(weights, f"aggregator.{name}.{i}", True, precision, device)
                    for i in range(depth)]

        cam = upload_at(weights, "aggregator.camera_token", precision, device).reshape(2, DIM)
        reg = upload_at(weights, "aggregator.register_token", precision, device)
        return Trunk(cam, reg.reshape(2 * N_REG, DIM), blocks("frame_blocks"),
                     blocks("inter_frame_blocks"), read_f32(weights, "aggregator.rope_embed.periods"),
                     precision)

    def forward(self, ctx: HipContext, dino_tokens, n: int, h_p: int, w_p: int, tap=None,
                fused: bool = True) -> list:
        """dino_tokens (N*P, 1024) f32 -> the head-input caches, each
        (N*T, 2048) f32, T = P + 17 (trunk.rs:49-146). ``tap(name, tensor)``
        sees "trunk.frame.NN" (N*T, 1024), "trunk.inter.NN" (N*T rows, or
        N*17 at the register layers) and "cache.NN"."""
        p = h_p * w_p
        assert dino_tokens.numel() == n * p * DIM, "dino tokens shape"
        assert dino_tokens.dtype == torch.float32, "DINO emits f32 tokens"
        t = p + PREFIX
        prec = self.precision
        note = tap or (lambda name, x: None)
        if fused:
            x = ctx.assemble_tokens(dino_tokens, n, p, self.camera_token, self.register_token,
                                    out_dtype=prec)
        else:
            toks = ctx.cast_to_f16(dino_tokens) if prec == torch.float16 else dino_tokens
            x = ctx.empty_typed((n * t, DIM), prec)
            for i in range(n):
                v = int(i != 0)
                ctx.copy_rows(self.camera_token, v, x, i * t, 1)
                ctx.copy_rows(self.register_token, v * N_REG, x, i * t + 1, N_REG)
                ctx.copy_rows(toks, i * p, x, i * t + PREFIX, p)

        sin, cos = (torch.from_numpy(a).to(ctx.device) for a in _rope.tables(self.periods, h_p, w_p))
        block = block_forward if fused else block_forward_reference
        caches = []
        for k in range(self.depth):
            frame_out = block(ctx, self.frame_blocks[k], x, n, t, HEADS, rope=(sin, cos, PREFIX),
                              eps=EPS)
            note(f"trunk.frame.{k:02}", frame_out)
            if k in REGISTER_ATTENTION_LAYERS:
                reg = ctx.empty_typed((n * PREFIX, DIM), prec)
                if fused:
                    ctx.copy_row_blocks(frame_out, 0, t, reg, 0, PREFIX, n, PREFIX)
                else:
                    for i in range(n):
                        ctx.copy_rows(frame_out, i * t, reg, i * PREFIX, PREFIX)
                reg_out = block(ctx, self.inter_blocks[k], reg, 1, n * PREFIX, HEADS, rope=None,
                                eps=EPS)
                note(f"trunk.inter.{k:02}", reg_out)
                if fused:
                    ctx.copy_row_blocks(reg_out, 0, PREFIX, frame_out, 0, t, n, PREFIX)
                else:
                    for i in range(n):
                        ctx.copy_rows(reg_out, i * PREFIX, frame_out, i * t, PREFIX)
                x = frame_out
            else:
                inter_out = block(ctx, self.inter_blocks[k], frame_out, 1, n * t, HEADS,
                                  rope=None, eps=EPS)
                note(f"trunk.inter.{k:02}", inter_out)
                if k in CACHED_LAYERS:
                    if fused:
                        cache = ctx.cache_build(frame_out, inter_out)
                    else:
                        cat = ctx.concat_channels(frame_out, inter_out)
                        cache = ctx.cast_to_f32(cat) if prec == torch.float16 else cat
                    note(f"cache.{k:02}", cache)
                    caches.append(cache)
                x = inter_out
        return caches
