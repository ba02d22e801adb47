"""Cache build (hs_cache_build, hs_concat_channels, hs_cast_f16_to_f32) and the
register gather/scatter (hs_copy_row_blocks) against the oracle and against
the reference's own op sequences; every result here is exact (bit-for-bit).
"""
import numpy as np
import pytest
import torch

from headshot_amd import _lib
from headshot_amd.parity import assert_bit_exact
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16]
NP = {torch.float32: np.float32, torch.float16: np.float16}


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def back(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,c1,c2", [(1, 8, 8), (37, 24, 40), (300, 1024, 1024), (19, 5, 3),
                                        (7, 0, 16), (5, 16, 0)])
def test_concat_and_cache_build(ctx, dtype, rows, c1, c2):
    rng = np.random.default_rng(rows * 100 + c1 + c2)
    a = rng.standard_normal((rows, c1)).astype(NP[dtype])
    b = rng.standard_normal((rows, c2)).astype(NP[dtype])
    got = back(ctx.concat_channels(dev(a), dev(b)))
    assert_bit_exact(got, O.concat_channels(a, b), f"concat {dtype} {(rows, c1, c2)}")
    cache = back(ctx.cache_build(dev(a), dev(b)))
    assert_bit_exact(cache, O.cache_build(a, b), f"cache_build {dtype} {(rows, c1, c2)}")


@pytest.mark.parametrize("n", [65536, 65536 - 3])
def test_cast_to_f32_every_f16(ctx, n):
    x = np.arange(65536, dtype=np.uint16)[:n].view(np.float16)
    got = back(ctx.cast_to_f32(dev(x)))
    want = O.cast_to_f32(x)
    nan = np.isnan(want)
    assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    assert np.isnan(got[nan]).all()


def test_cache_build_is_reference_sequence_full_size(ctx):
    """Cache::build at S=32 (43968 rows, 1024 + 1024 channels, f16 in): equal
    to concat_channels then cast_to_f32 (model/cache.rs:37-44), run through
    the same context, and to torch.cat(...).float()."""
    rows, c = 32 * 1374, 1024
    g = torch.Generator(device="cpu").manual_seed(3)
    fo = torch.randn((rows, c), generator=g).half().to("cuda:0")
    io = torch.randn((rows, c), generator=g).half().to("cuda:0")
    fused = ctx.cache_build(fo, io)
    seq = ctx.cast_to_f32(ctx.concat_channels(fo, io))
    torch.cuda.synchronize()
    assert torch.equal(fused, seq)
    assert torch.equal(fused, torch.cat([fo, io], dim=1).float())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,t,p,d", [(32, 1374, 17, 1024), (3, 11, 5, 64), (4, 9, 2, 3)])
def test_register_gather_scatter(ctx, dtype, n, t, p, d):
    """model/trunk.rs:103-116: gather the first p rows of every frame into
    (n*p, d), scatter them back; equal to the reference's per-frame
    copy_rows calls, and to numpy slicing."""
    rng = np.random.default_rng(n * t + p + d)
    x = rng.standard_normal((n * t, d)).astype(NP[dtype])
    gx = dev(x)
    reg = ctx.empty_typed((n * p, d), dtype)
    ctx.copy_row_blocks(gx, 0, t, reg, 0, p, n, p)
    want = x.reshape(n, t, d)[:, :p].reshape(n * p, d)
    assert_bit_exact(back(reg), want, "gather")
    reg_ref = ctx.empty_typed((n * p, d), dtype)
    for i in range(n):
        ctx.copy_rows(gx, i * t, reg_ref, i * p, p)
    assert_bit_exact(back(reg), back(reg_ref), "gather vs copy_rows")
    upd = dev((rng.standard_normal((n * p, d))).astype(NP[dtype]))
    ctx.copy_row_blocks(upd, 0, p, gx, 0, t, n, p)
    x2 = x.copy().reshape(n, t, d)
    x2[:, :p] = back(upd).reshape(n, p, d)
    assert_bit_exact(back(gx), x2.reshape(n * t, d), "scatter")


def test_copy_row_blocks_contract(ctx):
    x = torch.zeros((40, 16), device="cuda:0")
    y = torch.zeros((40, 16), device="cuda:0")
    with pytest.raises(_lib.HsContractError):  # blocks would overlap
        ctx.copy_row_blocks(x, 0, 2, y, 0, 4, 5, 3)
    with pytest.raises(_lib.HsContractError):  # src and dst overlap
        ctx.copy_row_blocks(x, 0, 4, x, 1, 4, 5, 2)
    with pytest.raises(AssertionError):  # past the end of dst
        ctx.copy_row_blocks(x, 0, 4, y, 0, 10, 5, 2)
    ctx.copy_row_blocks(x, 0, 4, y, 0, 4, 0, 2)  # nothing to do
