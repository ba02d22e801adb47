"""hs_linear_ln_gelu_noalloc (the allocation-free variant of
hs_linear_ln_gelu, row statistics in the library's per-device array)
through the C ABI against hs_linear_ln_gelu with a caller workspace: the
same kernels on the same statistics, so the outputs are bit-identical. Two
calls in a row, the second on fewer rows (the array keeps the first call's
statistics), in f16 and f32; rows beyond the array's capacity are refused
before anything runs."""
import numpy as np
import pytest
import torch

from headshot_amd import _lib

pytestmark = pytest.mark.gpu


def operands(seed, m, n, k, dtype):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn((m, k), generator=g) + 0.25).to(dtype).to("cuda:0")
    ln_w = (1 + 0.02 * torch.randn(k, generator=g)).to("cuda:0")
    ln_b = (0.02 * torch.randn(k, generator=g)).to("cuda:0")
    w = (torch.randn((n, k), generator=g) / k ** 0.5).to(dtype).to("cuda:0")
    b = (0.02 * torch.randn(n, generator=g)).to("cuda:0")
    return x, ln_w, ln_b, w, b


@pytest.mark.parametrize("dtype,n,k", [(torch.float16, 512, 1024), (torch.float32, 96, 80)])
def test_noalloc_matches_workspace_entry(ctx, dtype, n, k):
    L = _lib.load()
    dt = _lib.HS_F16 if dtype == torch.float16 else _lib.HS_F32
    stream = torch.cuda.current_stream().cuda_stream
    for call, m in enumerate((2 * 1374, 300)):  # the second call is smaller
        print(f"[noalloc {dtype} n={n} k={k} call {call} m={m}]", flush=True)
        x, ln_w, ln_b, w, b = operands(100 * call + n, m, n, k, dtype)
        f = ctx.fold_layernorm(w, b, ln_w, ln_b)
        want = ctx.linear_ln_gelu(x, f, eps=1e-6)
        got = torch.full_like(want, float("nan"))
        rc = L.hs_linear_ln_gelu_noalloc(stream, dt, x.data_ptr(), f.w_fold.data_ptr(),
                                         f.colsum.data_ptr(), f.shift.data_ptr(), got.data_ptr(),
                                         m, n, k, 1e-6)
        assert rc == _lib.HS_OK, L.hs_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16 if dtype == torch.float16 else torch.int32),
                           want.view(torch.int16 if dtype == torch.float16 else torch.int32)), \
            f"call {call}: {(got != want).sum().item()} values differ"


def test_noalloc_refuses_more_rows_than_the_array_holds(ctx):
    L = _lib.load()
    x, ln_w, ln_b, w, b = operands(7, 4, 256, 64, torch.float16)
    f = ctx.fold_layernorm(w, b, ln_w, ln_b)
    out = torch.empty((4, 256), dtype=torch.float16, device="cuda:0")
    rc = L.hs_linear_ln_gelu_noalloc(torch.cuda.current_stream().cuda_stream, _lib.HS_F16,
                                     x.data_ptr(), f.w_fold.data_ptr(), f.colsum.data_ptr(),
                                     f.shift.data_ptr(), out.data_ptr(), (1 << 19) + 1, 256, 64,
                                     1e-6)
    assert rc == _lib.HS_EINVAL
    assert "exceeds" in L.hs_last_error().decode()
