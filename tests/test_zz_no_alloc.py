"""hs_linear_ln_gelu_noalloc (the allocation-free variant of
hs_linear_ln_gelu, row statistics in the library's per-device array)
through the C ABI against hs_linear_ln_gelu with a caller workspace: the
same kernels on the same statistics, so the outputs are bit-identical.

- two calls in a row, the second on fewer rows (the array keeps the first
  call's statistics), in f16 and f32;
- rows beyond the array's capacity are refused before anything runs;
- the call captured into a HIP graph (the use it exists for) and replayed
  with other work between the replays, each replay bit-identical to the
  eager result, device memory unchanged around eager calls and replays;
- the first call of a fresh process, before any other launch of the
  library (the array's device address is taken then), in a child process.
"""
import os
import subprocess
import sys

import pytest
import torch

from headshot_amd import _lib

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def operands(seed, m, n, k, dtype):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn((m, k), generator=g) + 0.25).to(dtype).to("cuda:0")
    ln_w = (1 + 0.02 * torch.randn(k, generator=g)).to("cuda:0")
    ln_b = (0.02 * torch.randn(k, generator=g)).to("cuda:0")
    w = (torch.randn((n, k), generator=g) / k ** 0.5).to(dtype).to("cuda:0")
    b = (0.02 * torch.randn(n, generator=g)).to("cuda:0")
    return x, ln_w, ln_b, w, b


def noalloc(x, ln_w, ln_b, w, b, out, eps=1e-6):
    L = _lib.load()
    m, k = x.shape
    n = w.shape[0]
    dt = _lib.HS_F16 if x.dtype == torch.float16 else _lib.HS_F32
    rc = L.hs_linear_ln_gelu_noalloc(torch.cuda.current_stream().cuda_stream, dt, x.data_ptr(),
                                     ln_w.data_ptr(), ln_b.data_ptr(), w.data_ptr(), b.data_ptr(),
                                     out.data_ptr(), m, n, k, eps)
    assert rc == _lib.HS_OK, L.hs_last_error().decode()


def same_bits(a, b):
    iv = torch.int16 if a.dtype == torch.float16 else torch.int32
    return torch.equal(a.view(iv), b.view(iv))


@pytest.mark.parametrize("dtype,n,k", [(torch.float16, 512, 1024), (torch.float32, 96, 80)])
def test_noalloc_matches_workspace_entry(ctx, dtype, n, k):
    for call, m in enumerate((2 * 1374, 300)):  # the second call is smaller
        print(f"[noalloc {dtype} n={n} k={k} call {call} m={m}]", flush=True)
        x, ln_w, ln_b, w, b = operands(100 * call + n, m, n, k, dtype)
        want = ctx.linear_ln_gelu(x, (ln_w, ln_b), w, b, eps=1e-6)
        got = torch.full_like(want, float("nan"))
        noalloc(x, ln_w, ln_b, w, b, got)
        torch.cuda.synchronize()
        assert same_bits(got, want), f"call {call}: {(got != want).sum().item()} values differ"


def test_noalloc_refuses_more_rows_than_the_array_holds(ctx):
    L = _lib.load()
    x, ln_w, ln_b, w, b = operands(7, 4, 256, 64, torch.float16)
    out = torch.empty((4, 256), dtype=torch.float16, device="cuda:0")
    rc = L.hs_linear_ln_gelu_noalloc(torch.cuda.current_stream().cuda_stream, _lib.HS_F16,
                                     x.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(), w.data_ptr(),
                                     b.data_ptr(), out.data_ptr(), (1 << 19) + 1, 256, 64, 1e-6)
    assert rc == _lib.HS_EINVAL
    assert "exceeds" in L.hs_last_error().decode()


def test_noalloc_under_graph_capture(ctx):
    """Captured into a graph and replayed four times, with an eager call on
    other rows (which overwrites the shared statistics array) and a
    synchronisation between replays: every replay equals the eager result,
    and neither the eager calls nor the replays change the device's free
    memory."""
    m, n, k = 1374, 512, 1024
    x, ln_w, ln_b, w, b = operands(31, m, n, k, torch.float16)
    x2, *_ = operands(32, 600, n, k, torch.float16)
    want = ctx.linear_ln_gelu(x, (ln_w, ln_b), w, b, eps=1e-6)
    out = torch.empty_like(want)
    other = torch.empty((600, n), dtype=torch.float16, device="cuda:0")
    noalloc(x, ln_w, ln_b, w, b, out)  # warm-up outside the capture
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    noalloc(x2, ln_w, ln_b, w, b, other)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, "an eager call changed free device memory"
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            noalloc(x, ln_w, ln_b, w, b, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    for replay in range(4):
        print(f"[noalloc graph replay {replay}]", flush=True)
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert same_bits(out, want), f"replay {replay}: {(out != want).sum().item()} values differ"
        noalloc(x2, ln_w, ln_b, w, b, other)  # eager work between the replays
        torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free1, "the replays changed free device memory"
    del graph


CHILD = r"""
import sys, torch
sys.path.insert(0, {root!r})
from headshot_amd import _lib
L = _lib.load()
g = torch.Generator(device="cpu").manual_seed(5)
m, n, k = 700, 256, 1024
x = torch.randn((m, k), generator=g).half().cuda()
ln_w = (1 + 0.02 * torch.randn(k, generator=g)).cuda()
ln_b = (0.02 * torch.randn(k, generator=g)).cuda()
w = (torch.randn((n, k), generator=g) / 32).half().cuda()
b = (0.02 * torch.randn(n, generator=g)).cuda()
got = torch.empty((m, n), dtype=torch.float16, device="cuda")
s = torch.cuda.current_stream().cuda_stream
# the library's first launch in this process
rc = L.hs_linear_ln_gelu_noalloc(s, _lib.HS_F16, x.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(),
                                 w.data_ptr(), b.data_ptr(), got.data_ptr(), m, n, k, 1e-6)
assert rc == _lib.HS_OK, L.hs_last_error().decode()
want = torch.empty_like(got)
ws = torch.empty((m, 2), dtype=torch.float32, device="cuda")
rc = L.hs_linear_ln_gelu(s, _lib.HS_F16, x.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(),
                         w.data_ptr(), b.data_ptr(), ws.data_ptr(), want.data_ptr(), m, n, k, 1e-6)
assert rc == _lib.HS_OK, L.hs_last_error().decode()
torch.cuda.synchronize()
assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "first call differs"
print("first-call ok")
"""


def test_noalloc_first_call_in_a_fresh_process(ctx):
    proc = subprocess.run([sys.executable, "-c", CHILD.format(root=ROOT)], capture_output=True,
                          text=True, timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "first-call ok" in proc.stdout
