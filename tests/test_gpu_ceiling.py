"""bench.py's data-movement probes (bench_ceiling.hip) move what they claim:
each is checked exactly against torch on a small shape under both load/store
policies and every launch shape, so a ceiling the bench reports is the rate
of a kernel that did the op's data movement."""
import os

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu
# shapes: bit 0 cached (else streaming); 0-1 four vectors per lane (heads:
# two whole rows per wave), 2-3 one (heads: one token's 8-head chunk per
# wave), 4-5 two, 6-7 eight
POLICIES = list(range(8))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(bench.CEILING_LIB), "bench_ceiling.so not built"
    return bench.load_ceiling()


def _run(lib, kind, temporal, a, b, o, o2, n, s, t):
    ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    for out in (o, o2):
        if out is not None:
            out.zero_()
    rc = lib.hsc_run(bench.KINDS[kind], temporal, ptr(a), ptr(b), ptr(o), ptr(o2), n, s, t,
                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0


@pytest.mark.parametrize("temporal", POLICIES)
@pytest.mark.parametrize("rows", [1, 37, 1374])
def test_copy_and_add2(lib, rows, temporal):
    g = torch.Generator(device="cuda").manual_seed(rows)
    a = torch.randint(-2**31, 2**31 - 1, (rows, 512), device="cuda", dtype=torch.int32, generator=g)
    b = torch.randint(-2**31, 2**31 - 1, (rows, 512), device="cuda", dtype=torch.int32, generator=g)
    o = torch.empty_like(a)
    n = a.numel() // 4
    _run(lib, "copy", temporal, a, None, o, None, n, 0, 0)
    assert torch.equal(o, a)
    _run(lib, "add2", temporal, a, b, o, None, n, 0, 0)
    want = (a.to(torch.int64) + b.to(torch.int64)) & 0xFFFFFFFF
    want = torch.where(want >= 2**31, want - 2**32, want).to(torch.int32)
    assert torch.equal(o, want)


@pytest.mark.parametrize("temporal", POLICIES)
@pytest.mark.parametrize("s,t", [(1, 1), (2, 11), (3, 1374)])
def test_heads_is_the_head_split(lib, s, t, temporal):
    g = torch.Generator(device="cuda").manual_seed(t)
    q = torch.randn((s * t, 1024), device="cuda", generator=g).half()
    k = torch.randn((s * t, 1024), device="cuda", generator=g).half()
    oq, ok = torch.empty_like(q), torch.empty_like(k)
    _run(lib, "heads", temporal, q, k, oq, ok, 0, s, t)
    split = lambda x: x.view(s, t, 16, 64).permute(0, 2, 1, 3).contiguous().view(-1, 1024)  # noqa: E731
    assert torch.equal(oq, split(q)) and torch.equal(ok, split(k))


@pytest.mark.parametrize("temporal", POLICIES)
@pytest.mark.parametrize("n", [4, 1024 * 37, 1369 * 1024 * 2])
def test_cast(lib, n, temporal):
    g = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn(n, device="cuda", generator=g) * 100
    o = torch.empty(n, device="cuda", dtype=torch.float16)
    _run(lib, "cast", temporal, x, None, o, None, n, 0, 0)
    assert torch.equal(o, x.half())


@pytest.mark.parametrize("temporal", POLICIES)
@pytest.mark.parametrize("n", [8, 1024 * 37, 1374 * 2048])
def test_widen_and_inplace(lib, n, temporal):
    g = torch.Generator(device="cuda").manual_seed(n)
    x = (torch.randn(n, device="cuda", generator=g) * 100).half()
    o = torch.empty(n, device="cuda", dtype=torch.float32)
    _run(lib, "widen", temporal, x, None, o, None, n // 8, 0, 0)
    assert torch.equal(o, x.float())
    a = torch.randint(-2**31, 2**31 - 1, (n // 4, 4), device="cuda", dtype=torch.int32, generator=g)
    want = (a.to(torch.int64) + 1) & 0xFFFFFFFF
    want = torch.where(want >= 2**31, want - 2**32, want).to(torch.int32)
    rc = lib.hsc_run(bench.KINDS["inplace"], temporal, None, None, a.data_ptr(), None, n // 4, 0,
                     0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(a, want)


def test_kernel_event_times_what_torch_events_time():
    """bench.KernelEvent (no system-scope release at record) measures the
    same interval as torch's default events around a fixed-length GPU
    busy-wait: within the ~2 us the default events' cache flush adds."""
    torch.cuda.synchronize()
    pairs = {"kernel": (bench.KernelEvent(), bench.KernelEvent()),
             "torch": (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))}
    ms = {}
    for name, (a, b) in pairs.items():
        torch.cuda._sleep(1_000_000)  # untimed: the timed wait follows other work
        a.record()
        torch.cuda._sleep(5_000_000)
        b.record()
        torch.cuda.synchronize()
        ms[name] = a.elapsed_time(b)
    assert ms["kernel"] > 0.5, ms  # a ~5 M-cycle wait is milliseconds long
    assert abs(ms["kernel"] - ms["torch"]) < 0.01 + 0.05 * ms["torch"], ms


def test_clock_sampler(lib):
    """hsc_clock's samples: the real-time counter advances by at least the
    step between samples, the shader-clock counter advances too, and the
    clock they imply lies between 0.3 and 5 GHz; bad arguments are refused."""
    n, step = 64, 200  # 2 us apart
    buf = torch.zeros(2 * n, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert lib.hsc_clock(buf.data_ptr(), n, step, st) == 0
    torch.cuda.synchronize()
    s = buf.cpu().view(-1, 2).tolist()
    for (c0, r0), (c1, r1) in zip(s, s[1:]):
        assert r1 - r0 >= step and c1 > c0
    mhz = (s[-1][0] - s[0][0]) / ((s[-1][1] - s[0][1]) / 100.0)
    assert 300 < mhz < 5000, mhz
    assert lib.hsc_clock(buf.data_ptr(), 0, step, st) == -1
    assert lib.hsc_clock(buf.data_ptr(), 1, -1, st) == -1
    assert lib.hsc_clock(None, 1, 0, st) == -1


def test_gelu_in_pass_probe(ctx):
    """bench.gelu_in_pass_probe_us swaps the copy probe in for every bias +
    GELU of a pass, times it, and leaves the pass's own launch sequence in
    place."""
    b = bench.Pass(ctx, 2, torch.float16, distinct=True)
    seq = b.seq
    us = bench.gelu_in_pass_probe_us(b, 1)
    assert us is not None and 0 < us < 1e4
    assert b.seq is seq
    b.run()
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind", ["gelu", "matrix"])
def test_clock_trace_runs(ctx, capsys, kind):
    """bench.py --clock-trace at a small S: one JSON line with every phase,
    its launch times and a shader clock between 0.3 and 5 GHz."""
    import json

    bench.clock_trace(kind, 2)
    line = capsys.readouterr().out.strip().splitlines()[-1]
    d = json.loads(line)
    assert d["clock_trace"] == kind and d["frames"] == 2
    assert len(d["phases"]) == (3 if kind == "gelu" else 4)
    for p in d["phases"]:
        assert len(p["launch_us"]) == p["launches"] and min(p["launch_us"]) > 0
        assert p["end_ms"] >= p["start_ms"]
    mhz = [m for _, m in d["clock_mhz_per_0.5ms"]]
    assert mhz and 300 < min(mhz) and max(mhz) < 5000
