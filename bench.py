"""Benchmark: headshot's aggregator fused-op pass on one MI355X.

A step is one aggregator pass of the per-layer ops at S frames x 1374 tokens
x 1024 (f16 storage, f32 math): patch-token assembly, then 24 frame blocks
(QK-norm + 2D RoPE, prefix 5, 37x37 grid) and 24 global blocks (QK-norm, no
RoPE, one sequence of S*1374 tokens), each block running

    LN1 -> QK-norm(+RoPE) on q -> on k -> proj bias + LayerScale + residual
        -> LN2 -> fc1 bias + GELU (hidden 4096) -> fc2 bias + LayerScale + residual

(model/block.rs:118-159 with the GEMMs and attention out of scope: their
outputs are synthetic resident buffers). Inputs are synthetic and already in
HBM when timing starts.

Timed region: K replays of a HIP graph holding one pass (launch overhead
removed, as a serving loop would run it), bracketed by synchronisation and
HIP events. ``value`` = algorithmic bytes of the pass / pass time (GB/s).
Per-op kernel durations: every op of one more pass launched eagerly behind a
GPU busy-wait head start, with a HIP event pair around each launch on the
launch stream, averaged over ``--op-passes`` passes.

The line also carries an ``attention`` section (the same pass's attention
calls, frame and global, fused with the head merge, timed on their own and
priced against the f16 matrix-core peak), a ``cache_build`` section (the
trunk's f32 head-input cache build at the same S, against HBM) and a
``linear`` section (the block's four linear layers with their epilogues
fused, against the matrix-core peak), a ``block`` section (a whole frame
block and global block on HIP, fused, beside the reference's unfused
dispatch sequence through the same library) and a ``trunk`` section (one
whole aggregator trunk forward from DINO tokens to the head-input caches,
the same two ways).

``ceilings``: each fused op beside a data-movement probe that moves the same
bytes in the same access pattern with no arithmetic (bench_ceiling.hip:
copy, two-input add, the token-major to head-major copy of the QK-norm pair
kernel, f32 to f16 cast), warm and cold, with the op's rate as a fraction of
the probe's.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--frames S]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fused-layer-op HBM GB/s (% of peak) + ms/aggregator pass at S=32 f16"
PEAK_GBS = 8000.0  # MI355X HBM3E
DIM, HEADS, HEAD_DIM, HIDDEN = 1024, 16, 64, 4096
GRID = (37, 37)
PREFIX = 5  # 1 camera + 4 register tokens
N_REG = 4
EPS = 1e-6
N_FRAME_BLOCKS = N_GLOBAL_BLOCKS = 24
OPS = ["assemble", "layernorm", "qknorm_rope", "bias_ls_residual", "bias_gelu",
       "bias_ls_residual_layernorm"]


def op_bytes(rows: int, esz: int, n_patch_rows: int, n_pos_rows: int) -> dict:
    """Algorithmic (minimal) HBM bytes per launch of each fused op."""
    return {
        "layernorm": rows * DIM * esz * 2,                   # read x, write out
        "qknorm_rope": rows * DIM * esz * 2 * 2,             # q and k, one launch
        "bias_ls_residual": rows * DIM * esz * 3,            # read res, x; write out
        "bias_ls_residual_layernorm": rows * DIM * esz * 4,  # read res, x; write out, normed
        "bias_gelu": rows * HIDDEN * esz * 2,                # read h, write act
        "assemble": (n_patch_rows * DIM * 4                  # read f32 patches
                     + n_pos_rows * DIM * 4                  # pos-embed once
                     + rows * DIM * esz),                    # write tokens
    }


def pass_launches(n_frame: int, n_global: int, fuse: bool = False) -> dict:
    """Launches of each op in one pass (FusedOpPass's sequence): per block
    the QK-norm pair and GELU; fused, LayerScale + residual with the
    LayerNorm after it twice (the first block's LN1 and the last block's LS2
    alone), unfused, two LayerNorms and two LayerScale + residual."""
    n = n_frame + n_global
    if fuse:
        return {"assemble": 1, "layernorm": 1, "qknorm_rope": n, "bias_gelu": n,
                "bias_ls_residual_layernorm": 2 * n - 1, "bias_ls_residual": 1}
    return {"assemble": 1, "layernorm": 2 * n, "qknorm_rope": n, "bias_gelu": n,
            "bias_ls_residual": 2 * n}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--frames", type=int, default=32)
    ap.add_argument("--dtype", choices=["f16", "f32"], default="f16")
    ap.add_argument("--op-passes", type=int, default=3)
    ap.add_argument("--fuse-layernorm", action="store_true",
                    help="time the four-op block sequence (each LayerScale + residual fused with "
                         "the LayerNorm after it) as the headline pass")
    ap.add_argument("--shared-inputs", action="store_true",
                    help="all blocks read one set of raw GEMM outputs (default: each its own)")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the other workloads' legs (S=2, 8, 200, 16 at 21x37)")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the data-movement probes timed beside each op")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target CPU work for the oracle baseline sample")
    ap.add_argument("--calibrate-copy-mib", type=int, default=512,
                    help="size of one plain torch copy launched before timing (HBM counter "
                         "calibration for rocprofv3 --pmc runs)")
    ap.add_argument("--attention-iters", type=int, default=10,
                    help="timed launches of each attention shape (0 skips the attention, "
                         "cache, linear, block and trunk legs)")
    ap.add_argument("--trunk-iters", type=int, default=-1,
                    help="timed trunk forwards (default attention-iters // 5, at least 1; "
                         "0 skips the trunk leg)")
    ap.add_argument("--summarize", metavar="KERNEL_TRACE_CSV",
                    help="print a summary of rocprofv3 output for this benchmark instead of "
                         "running it")
    ap.add_argument("--legs-trace", metavar="KERNEL_TRACE_CSV",
                    help="kernel trace of a run with the attention/cache/linear legs (default: "
                         "the --summarize trace)")
    ap.add_argument("--pmc-fetch", metavar="CSV", help="counter_collection CSV of a FETCH_SIZE run")
    ap.add_argument("--pmc-write", metavar="CSV", help="counter_collection CSV of a WRITE_SIZE run")
    ap.add_argument("--traffic-json", metavar="PATH", help="write per-op HBM bytes here")
    ap.add_argument("--summarize-counters", metavar="CSV", nargs="+",
                    help="print derived shader-counter ratios (matrix-core and LDS use) per "
                         "kernel from rocprofv3 --pmc counter_collection CSVs of this benchmark")
    ap.add_argument("--counter-pair", action="store_true",
                    help="launch bias + GELU at this S (rows x 4096 f16) and its copy probe 8 "
                         "times each over rotating buffers, then exit (for rocprofv3 --pmc)")
    ap.add_argument("--clock-trace", choices=["gelu", "pass", "matrix"],
                    help="sample the shader clock (a one-wave sampler on a second stream) "
                         "during 16 bias + GELU launches at this S, 16 of its copy probe and 16 "
                         "GELU again (gelu), during 18 replays of the pass (pass), or during "
                         "this S's global and frame attention and fc1 with and without its GELU "
                         "(matrix); print per-launch times and the clock per phase, then exit")
    ap.add_argument("--summarize-pair", metavar="CSV", nargs="+",
                    help="print each counter's mean per dispatch for bias + GELU and its copy "
                         "probe, and their ratio, from --counter-pair counter_collection CSVs")
    return ap.parse_args()


class Pass:
    """One aggregator fused-op pass (headshot_amd.aggregator.FusedOpPass)
    plus its algorithmic byte counts. ``distinct``: each block reads raw
    GEMM outputs of its own (48 x 720 MB at S=32)."""

    def __init__(self, ctx, frames: int, dtype, grid=GRID, n_frame: int = N_FRAME_BLOCKS,
                 n_global: int = N_GLOBAL_BLOCKS, distinct: bool = True, fuse: bool = False):
        import torch

        from headshot_amd.aggregator import FusedOpPass

        self.fp = fp = FusedOpPass(ctx, frames, grid=grid, n_reg=N_REG, n_frame=n_frame,
                                   n_global=n_global, dtype=dtype, eps=EPS,
                                   distinct_inputs=distinct, fuse=fuse)
        self.ctx, self.frames, self.dtype = ctx, frames, dtype
        self.p, self.t, self.rows = fp.p, fp.t, fp.rows
        self.seq = fp.seq
        esz = 2 if dtype == torch.float16 else 4
        self.bytes = op_bytes(self.rows, esz, frames * fp.p, fp.p)
        self.launches = fp.launches()
        assert self.launches == pass_launches(n_frame, n_global, fuse), "launch sequence"
        self.ops = [op for op in OPS if op in self.launches]
        self.pass_bytes = sum(self.bytes[k] * self.launches[k] for k in self.ops)

    def run(self):
        self.fp.run()


class KernelEvent:
    """A HIP timing event recorded without the system-scope release
    (hipEventCreateWithFlags with hipEventDisableSystemFence), with
    torch.cuda.Event's record/elapsed_time surface, on torch's current
    stream. A default event's record releases to system scope, writing back
    and invalidating the GPU caches: between two back-to-back kernels that
    adds ~1.7 us to every event pair (S=32 pass: the ops' event durations
    fall from 48.4 / 30.8 / 63.8 / 42.4 / 122.3 us to 46.5 / 29.1 / 62.2 /
    40.7 / 120.7 us, against 45.8 / 28.7 / 61.4 / 39.8 / 120.8 in the kernel
    trace) and empties the L2 that the next kernel would otherwise find as
    the graph-replayed pass leaves it. The HIP runtime is the one torch
    loaded (same soname, so the same handle)."""

    _hip = None

    def __init__(self):
        import ctypes

        if KernelEvent._hip is None:
            hip = ctypes.CDLL("libamdhip64.so.7")
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            KernelEvent._hip = hip
        self._ev = ctypes.c_void_p()
        rc = self._hip.hipEventCreateWithFlags(ctypes.byref(self._ev), 0x20000000)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags returned {rc}")

    def record(self):
        import ctypes

        import torch

        rc = self._hip.hipEventRecord(self._ev, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord returned {rc}")

    def elapsed_time(self, end: "KernelEvent") -> float:
        import ctypes

        ms = ctypes.c_float()
        rc = self._hip.hipEventElapsedTime(ctypes.byref(ms), self._ev, end._ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime returned {rc}")
        return ms.value

    def __del__(self):
        try:
            if self._hip is not None and self._ev:
                self._hip.hipEventDestroy(self._ev)
        except Exception:  # interpreter shutdown: the runtime may be gone
            pass


def per_op_times(bench: Pass, passes: int, flush=None) -> dict:
    """Mean kernel duration per op (ms) from event pairs on the launch
    stream (KernelEvent: no cache flush at each record). A GPU busy-wait
    ahead of each pass lets the host enqueue the whole pass first, so the
    kernels run back to back as in the timed loop. One untimed pass runs
    between the busy-wait and the timed one: the first
    kernel after the wait runs slower (the assembly at S=32: 52.1 us against
    49.4 us back to back), and in the timed loop every op, the assembly
    included, follows other work.

    ``flush`` (a callable enqueueing GPU work) runs untimed before every
    timed launch: with a read of more than the last-level caches hold, no
    input of the timed op is cache-resident (cold timing)."""
    import torch

    pairs = [(KernelEvent(), KernelEvent()) for _ in bench.seq]
    sums = {op: 0.0 for op in bench.ops}
    counts = {op: 0 for op in bench.ops}
    for _ in range(passes):
        torch.cuda.synchronize()
        torch.cuda._sleep(100_000_000)  # ~40 ms head start
        for _, thunk in bench.seq:
            thunk()
        for (op, thunk), (a, b) in zip(bench.seq, pairs):
            if flush is not None:
                flush()
            a.record()
            thunk()
            b.record()
        torch.cuda.synchronize()
        for (op, _), (a, b) in zip(bench.seq, pairs):
            sums[op] += a.elapsed_time(b)
            counts[op] += 1
    return {op: sums[op] / counts[op] for op in bench.ops}


FLUSH_BYTES = 1 << 30  # > the 256 MB Infinity Cache + 8 x 4 MB L2


def cache_flusher(device):
    """A read-only sweep of FLUSH_BYTES: torch.sum over a resident f32 buffer
    (reads it once, writes one value), so the caches hold only clean lines
    of that buffer afterwards."""
    import torch

    buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=device)
    acc = torch.empty((), dtype=torch.float32, device=device)

    def flush():
        torch.sum(buf, dim=0, out=acc)

    return flush


def op_rates(bench: Pass, mean_ms: dict) -> dict:
    per_op = {}
    for op in bench.ops:
        us = mean_ms[op] * 1e3
        gbs = bench.bytes[op] / (us * 1e-6) / 1e9
        per_op[op] = {"us": round(us, 2), "GB/s": round(gbs, 1),
                      "frac": round(gbs / PEAK_GBS, 4), "bytes": bench.bytes[op],
                      "launches_per_pass": bench.launches[op]}
    return per_op


def sequence_pass(ctx, frames: int, dtype, distinct: bool, steps: int, fuse: bool) -> dict:
    """The same pass with the other op sequence (fuse False: LayerScale +
    residual and LayerNorm as separate launches, six per block), replayed
    from a HIP graph like the headline: ms, its own algorithmic bytes, GB/s."""
    import torch

    b = Pass(ctx, frames, dtype, distinct=distinct, fuse=fuse)
    b.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        b.run()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    gbs = b.pass_bytes / (ms * 1e-3) / 1e9
    out = {"fused_layernorm": fuse, "launches": sum(b.launches.values()), "ms": round(ms, 3),
           "pass_bytes": b.pass_bytes, "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
    del graph, b
    torch.cuda.empty_cache()
    return out


def pass_from_ops(bench: Pass, per_op: dict) -> dict:
    """The pass rate that the per-op kernel times imply: pass bytes / the sum
    of each op's mean duration x its launches (with cold per-op times: every
    launch finding none of its inputs in a cache)."""
    ms = sum(per_op[op]["us"] * bench.launches[op] for op in bench.ops) / 1e3
    gbs = bench.pass_bytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}


# The op sequence's other workloads, each timed like the headline pass:
# key -> (frames, (patch rows, patch columns), storage, frame blocks, global
# blocks). A frame block runs S sequences of T tokens with RoPE; a global
# block one sequence of S*T tokens without.
WORKLOADS = {
    "s2_f32_frame_global": (2, (37, 37), "f32", 1, 1),
    "s8_f16_frame": (8, (37, 37), "f16", 1, 0),
    "s200_f16_global": (200, (37, 37), "f16", 0, 1),
    "s200_f16_frame": (200, (37, 37), "f16", 1, 0),
    "s16_21x37_f32_frame_global": (16, (21, 37), "f32", 1, 1),
    "s16_21x37_f16_frame_global": (16, (21, 37), "f16", 1, 1),
}


def workload_legs(ctx, op_passes: int, flush, min_launches: int = 64, replays: int = 10) -> dict:
    """Each workload's sequence (assembly, then its blocks' fused ops, every
    block with raw GEMM outputs of its own) captured in a HIP graph,
    repeated until the graph holds at least ``min_launches`` launches (so a
    few short kernels are not timed against one graph launch), replayed
    ``replays`` times: ms per sequence, GB/s of its algorithmic bytes,
    tokens/s (S*T tokens per sequence); and each op's kernel time warm and
    cold (event pairs, as the headline's ``ops``)."""
    import torch

    def replayed_ms(b):
        reps = max(1, -(-min_launches // len(b.fp.seq)))
        b.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                b.run()
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(replays):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        del graph
        return start.elapsed_time(end) / (replays * reps), reps

    out = {}
    for key, (frames, grid, dt, nf, ng) in WORKLOADS.items():
        dtype = torch.float16 if dt == "f16" else torch.float32
        b = Pass(ctx, frames, dtype, grid=grid, n_frame=nf, n_global=ng, distinct=True)
        ms, reps = replayed_ms(b)
        gbs = b.pass_bytes / (ms * 1e-3) / 1e9
        warm = op_rates(b, per_op_times(b, op_passes))
        cold = op_rates(b, per_op_times(b, op_passes, flush=flush))
        out[key] = {"frames": frames, "tokens_per_frame": b.t, "grid": f"{grid[0]}x{grid[1]}",
                    "dtype": dt, "frame_blocks": nf, "global_blocks": ng, "rows": b.rows,
                    "ms_per_sequence": round(ms, 4), "bytes_per_sequence": b.pass_bytes,
                    "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                    "tokens_per_s": round(b.rows / (ms * 1e-3), 1),
                    "pass_cold": pass_from_ops(b, cold), "ops": warm, "ops_cold": cold,
                    "graph_repeats": reps}
        del b
        f = Pass(ctx, frames, dtype, grid=grid, n_frame=nf, n_global=ng, distinct=True, fuse=True)
        ms_f, _ = replayed_ms(f)
        gbs_f = f.pass_bytes / (ms_f * 1e-3) / 1e9
        out[key]["fused_layernorm"] = {"ms_per_sequence": round(ms_f, 4),
                                       "bytes_per_sequence": f.pass_bytes,
                                       "GB/s": round(gbs_f, 1), "frac": round(gbs_f / PEAK_GBS, 4),
                                       "tokens_per_s": round(f.rows / (ms_f * 1e-3), 1)}
        del f
        torch.cuda.empty_cache()
    return out


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense f16 matrix peak


CEILING_SRC = os.path.join(ROOT, "bench_ceiling.hip")
CEILING_LIB = os.path.join(ROOT, "bench_ceiling.so")


def build_ceiling() -> str:
    """Compile bench_ceiling.hip (the data-movement probes) for gfx950 with
    the library's flags into bench_ceiling.so."""
    from headshot_amd import build as hs_build

    tmp = CEILING_LIB + ".tmp"
    hs_build._run([hs_build.HIPCC, *hs_build.HIP_FLAGS, "-shared", "-o", tmp, CEILING_SRC])
    os.replace(tmp, CEILING_LIB)
    return CEILING_LIB


def load_ceiling():
    import ctypes

    lib = ctypes.CDLL(CEILING_LIB)
    lib.hsc_run.restype = ctypes.c_int
    lib.hsc_run.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 4 + \
        [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.hsc_clock.restype = ctypes.c_int
    lib.hsc_clock.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    return lib


# op -> (probe kernel, what it moves)
CEILING_PROBES = {
    "layernorm": ("copy", "rows x 1024 f16 read and written, contiguous"),
    "bias_gelu": ("copy", "rows x 4096 f16 read and written, contiguous"),
    "bias_ls_residual": ("add2", "two rows x 1024 f16 read, one written, contiguous"),
    "qknorm_rope": ("heads", "q and k, rows x 1024 f16 each, token-major in, head-major out, "
                             "the pair kernel's addressing (a wave per 2 tokens, 8 heads' "
                             "128-byte vectors per store); the mean of the frame-block "
                             "layout (S frames of T) and the global-block layout (one "
                             "sequence of S*T), as the pass runs 24 of each"),
    "assemble": ("cast", "S*P x 1024 f32 read, f16 written, contiguous (positional table "
                         "and prefix rows not included)"),
    "bias_ls_residual_layernorm": ("add2w2", "two rows x 1024 f16 read, two written, "
                                             "contiguous"),
}
KINDS = {"copy": 0, "add2": 1, "heads": 2, "cast": 3, "widen": 4, "inplace": 5, "add2w2": 6}
# hsc_run shapes: bit 0 cached loads/stores (else streaming); 0-1 four 16-byte
# vectors per lane (heads: two whole rows per wave), 2-3 one (heads: one
# token's 8-head chunk per wave, chunk by chunk), 4-5 two, 6-7 eight
CEILING_SHAPES = {"streaming x4": 0, "cached x4": 1, "streaming x1": 2, "cached x1": 3,
                  "streaming x2": 4, "cached x2": 5, "streaming x8": 6, "cached x8": 7}


ROTATE_BYTES = 768 << 20  # > the 256 MB Infinity Cache: no reuse across launches


def probe_times(lib, probe: str, args, sets, flush, iters: int = 20):
    """(warm us per policy, cold us) of one probe: warm, ``iters``
    back-to-back launches rotating over the buffer ``sets`` (each set: a, b,
    o, o2 tensors or None), each policy and launch shape; cold, a cache
    flush then one launch per event pair, streaming stores only."""
    import torch

    stream = torch.cuda.current_stream().cuda_stream

    def ptrs(bufs):
        return tuple(None if x is None else x.data_ptr() for x in bufs[:4])

    def launch(shape, bufs):
        rc = lib.hsc_run(KINDS[probe], shape, *bufs, *args, stream)
        if rc != 0:
            raise RuntimeError(f"hsc_run({probe}) returned {rc}")

    warm = {}
    for policy, shape in CEILING_SHAPES.items():
        for bufs in sets:
            launch(shape, ptrs(bufs))
        torch.cuda.synchronize()
        ev = [(KernelEvent(), KernelEvent()) for _ in range(iters)]
        torch.cuda._sleep(20_000_000)  # the host enqueues ahead
        for i, (a, b) in enumerate(ev):
            a.record()
            launch(shape, ptrs(sets[i % len(sets)]))
            b.record()
        torch.cuda.synchronize()
        warm[policy] = sum(a.elapsed_time(b) for a, b in ev) / iters * 1e3
    cold = []
    for shape in (s for s in CEILING_SHAPES.values() if not s & 1):  # streaming stores only
        ev = [(KernelEvent(), KernelEvent()) for _ in range(iters)]
        for a, b in ev:
            flush()
            a.record()
            launch(shape, ptrs(sets[0]))
            b.record()
        torch.cuda.synchronize()
        cold.append(sum(a.elapsed_time(b) for a, b in ev) / iters * 1e3)
    return warm, min(cold)


def probe_entry(lib, probe: str, make_set, nbytes: int, args, flush, op_us: float,
                op_cold_us: float | None = None) -> dict:
    """A probe's warm (fastest policy) and cold rates beside an op that moves
    the same ``nbytes``: ``make_set()`` builds one buffer set; enough sets
    rotate to exceed ROTATE_BYTES."""
    sets = [make_set() for _ in range(max(1, -(-ROTATE_BYTES // nbytes)))]
    warm, cold_us = probe_times(lib, probe, args, sets, flush)
    policy = min(warm, key=warm.get)
    us = warm[policy]
    out = {"probe": probe, "bytes": nbytes, "us": round(us, 2),
           "GB/s": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / PEAK_GBS, 4),
           "policy": policy, "cold_us": round(cold_us, 2),
           "cold_frac": round(nbytes / cold_us / 1e3 / PEAK_GBS, 4),
           "op_frac_of_probe": round(us / op_us, 4)}
    if op_cold_us is not None:
        out["op_cold_frac_of_probe"] = round(cold_us / op_cold_us, 4)
    del sets
    return out


def ceiling_times(bench: Pass, op_warm: dict, op_cold: dict, flush, iters: int = 20) -> dict:
    """Each op beside a data-movement probe with its byte mix and access
    pattern (bench_ceiling.hip).

    Warm: ``iters`` back-to-back launches, an event pair around each as
    for the ops, that rotate over as many buffer sets as make ROTATE_BYTES,
    so no launch finds its inputs in a cache and each pays for its own
    write-back (streaming and cached loads/stores, each with one, two, four
    and eight 16-byte vectors per lane; the fastest is the ceiling). Compared with the op's rate inside the pass. Cold: the per-op
    cold method (cache flush, then a HIP event pair around one launch) with
    streaming stores only, the faster launch shape: cached stores leave their
    write-back for after the end event, so their cold time undercounts.
    Compared with the op's cold rate."""
    import torch

    if not os.path.exists(CEILING_LIB):
        return {"error": "bench_ceiling.so is not built (python -c 'import bench; "
                         "bench.build_ceiling()')"}
    if bench.dtype != torch.float16:
        return {"error": "the probes move f16 activations"}
    lib = load_ceiling()
    dev = bench.ctx.device
    stream = torch.cuda.current_stream(dev).cuda_stream
    rows, frames, t, p = bench.rows, bench.frames, bench.t, bench.p
    f16 = torch.float16

    def buffers(op, probe):
        """(a, b, o, o2, bytes moved, (n, s, t)) for one launch."""
        if probe in ("copy", "add2", "add2w2"):
            width = HIDDEN if op == "bias_gelu" else DIM
            a = torch.ones((rows, width), device=dev, dtype=f16)
            b = torch.ones_like(a) if probe != "copy" else None
            o2 = torch.empty_like(a) if probe == "add2w2" else None
            n = a.numel() * 2 // 16
            streams = {"copy": 2, "add2": 3, "add2w2": 4}[probe]
            return a, b, torch.empty_like(a), o2, n * 16 * streams, (n, 0, 0)
        if probe == "heads":
            a = torch.ones((rows, DIM), device=dev, dtype=f16)
            return (a, torch.ones_like(a), torch.empty_like(a), torch.empty_like(a),
                    4 * a.numel() * 2, (0, frames, t))
        a = torch.ones((frames * p, DIM), device=dev, dtype=torch.float32)
        return (a, None, torch.empty((frames * p, DIM), device=dev, dtype=f16), None,
                a.numel() * 6, (a.numel(), 0, 0))

    def timed(probe, args, sets):
        return probe_times(lib, probe, args, sets, flush, iters)

    out = {}
    for op, (probe, what) in CEILING_PROBES.items():
        if op not in bench.ops:
            continue
        first = buffers(op, probe)
        nbytes, args = first[4], first[5]
        sets = [first] + [buffers(op, probe) for _ in range(max(1, -(-ROTATE_BYTES // nbytes)) - 1)]
        warm, cold_us = timed(probe, args, sets)
        layouts = None
        if probe == "heads":
            # the pass's global blocks: one sequence of S*T tokens; each
            # layout takes its own fastest shape, as the op picks its order
            # by sequence length
            gwarm, gcold = timed(probe, (0, 1, frames * t), sets)
            fpol, gpol = min(warm, key=warm.get), min(gwarm, key=gwarm.get)
            layouts = {"frame_us": round(warm[fpol], 2), "frame_cold_us": round(cold_us, 2),
                       "frame_policy": fpol, "global_us": round(gwarm[gpol], 2),
                       "global_cold_us": round(gcold, 2), "global_policy": gpol}
            warm = {f"{fpol} / {gpol}": (warm[fpol] + gwarm[gpol]) / 2}
            cold_us = (cold_us + gcold) / 2
        policy = min(warm, key=warm.get)
        us = warm[policy]
        gbs, cold_gbs = nbytes / us / 1e3, nbytes / cold_us / 1e3
        entry = {"probe": probe, "moves": what, "bytes": nbytes, "buffer_sets": len(sets),
                 "us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                 "policy": policy,
                 "cold_us": round(cold_us, 2), "cold_GB/s": round(cold_gbs, 1),
                 "cold_frac": round(cold_gbs / PEAK_GBS, 4)}
        if layouts:
            entry["layouts"] = layouts
        if op_warm:
            entry["op_frac_of_probe"] = round(op_warm[op]["GB/s"] / gbs, 4)
        if op_cold:
            entry["op_cold_frac_of_probe"] = round(op_cold[op]["GB/s"] / cold_gbs, 4)
        out[op] = entry
        del sets, first
    torch.cuda.synchronize()
    return out


def gelu_in_pass_probe_us(bench: Pass, passes: int) -> float | None:
    """The copy probe (one 16-byte vector per lane, streaming: its fastest
    shape) launched in place of every bias + GELU of the pass, on the same
    fc1-output and activation buffers, timed as the ops are
    (per_op_times): the op's ceiling in the op's own context (after the
    same LayerNorm, before the same LayerScale), where the probe loop of
    ceiling_times runs it back to back."""
    if not os.path.exists(CEILING_LIB):
        return None
    import torch

    lib = load_ceiling()
    stream = torch.cuda.current_stream().cuda_stream
    fp, act = bench.fp, bench.fp.io.act
    esz = act.element_size()
    seq, k = [], 0
    for op, thunk in bench.seq:
        if op == "bias_gelu":
            x = fp.raws[k][3]
            k += 1

            def thunk(x=x, n16=x.numel() * esz // 16):
                rc = lib.hsc_run(KINDS["copy"], CEILING_SHAPES["streaming x1"], x.data_ptr(), None,
                                 act.data_ptr(), None, n16, 0, 0, stream)
                if rc != 0:
                    raise RuntimeError(f"hsc_run(copy) returned {rc}")
        seq.append((op, thunk))
    saved = bench.seq
    bench.seq = seq
    try:
        t = per_op_times(bench, passes)
    finally:
        bench.seq = saved
    return t["bias_gelu"] * 1e3


def attention_times(ctx, frames: int, iters: int) -> dict:
    """The aggregator's attention calls at this S, fused with the head merge
    (hs_attention_merged, as model/block.rs:148-149 consumes it): frame
    blocks run S sequences of 1374 tokens, global blocks one sequence of
    S*1374, 16 heads of 64, f16. Kernel time from HIP events on the launch
    stream; flops = 4*T^2*D per (sequence, head). For reference torch's own
    fused attention (scaled_dot_product_attention, the backend it picks on
    ROCm; head-major output, no merge; not part of this library) is timed
    beside it in alternating rounds, each figure its fastest of three."""
    import torch

    out = {}
    t = GRID[0] * GRID[1] + PREFIX
    shapes = {"frame": (frames, HEADS, t), "global": (1, HEADS, frames * t)}
    g = torch.Generator(device="cpu").manual_seed(7)
    for name, (s, h, tt) in shapes.items():
        q, k, v = (torch.randn((s, h, tt, HEAD_DIM), generator=g).to(torch.float16).to(ctx.device)
                   for _ in range(3))
        o = torch.empty((s * tt, h * HEAD_DIM), dtype=torch.float16, device=ctx.device)
        ctx.attention_merged(q, k, v, out=o)
        call = ctx.last_launch

        def timed(fn):
            fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(iters):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / iters

        best = alternating_best(
            {"hip": call,
             "library": lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v)}, timed)
        ms, ms_lib = best["hip"], best["library"]
        flops = 4.0 * tt * tt * HEAD_DIM * s * h
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"shape_SHTD": [s, h, tt, HEAD_DIM], "ms": round(ms, 3),
                     "TFLOP/s": round(tf, 1), "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                     "calls_per_pass": N_FRAME_BLOCKS if name == "frame" else N_GLOBAL_BLOCKS,
                     "library_sdpa_ms": round(ms_lib, 3),
                     "library_sdpa_TFLOP/s": round(flops / (ms_lib * 1e-3) / 1e12, 1)}
        del q, k, v, o
    out["roofline"] = {"bound": "mfma", "kernel": "flash_f16_kernel (global)",
                       "achieved": out["global"]["TFLOP/s"], "peak": MFMA_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": out["global"]["frac"]}
    out["ms_per_pass"] = round(sum(out[n]["ms"] * out[n]["calls_per_pass"]
                                   for n in ("frame", "global")), 2)
    return out


CACHED_LAYERS = 4  # trunk layers whose outputs feed the heads (model/trunk.rs:125-135)


def cold_us(fn, flush, iters: int) -> float:
    """Mean kernel time (us) of ``fn``'s launch behind a cache flush, one
    KernelEvent pair per launch."""
    import torch

    ev = [(KernelEvent(), KernelEvent()) for _ in range(iters)]
    for a, b in ev:
        flush()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in ev) / iters * 1e3


def warm_us(fn, iters: int) -> float:
    """Mean kernel time (us) of ``iters`` back-to-back launches of ``fn``,
    one KernelEvent pair around each (as the per-op pass timing), so the
    gaps between launches are not counted; the host enqueues ahead behind a
    GPU busy-wait."""
    import torch

    fn()
    torch.cuda.synchronize()
    ev = [(KernelEvent(), KernelEvent()) for _ in range(iters)]
    torch.cuda._sleep(20_000_000)  # ~8 ms head start
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in ev) / iters * 1e3


def cache_times(ctx, frames: int, iters: int, flush) -> dict:
    """Cache::build at this S (model/cache.rs:21-52): the frame- and
    inter-block outputs (S*1374, 1024) f16 each, concatenated and cast to f32
    in one pass (hs_cache_build); the reference's two-dispatch sequence
    (concat_channels, then cast_to_f32) through the same library beside it.
    Algorithmic bytes: rows * 2048 * (2 read + 4 written). Beside it the
    ``widen`` probe (f16 read, f32 written, the same bytes, no
    concatenation), warm and cold."""
    import torch

    rows = frames * (GRID[0] * GRID[1] + PREFIX)
    g = torch.Generator(device="cpu").manual_seed(11)
    fo = torch.randn((rows, DIM), generator=g).half().to(ctx.device)
    io = torch.randn((rows, DIM), generator=g).half().to(ctx.device)
    out = torch.empty((rows, 2 * DIM), dtype=torch.float32, device=ctx.device)
    nbytes = rows * 2 * DIM * (2 + 4)

    ctx.cache_build(fo, io, out=out)
    fused = ctx.last_launch
    us = warm_us(fused, iters)
    us_cold = cold_us(fused, flush, iters)
    cat = ctx.concat_channels(fo, io)
    c1 = ctx.last_launch
    cast_out = ctx.cast_to_f32(cat)  # noqa: F841 (the replayed launch writes it)
    c2 = ctx.last_launch
    us_seq = warm_us(lambda: (c1(), c2()), iters)
    gbs = nbytes / us / 1e3
    res = {"rows": rows, "channels": 2 * DIM, "us": round(us, 2), "GB/s": round(gbs, 1),
           "frac": round(gbs / PEAK_GBS, 4), "cold_us": round(us_cold, 2),
           "cold_frac": round(nbytes / us_cold / 1e3 / PEAK_GBS, 4), "bytes": nbytes,
           "reference_sequence_us": round(us_seq, 2), "calls_per_pass": CACHED_LAYERS}
    if os.path.exists(CEILING_LIB):
        n16 = rows * 2 * DIM * 2 // 16  # f16 input vectors

        def make_set():
            return (torch.ones(rows * 2 * DIM, device=ctx.device, dtype=torch.float16), None,
                    torch.empty(rows * 2 * DIM, device=ctx.device, dtype=torch.float32), None)

        res["ceiling"] = probe_entry(load_ceiling(), "widen", make_set, nbytes, (n16, 0, 0), flush,
                                     us, us_cold)
    return res


def surface_times(ctx, frames: int, iters: int, flush) -> dict:
    """The reference's single ops that the fused ops replace in the pass,
    timed alone at this S (f16, head-major (S, 16, T, 64) where the op is
    head-major): rope_apply in place (engine/ops.rs:202-223), attn_merge
    (:255-267), tiled_add of the positional table (:374-389) and
    cast_to_f16 (tensor.rs:148-160). Warm (back-to-back launches) and cold
    (behind a cache flush); rope_apply beside the ``inplace`` probe (one
    buffer read and written back)."""
    import torch

    from headshot_amd import rope as _rope

    t = GRID[0] * GRID[1] + PREFIX
    p = GRID[0] * GRID[1]
    rows = frames * t
    d = ctx.device
    g = torch.Generator(device="cpu").manual_seed(12)
    sin, cos = (torch.from_numpy(a).to(d) for a in _rope.tables(_rope.periods(), *GRID))
    out = {}

    def entry(fn, nbytes):
        us, us_c = warm_us(fn, iters), cold_us(fn, flush, iters)
        return {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1),
                "frac": round(nbytes / us / 1e3 / PEAK_GBS, 4), "cold_us": round(us_c, 2),
                "cold_frac": round(nbytes / us_c / 1e3 / PEAK_GBS, 4), "bytes": nbytes}

    q = torch.randn((frames, HEADS, t, HEAD_DIM), generator=g).half().to(d)
    ctx.rope_apply(q, sin, cos, PREFIX)
    rope_call = ctx.last_launch
    nb = q.numel() * 2 * 2
    out["rope_apply"] = entry(rope_call, nb)
    if os.path.exists(CEILING_LIB):
        def make_set():
            return (None, None, torch.ones(q.numel(), device=d, dtype=torch.float16), None)

        out["rope_apply"]["ceiling"] = probe_entry(
            load_ceiling(), "inplace", make_set, nb, (q.numel() * 2 // 16, 0, 0), flush,
            out["rope_apply"]["us"], out["rope_apply"]["cold_us"])
    merged = ctx.attn_merge(q)
    out["attn_merge"] = entry(ctx.last_launch, q.numel() * 2 * 2)
    del merged
    x = torch.randn((rows, DIM), generator=g).half().to(d)
    pos = torch.randn((p, DIM), generator=g).to(d) * 0.02
    x32 = torch.randn((frames * p, DIM), generator=g).to(d)
    tiled = ctx.tiled_add(x32, pos)
    out["tiled_add"] = entry(ctx.last_launch, x32.numel() * 4 * 2 + pos.numel() * 4)
    del tiled
    h = ctx.cast_to_f16(x32)
    out["cast_to_f16"] = entry(ctx.last_launch, x32.numel() * (4 + 2))
    del h, x, q
    return out


def alternating_best(fns: dict, timed, rounds: int = 3) -> dict:
    """Times each contestant (name -> callable) with timed(fn) -> ms in
    `rounds` rounds that take them in turn, rotating which goes first, and
    keeps each one's fastest round: no contestant always runs first (right
    after its inputs were made, on a clock the others then warm up)."""
    best = {k: float("inf") for k in fns}
    names = list(fns)
    for r in range(rounds):
        for k in names[r % len(names):] + names[:r % len(names)]:
            best[k] = min(best[k], timed(fns[k]))
    return best


def gemm_times(ctx, frames: int, iters: int) -> dict:
    """The aggregator block's four linear layers at this S (S*1374 rows, f16),
    each with the epilogue the block applies fused in: qkv (bias, split into
    heads, QK-norm and RoPE of a frame block), proj (bias + LayerScale +
    residual), fc1 (bias + exact GELU), fc2 (bias + LayerScale + residual).
    flops = 2*m*n*k. For reference the same shapes' plain product through
    torch (the ROCm BLAS library, no bias or epilogue) is timed beside them
    (not part of this library), and so is this library's standalone op that
    each fused epilogue replaces, so library_plus_op_ms is the unfused
    alternative. Each figure is its fastest of three alternating rounds."""
    from headshot_amd import rope as _rope
    import torch

    m = frames * (GRID[0] * GRID[1] + PREFIX)
    g = torch.Generator(device="cpu").manual_seed(13)
    shapes = {"qkv": (3 * DIM, DIM), "proj": (DIM, DIM), "fc1": (HIDDEN, DIM), "fc2": (DIM, HIDDEN)}
    out = {}

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters

    total_ms = 0.0
    for name, (n, k) in shapes.items():
        x = torch.randn((m, k), generator=g).half().to(ctx.device)
        w = (torch.randn((n, k), generator=g) / k ** 0.5).half().to(ctx.device)
        b = (torch.randn(n, generator=g) * 0.02).to(ctx.device)
        o = torch.empty((m, n), dtype=torch.float16, device=ctx.device)
        if name == "qkv":
            t = GRID[0] * GRID[1] + PREFIX
            sin, cos = (torch.from_numpy(a).to(ctx.device) for a in _rope.tables(_rope.periods(), *GRID))
            nrm = (torch.ones(HEAD_DIM, device=ctx.device), torch.zeros(HEAD_DIM, device=ctx.device))
            qkv = tuple(torch.empty((frames, HEADS, t, HEAD_DIM), dtype=torch.float16,
                                    device=ctx.device) for _ in range(3))
            ctx.linear_qkv_heads(x, w, b, frames, t, HEADS, qn=nrm, kn=nrm, rope=(sin, cos, PREFIX),
                                 eps=EPS, out=qkv)
        elif name == "fc1":
            ctx.linear_gelu(x, w, b, out=o)
        else:
            res = torch.randn((m, n), generator=g).half().to(ctx.device)
            gam = torch.full((n,), 1e-5, device=ctx.device)
            ctx.linear_ls_residual(x, w, gam, res, b, out=o)
        call = ctx.last_launch
        # the standalone op that the fused epilogue replaces, on a product-
        # shaped input: the q and k heads (QK-norm + RoPE pair), LayerScale +
        # residual, or bias + GELU
        y = torch.randn((m, DIM if name == "qkv" else n), generator=g).half().to(ctx.device)
        if name == "qkv":
            y2 = torch.randn((m, DIM), generator=g).half().to(ctx.device)
            ctx.qknorm_rope_pair(y, y2, frames, t, HEADS, HEAD_DIM, qn=nrm, kn=nrm,
                                 rope=(sin, cos, PREFIX), eps=EPS, out_q=qkv[0], out_k=qkv[1])
            op_name = "qknorm_rope_pair"
        elif name == "fc1":
            ctx.bias_gelu(y, b, out=o)
            op_name = "bias_gelu"
        else:
            ctx.bias_ls_residual(res, y, gam, b, out=o)
            op_name = "bias_ls_residual"
        op_call = ctx.last_launch
        best = alternating_best({"fused": call, "library": lambda: torch.nn.functional.linear(x, w),
                                 "op": op_call}, timed)
        ms, ms_lib, ms_op = best["fused"], best["library"], best["op"]
        fl = 2.0 * m * n * k
        tf = fl / (ms * 1e-3) / 1e12
        out[name] = {"m": m, "n": n, "k": k, "ms": round(ms, 3), "TFLOP/s": round(tf, 1),
                     "frac": round(tf / MFMA_PEAK_TFLOPS, 4), "library_gemm_ms": round(ms_lib, 3),
                     "standalone_op": op_name, "standalone_op_ms": round(ms_op, 3),
                     "library_plus_op_ms": round(ms_lib + ms_op, 3)}
        total_ms += ms
        del x, w, o
    out["ms_per_block"] = round(total_ms, 3)
    out["ms_per_pass"] = round(total_ms * (N_FRAME_BLOCKS + N_GLOBAL_BLOCKS), 2)
    out["layernorm_prologue"] = ln_prologue_times(ctx, m, timed, g)
    return out


def ln_prologue_times(ctx, m: int, timed, g) -> dict:
    """The pre-norm LayerNorm as the prologue of the product after it
    (hs_layernorm_stats + hs_linear_ln_gelu / hs_linear_ln_qkv_heads, which
    normalise the x tiles in LDS; bit-identical results) against layernorm
    then the fused product, at the block's LN2 -> fc1 + GELU and LN1 ->
    q|k|v (heads, QK-norm, RoPE) shapes. Times include the statistics pass;
    each is its fastest of three alternating rounds."""
    import torch

    from headshot_amd import rope as _rope

    t = GRID[0] * GRID[1] + PREFIX
    frames = m // t
    x = torch.randn((m, DIM), generator=g).half().to(ctx.device)
    lw = (1 + 0.02 * torch.randn(DIM, generator=g)).to(ctx.device)
    lb = (0.02 * torch.randn(DIM, generator=g)).to(ctx.device)
    normed = ctx.layernorm(x, lw, lb, eps=EPS)
    ln_call = ctx.last_launch
    ws = torch.empty((m, 2), dtype=torch.float32, device=ctx.device)
    ctx.layernorm_stats(x, eps=EPS, out=ws)
    best = alternating_best({"layernorm": ln_call, "stats": ctx.last_launch}, timed)
    out = {"layernorm_us": round(best["layernorm"] * 1e3, 1), "stats_us": round(best["stats"] * 1e3, 1)}
    sin, cos = (torch.from_numpy(a).to(ctx.device) for a in _rope.tables(_rope.periods(), *GRID))
    nrm = (torch.ones(HEAD_DIM, device=ctx.device), torch.zeros(HEAD_DIM, device=ctx.device))
    for name, n in (("fc1", HIDDEN), ("qkv", 3 * DIM)):
        w = (torch.randn((n, DIM), generator=g) / DIM ** 0.5).half().to(ctx.device)
        b = (torch.randn(n, generator=g) * 0.02).to(ctx.device)
        if name == "fc1":
            o = torch.empty((m, n), dtype=torch.float16, device=ctx.device)
            ctx.linear_gelu(normed, w, b, out=o)
            plain = ctx.last_launch
            ctx.linear_ln_gelu(x, (lw, lb), w, b, eps=EPS, out=o, workspace=ws)
            fused = ctx.last_launch
        else:
            o = tuple(torch.empty((frames, HEADS, t, HEAD_DIM), dtype=torch.float16,
                                  device=ctx.device) for _ in range(3))
            ctx.linear_qkv_heads(normed, w, b, frames, t, HEADS, qn=nrm, kn=nrm,
                                 rope=(sin, cos, PREFIX), eps=EPS, out=o)
            plain = ctx.last_launch
            ctx.linear_ln_qkv_heads(x, (lw, lb), w, b, frames, t, HEADS, qn=nrm, kn=nrm,
                                    rope=(sin, cos, PREFIX), eps=EPS, out=o, workspace=ws)
            fused = ctx.last_launch
        best = alternating_best({"plain": lambda: (ln_call(), plain()), "prologue": fused,
                                 "plain_product": plain}, timed)
        ms_plain, ms_pro = best["plain"], best["prologue"]
        fl = 2.0 * m * n * DIM
        out[name] = {"layernorm_then_product_ms": round(ms_plain, 3),
                     "product_alone_ms": round(best["plain_product"], 3),
                     "prologue_ms": round(ms_pro, 3),
                     "prologue_TFLOP/s": round(fl / (ms_pro * 1e-3) / 1e12, 1)}
        del w, o
    return out


def block_times(ctx, frames: int, iters: int) -> dict:
    """One whole frame block and one global block at this S with every op on
    HIP (headshot_amd.aggregator.block_forward: linears with fused
    epilogues, fused QK-norm/RoPE, attention written token-major), and the
    reference's unfused dispatch sequence through the same library's single
    ops beside it (block_forward_reference). Random-init f16 weights. Each
    figure is its fastest of three alternating rounds."""
    import torch

    from headshot_amd import rope as _rope
    from headshot_amd.aggregator import BlockWeights, block_forward, block_forward_reference

    t = GRID[0] * GRID[1] + PREFIX
    gen = torch.Generator(device=ctx.device).manual_seed(17)
    wts = BlockWeights.random(DIM, HIDDEN, HEAD_DIM, torch.float16, ctx.device, gen)
    x = torch.randn((frames * t, DIM), generator=gen, device=ctx.device).half()
    sin, cos = (torch.from_numpy(a).to(ctx.device) for a in _rope.tables(_rope.periods(), *GRID))
    out = {}

    def ln_prologue(*a, **kw):
        return block_forward(*a, fuse_ln=True, **kw)

    for kind, (s, tt, rope) in {"frame": (frames, t, (sin, cos, PREFIX)),
                                "global": (1, frames * t, None)}.items():
        def timed(fn):
            fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(iters):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / iters

        fns = {name: (lambda f=f: f(ctx, wts, x, s, tt, rope=rope, eps=EPS))
               for name, f in (("fused", block_forward), ("reference_sequence", block_forward_reference),
                               ("fused_layernorm_prologue", ln_prologue))}
        out[kind] = {name + "_ms": round(ms, 3) for name, ms in alternating_best(fns, timed).items()}
    out["aggregator_ms"] = round(N_FRAME_BLOCKS * out["frame"]["fused_ms"]
                                 + N_GLOBAL_BLOCKS * out["global"]["fused_ms"], 1)
    out["aggregator_reference_sequence_ms"] = round(
        N_FRAME_BLOCKS * out["frame"]["reference_sequence_ms"]
        + N_GLOBAL_BLOCKS * out["global"]["reference_sequence_ms"], 1)
    out["aggregator_layernorm_prologue_ms"] = round(
        N_FRAME_BLOCKS * out["frame"]["fused_layernorm_prologue_ms"]
        + N_GLOBAL_BLOCKS * out["global"]["fused_layernorm_prologue_ms"], 1)
    return out


def f32_block_times(ctx, iters: int) -> dict:
    """The reference's f32 path at S=2 x 1374 (its CPU-runnable case): one
    frame block and one global block with every op on HIP in f32
    (block_forward, random-init f32 weights), and the blocks' matrix kernels
    in f32: attention fused with the head merge (hs_attention_merged), the
    q|k|v projection with its head split, QK-norm and RoPE (three products
    and the head ops in f32), proj and fc2 with LayerScale + residual, fc1
    with GELU. Beside each, torch's library op (f32 scaled_dot_product_
    attention, F.linear of the same shape; not part of this library). HIP
    events around `iters` back-to-back calls; each figure the fastest of
    three alternating rounds."""
    import torch

    from headshot_amd import rope as _rope
    from headshot_amd.aggregator import BlockWeights, block_forward

    frames = 2
    t = GRID[0] * GRID[1] + PREFIX
    m = frames * t
    gen = torch.Generator(device=ctx.device).manual_seed(19)
    wts = BlockWeights.random(DIM, HIDDEN, HEAD_DIM, torch.float32, ctx.device, gen)
    p = wts.p
    x = torch.randn((m, DIM), generator=gen, device=ctx.device)
    sin, cos = (torch.from_numpy(a).to(ctx.device) for a in _rope.tables(_rope.periods(), *GRID))

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters

    out = {"shape": {"frames": frames, "tokens": t, "dim": DIM}}
    blocks = {"frame": (frames, t, (sin, cos, PREFIX)), "global": (1, m, None)}
    best = alternating_best({kind: (lambda s_=s_, tt=tt, r=r: block_forward(ctx, wts, x, s_, tt, rope=r,
                                                                             eps=EPS))
                             for kind, (s_, tt, r) in blocks.items()}, timed)
    out["block_ms"] = {kind: round(ms, 3) for kind, ms in best.items()}

    att = {}
    g = torch.Generator(device="cpu").manual_seed(23)
    for name, (s_, tt) in {"frame": (frames, t), "global": (1, m)}.items():
        q, k, v = (torch.randn((s_, HEADS, tt, HEAD_DIM), generator=g).to(ctx.device) for _ in range(3))
        o = torch.empty((s_ * tt, HEADS * HEAD_DIM), device=ctx.device)
        ctx.attention_merged(q, k, v, out=o)
        call = ctx.last_launch
        b = alternating_best({"hip": call, "library": lambda: torch.nn.functional.
                              scaled_dot_product_attention(q, k, v)}, timed)
        flops = 4.0 * tt * tt * HEAD_DIM * s_ * HEADS
        att[name] = {"shape_SHTD": [s_, HEADS, tt, HEAD_DIM], "ms": round(b["hip"], 3),
                     "TFLOP/s": round(flops / (b["hip"] * 1e-3) / 1e12, 1),
                     "library_sdpa_ms": round(b["library"], 3)}
        del q, k, v, o
    out["attention"] = att

    lin = {}
    xa = torch.randn((m, DIM), generator=g).to(ctx.device)
    xh = torch.randn((m, HIDDEN), generator=g).to(ctx.device)
    res = torch.randn((m, DIM), generator=g).to(ctx.device)
    o_d = torch.empty((m, DIM), device=ctx.device)
    o_h = torch.empty((m, HIDDEN), device=ctx.device)
    layers = {
        "qkv_heads": (lambda: ctx.linear_qkv_heads(xa, wts.qkv_w, wts.qkv_b, frames, t, HEADS,
                                                   qn=p.qn, kn=p.kn, rope=(sin, cos, PREFIX), eps=EPS),
                      lambda: torch.nn.functional.linear(xa, wts.qkv_w, wts.qkv_b), 3 * DIM, DIM),
        "proj_ls": (lambda: ctx.linear_ls_residual(xa, wts.proj_w, p.ls1, res, p.proj_b, out=o_d),
                    lambda: torch.nn.functional.linear(xa, wts.proj_w, p.proj_b), DIM, DIM),
        "fc1_gelu": (lambda: ctx.linear_gelu(xa, wts.fc1_w, p.fc1_b, out=o_h),
                     lambda: torch.nn.functional.linear(xa, wts.fc1_w, p.fc1_b), HIDDEN, DIM),
        "fc2_ls": (lambda: ctx.linear_ls_residual(xh, wts.fc2_w, p.ls2, res, p.fc2_b, out=o_d),
                   lambda: torch.nn.functional.linear(xh, wts.fc2_w, p.fc2_b), DIM, HIDDEN),
    }
    for name, (hip, library, n, k) in layers.items():
        b = alternating_best({"hip": hip, "library": library}, timed)
        flops = 2.0 * m * n * k
        lin[name] = {"MNK": [m, n, k], "ms": round(b["hip"], 3),
                     "TFLOP/s": round(flops / (b["hip"] * 1e-3) / 1e12, 1),
                     "library_linear_ms": round(b["library"], 3)}
    out["linear"] = lin
    return out


def trunk_times(ctx, frames: int, iters: int) -> dict:
    """One whole aggregator trunk forward at this S (model/trunk.rs:49-146)
    on HIP: token assembly from f32 DINO tokens (S x 37 x 37 patches, 17
    prefix tokens), 24 frame blocks and 24 inter-frame blocks (5 of them
    register-attention layers over S*17 tokens, 19 global over S*1386), the
    register gather/scatter and the 4 head-input caches. Random-init f16
    weights in the checkpoint's layout (fused q|k|v), generated on the
    device. Beside it the reference's dispatch sequence through the same
    library's single ops (Trunk.forward(fused=False)). Each figure is its
    fastest of three alternating rounds."""
    import torch

    from headshot_amd.aggregator import BlockWeights
    from headshot_amd.trunk import DIM as TDIM
    from headshot_amd.trunk import N_REG as TREG
    from headshot_amd.trunk import Trunk

    gen = torch.Generator(device=ctx.device).manual_seed(23)
    blocks = lambda: [BlockWeights.random(TDIM, 4 * TDIM, HEAD_DIM, torch.float16, ctx.device,  # noqa: E731
                                          gen, ls_init=0.05) for _ in range(N_FRAME_BLOCKS)]
    cam = torch.randn((2, TDIM), generator=gen, device=ctx.device).half()
    reg = torch.randn((2 * TREG, TDIM), generator=gen, device=ctx.device).half()
    from headshot_amd import rope as _rope
    trunk = Trunk(cam, reg, blocks(), blocks(), _rope.periods(), torch.float16)
    p = GRID[0] * GRID[1]
    tokens = torch.randn((frames * p, TDIM), generator=gen, device=ctx.device)
    out = {"frames": frames, "tokens_per_frame": p + 17}

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters

    fns = {name: (lambda fu=fused: trunk.forward(ctx, tokens, frames, *GRID, fused=fu))
           for name, fused in (("fused", True), ("reference_sequence", False))}
    for name, ms in alternating_best(fns, timed).items():
        out[name + "_ms"] = round(ms, 1)
    out["frames_per_s"] = round(frames / (out["fused_ms"] * 1e-3), 1)
    return out


def cpu_baseline_legs(frames: int) -> dict:
    """The oracle (the reference's kernels restated in C: attention.wesl's
    one-query-at-a-time online softmax, linear.wesl's k-order sums, the
    concat + cast of the cache build) on the host cores, over bounded
    samples of the extra legs' workloads at this S, in their units."""
    import numpy as np

    from oracle import oracle as O

    threads, _ = host_threads()
    O.set_num_threads(threads)
    rng = np.random.default_rng(3)
    t = GRID[0] * GRID[1] + PREFIX
    out = {}
    # global attention: 16 heads x 8 queries against all S*1374 keys
    tt = frames * t
    q, k, v = (rng.standard_normal((1, HEADS, tt, HEAD_DIM)).astype(np.float16) for _ in range(3))
    idx = np.arange(8, dtype=np.int32) * (tt // 8)
    t0 = time.perf_counter()
    O.attention(q, k, v, q_idx=idx)
    dt = time.perf_counter() - t0
    fl = 4.0 * idx.size * tt * HEAD_DIM * HEADS
    out["attention_global"] = {"value": round(fl / dt / 1e12, 5), "unit": "TFLOP/s",
                               "sample": f"{HEADS} heads x {idx.size} queries x {tt} keys, f16 "
                                         f"storage, {dt:.2f} s"}
    # fc1 linear rows: 64 rows of (S*1374, 1024) x (4096, 1024)^T
    x = rng.standard_normal((64, DIM)).astype(np.float16)
    w = (rng.standard_normal((HIDDEN, DIM)) / 32).astype(np.float16)
    t0 = time.perf_counter()
    O.linear(x, w)
    dt = time.perf_counter() - t0
    out["linear_fc1"] = {"value": round(2.0 * 64 * HIDDEN * DIM / dt / 1e12, 5), "unit": "TFLOP/s",
                         "sample": f"64 rows x {HIDDEN} x {DIM}, f16 storage, {dt:.2f} s"}
    # cache build: 4096 rows of 1024 + 1024 f16 -> f32
    a = rng.standard_normal((4096, DIM)).astype(np.float16)
    b = rng.standard_normal((4096, DIM)).astype(np.float16)
    t0 = time.perf_counter()
    for _ in range(5):
        O.cache_build(a, b)
    dt = (time.perf_counter() - t0) / 5
    out["cache_build"] = {"value": round(4096 * 2 * DIM * 6 / dt / 1e9, 3), "unit": "GB/s",
                          "sample": f"4096 rows x 2048 channels, {dt * 1e3:.1f} ms"}
    out["cores"] = threads
    out["kind"] = "port"
    return out


def host_threads() -> tuple:
    """(threads used, cores visible): every core this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS where the host sets it as
    this process's CPU share."""
    visible = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    used = min(visible, int(share)) if share.isdigit() and int(share) > 0 else visible
    return used, visible


def s2_f32_frame_block(ctx, seed: int = 0):
    """One frame block's fused-op sequence at S=2 frames
    x 1374 tokens x 1024, f32, 37 x 37 RoPE grid, prefix 5, eps 1e-6, with
    random-init parameters (LN gamma N(1,.02), beta/biases N(0,.02),
    LayerScale 1e-5) and N(0,1) activations and GEMM outputs."""
    import torch

    from headshot_amd import rope
    from headshot_amd.aggregator import BlockIO, BlockParams

    frames, t = 2, GRID[0] * GRID[1] + PREFIX
    rows = frames * t
    g = torch.Generator(device=ctx.device)
    g.manual_seed(seed)
    n = lambda *sh: torch.randn(sh, generator=g, device=ctx.device)  # noqa: E731
    io = BlockIO.empty_like_inputs(n(rows, DIM), n(rows, DIM), n(rows, DIM), n(rows, DIM),
                                   n(rows, HIDDEN), n(rows, DIM))
    p = BlockParams.random(DIM, HIDDEN, HEAD_DIM, ctx.device, g)
    sin, cos = rope.tables(rope.periods(), *GRID)
    tabs = (torch.from_numpy(sin).to(ctx.device), torch.from_numpy(cos).to(ctx.device), PREFIX)
    return io, p, tabs, frames, t


def cpu_baseline(ctx, target_s: float):
    """The CPU baseline: one frame block's fused-op sequence, f32, S=2 x
    1374 x 1024, through the oracle (the reference's f32
    WGSL kernels restated in C, run in the reference's unfused dispatch
    order: layernorm, split_heads + layernorm + rope_apply for q and k,
    residual_ls, layernorm, gelu, residual_ls), OpenMP over rows on the host
    cores; median of repeated runs (at least 5, about ``target_s`` seconds).
    The same block on the GPU (HipContext, the fused ops) is timed beside it
    on the same inputs."""
    import numpy as np
    import torch

    from headshot_amd.aggregator import run_block_ops
    from oracle import oracle as O

    threads, visible = host_threads()
    O.set_num_threads(threads)
    io, p, (sin, cos, prefix), frames, t = s2_f32_frame_block(ctx)
    rows = frames * t
    nbytes = rows * 45056 * 2  # per-token algorithmic bytes of a block, f32 storage
    h = lambda x: x.detach().cpu().numpy()  # noqa: E731
    P = {k: tuple(h(x) for x in v) if isinstance(v, tuple) else h(v) for k, v in vars(p).items()}
    x, q, k = h(io.x), h(io.q_raw), h(io.k_raw)
    proj, fc1, fc2 = h(io.proj_raw), h(io.fc1_raw), h(io.fc2_raw)
    out = dict(normed=np.empty_like(x), q_head=np.empty_like(q), k_head=np.empty_like(k),
               x1=np.empty_like(x), normed2=np.empty_like(x), act=np.empty_like(fc1),
               x_out=np.empty_like(x))
    hs, hc = h(sin), h(cos)

    def cpu_block():
        O.block_ops(O.F32, x, *P["ln1"], q, k, *P["qn"], *P["kn"], hs, hc, prefix, proj,
                    P["proj_b"], P["ls1"], *P["ln2"], fc1, P["fc1_b"], fc2, P["fc2_b"], P["ls2"],
                    out, frames, t, DIM, HEADS, HIDDEN, EPS)

    cpu_block()  # first touch of the output pages, thread pool start
    runs = []
    t_all = time.perf_counter()
    while len(runs) < 5 or time.perf_counter() - t_all < target_s:
        t0 = time.perf_counter()
        cpu_block()
        runs.append(time.perf_counter() - t0)
    cpu_s = float(np.median(runs))

    # the GPU, same inputs and op sequence
    def gpu_block():
        run_block_ops(ctx, p, io, frames, t, HEADS, HEAD_DIM, rope=(sin, cos, prefix), eps=EPS)

    seq = []
    run_block_ops(ctx, p, io, frames, t, HEADS, HEAD_DIM, rope=(sin, cos, prefix), eps=EPS,
                  record=lambda op: seq.append(ctx.last_launch))
    for _ in range(10):
        gpu_block()
    torch.cuda.synchronize()
    # a HIP graph of `reps` back-to-back blocks, replayed: the kernels' time,
    # not the host's launch rate (6 small launches per block)
    reps, replays = 64, 5
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            for thunk in seq:
                thunk()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    gpu_ms = a.elapsed_time(b) / (reps * replays)
    del graph
    gpu_gbs = nbytes / (gpu_ms * 1e-3) / 1e9
    return {
        "value": round(nbytes / cpu_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"one frame block's fused-op sequence, f32, S={frames} x {t} x "
                   f"{DIM}, 37x37 RoPE, prefix {prefix}, through oracle/hs_oracle.c (C "
                   f"restatement of the reference's f32 WGSL kernels, unfused reference "
                   f"dispatch order), {threads} OpenMP threads of {visible} visible cores; "
                   f"median of {len(runs)} runs"),
        "ms_per_block": round(cpu_s * 1e3, 2),
        "tokens_per_s": round(rows / cpu_s, 1),
        "bytes_per_block": nbytes,
        "runs": len(runs),
        "cpu_model": cpu_model(),
        "gpu_same_config": {"ms_per_block": round(gpu_ms, 4), "GB/s": round(gpu_gbs, 1),
                            "frac": round(gpu_gbs / PEAK_GBS, 4),
                            "tokens_per_s": round(rows / (gpu_ms * 1e-3), 1),
                            "timing": f"HIP graph of {reps} back-to-back blocks (6 launches "
                                      f"each, fused ops), {replays} replays"},
    }


def cpu_pass_sample(bench: Pass, target_s: float):
    """The oracle (C restatement of the reference's f32-math kernels, run
    with the reference's unfused dispatch sequence and f16 storage rounding)
    on the host cores over a bounded sample of the benchmarked pass."""
    import numpy as np
    import torch

    from oracle import oracle as O

    threads, _ = host_threads()
    O.set_num_threads(threads)
    dt = O.F16 if bench.dtype == torch.float16 else O.F32
    h = lambda t: t.cpu().numpy()  # noqa: E731
    rows, frames = bench.rows, bench.frames
    fp = bench.fp
    x = h(fp.x[0])
    q, k = h(fp.io.q_raw), h(fp.io.k_raw)
    proj, fc1, fc2 = h(fp.io.proj_raw), h(fp.io.fc1_raw), h(fp.io.fc2_raw)
    sin, cos = h(fp.sin), h(fp.cos)
    out = dict(normed=np.empty_like(x), q_head=np.empty_like(q), k_head=np.empty_like(k),
               x1=np.empty_like(x), normed2=np.empty_like(x), act=np.empty_like(fc1),
               x_out=np.empty_like(x))
    patches, pos, pb = h(fp.patches), h(fp.pos), h(fp.patch_bias)
    cam, reg = h(fp.cam), h(fp.reg)

    done_bytes = 0
    blocks_done = 0
    t0 = time.perf_counter()
    O.assemble_tokens(patches, pb, pos, cam, reg, frames, bench.p, N_REG, x.dtype)
    done_bytes += bench.bytes["assemble"]
    block_bytes = (2 * bench.bytes["layernorm"] + bench.bytes["qknorm_rope"]
                   + 2 * bench.bytes["bias_ls_residual"] + bench.bytes["bias_gelu"])
    for kind, b in zip(fp.kinds, fp.blocks):
        p = {kk: tuple(h(t) for t in v) if isinstance(v, tuple) else h(v)
             for kk, v in vars(b).items()}
        frame_block = kind == "frame"
        s, t = (frames, bench.t) if frame_block else (1, rows)
        O.block_ops(dt, x, *p["ln1"], q, k, *p["qn"], *p["kn"],
                    sin if frame_block else None, cos if frame_block else None, PREFIX,
                    proj, p["proj_b"], p["ls1"], *p["ln2"], fc1, p["fc1_b"], fc2, p["fc2_b"],
                    p["ls2"], out, s, t, DIM, HEADS, HIDDEN, EPS)
        done_bytes += block_bytes
        blocks_done += 1
        if time.perf_counter() - t0 >= target_s and blocks_done >= 2:
            break
    elapsed = time.perf_counter() - t0
    return {
        "value": round(done_bytes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle over assembly + {blocks_done} of 48 blocks of the benchmarked pass "
                   f"at S={frames}, {'f16' if dt == O.F16 else 'f32'} storage: "
                   f"{done_bytes / 1e9:.2f} GB algorithmic in {elapsed:.1f} s, {threads} threads"),
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the baseline record."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


KERNEL_OPS = {"ln_vec_kernel": "layernorm", "ln_generic_kernel": "layernorm",
              "qkn_row_kernel": "qknorm_rope", "qkn_generic_kernel": "qknorm_rope",
              "bias_ls_kernel": "bias_ls_residual", "bias_gelu_kernel": "bias_gelu",
              "assemble_kernel": "assemble", "ls_ln_kernel": "bias_ls_residual_layernorm"}
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "aggregator_pass_s32_f16_traffic.json")


def kernel_op(name: str):
    for k, op in KERNEL_OPS.items():
        if k in name:
            return op
    return None


def load_traffic(op: str, frames: int, dtype: str):
    """HBM bytes per launch of `op` measured by rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE runs of this benchmark (written by --summarize), if recorded
    for this workload."""
    try:
        t = json.load(open(TRAFFIC_JSON))
    except (OSError, ValueError):
        return None
    if t.get("frames") != frames or t.get("dtype") != dtype or op not in t.get("ops", {}):
        return None
    return {"bytes_per_launch": t["ops"][op]["hbm_bytes_per_launch"],
            "source": f"profiles/{os.path.basename(TRAFFIC_JSON)}"}


def summarize_counters(paths) -> None:
    """Per matrix-core kernel and launch shape, the mean of each shader
    counter over its dispatches, and ratios derived from them (MI355X: 8
    XCDs, 256 CUs, 1024 SIMDs; rocprofv3 reports GRBM_GUI_ACTIVE summed over
    the XCDs, so one XCD's busy cycles are an eighth of it, and that over the
    dispatch's duration is the clock the kernel ran at)."""
    import csv
    import statistics as st
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))
    dur = defaultdict(list)
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            op = kernel_op(name)
            if op is None:
                if "flash_f16_kernel" in name:
                    op = "flash_f16_kernel"
                elif "gemm_f16_kernel" in name:
                    op = "gemm_f16_kernel<" + name.split("gemm_f16_kernelILi")[1][0] + ">"
                else:
                    continue
            key = (op, int(r["Grid_Size"]))
            vals[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
            dur[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9)
    out = ["| kernel | grid work-items | dispatches | mean us | shader clock GHz "
           "| matrix core busy | VALU co-issue with MFMA "
           "| cycles / MFMA | VALU / MFMA | transcendental / MFMA | LDS busy "
           "| bank-conflict cycles / LDS instr |",
           "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for key in sorted(vals):
        c = {k: st.mean(v) for k, v in vals[key].items()}
        cyc = c.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
        if not cyc or not c.get("SQ_INSTS_MFMA"):
            continue  # matrix-core kernels only

        def f(expr, fmt):
            try:
                return format(expr(), fmt)
            except (KeyError, ZeroDivisionError):
                return "-"
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        mean_s = st.mean(dur[key])
        out.append("| " + " | ".join([
            key[0], str(key[1]), str(len(dur[key]) // max(1, len(vals[key]))),
            format(mean_s * 1e6, ".1f"), format(cyc / mean_s / 1e9, ".2f"),
            f(lambda: c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * 1024), ".1%"),
            f(lambda: c["SQ_VALU_MFMA_COEXEC_CYCLES"] / (cyc * 1024), ".1%"),
            f(lambda: c["SQ_VALU_MFMA_BUSY_CYCLES"] / mf, ".1f"),
            f(lambda: (c["SQ_INSTS_VALU"] - mf) / mf, ".2f"),
            f(lambda: c["SQ_INSTS_VALU_TRANS_F32"] / mf, ".2f"),
            f(lambda: c["SQ_LDS_IDX_ACTIVE"] / (cyc * 256), ".1%"),
            f(lambda: c["SQ_LDS_BANK_CONFLICT"] / c["SQ_INSTS_LDS"], ".2f")]) + " |")
    # Wave stall breakdown, when a pass collected it: SQ_WAVE_CYCLES and the
    # SQ_WAIT_* counters all count quad-cycles per resident wave.
    stall = ["", "| kernel | grid work-items | waves resident per SIMD | waiting on a dependency "
             "| ready, waiting for issue | waiting for LDS issue |", "|---|---|---|---|---|---|"]
    for key in sorted(vals):
        c = {k: st.mean(v) for k, v in vals[key].items()}
        cyc = c.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
        w = c.get("SQ_WAVE_CYCLES", 0.0)
        if not cyc or not w or "SQ_WAIT_ANY" not in c or not c.get("SQ_INSTS_MFMA"):
            continue
        stall.append("| " + " | ".join([
            key[0], str(key[1]), format(4 * w / (cyc * 1024), ".2f"),
            format(c["SQ_WAIT_ANY"] / w, ".1%"), format(c.get("SQ_WAIT_INST_ANY", 0.0) / w, ".1%"),
            format(c.get("SQ_WAIT_INST_LDS", 0.0) / w, ".1%")]) + " |")
    if len(stall) > 3:
        out += stall
    print("\n".join(out))


def summarize(args) -> None:
    """Markdown summary of rocprofv3 CSV output for this benchmark's kernels:
    kernel-trace durations against the algorithmic bytes, and (with
    --pmc-fetch/--pmc-write counter_collection CSVs) HBM bytes per launch,
    scaled by what the counters read for the calibration copy
    (--calibrate-copy-mib MiB each way, the largest copy-kernel dispatch)."""
    import csv
    import statistics as st
    from collections import defaultdict

    esz = 2 if args.dtype == "f16" else 4
    p = GRID[0] * GRID[1]
    rows = args.frames * (p + PREFIX)
    nbytes = op_bytes(rows, esz, args.frames * p, p)
    launches = pass_launches(N_FRAME_BLOCKS, N_GLOBAL_BLOCKS, args.fuse_layernorm)
    legs = args.legs_trace or args.summarize
    dur = defaultdict(list)
    for r in csv.DictReader(open(args.summarize)):
        op = kernel_op(r["Kernel_Name"])
        if op:
            dur[op].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = [f"## Kernel durations (rocprofv3 --kernel-trace), S={args.frames} {args.dtype}", "",
           "| op | kernel calls | mean us | median us | algorithmic MB/launch | GB/s (mean) "
           "| of 8 TB/s |", "|---|---|---|---|---|---|---|"]
    pass_us = 0.0
    other = pass_launches(N_FRAME_BLOCKS, N_GLOBAL_BLOCKS, not args.fuse_layernorm)
    for op in dict.fromkeys([*launches, *other]):  # the other sequence's op after the pass's
        if not dur[op]:
            continue
        m, med = st.mean(dur[op]), st.median(dur[op])
        gbs = nbytes[op] / (m * 1e-6) / 1e9
        if op in launches:
            pass_us += m * launches[op]
        out.append(f"| {op} | {len(dur[op])} | {m:.2f} | {med:.2f} | {nbytes[op] / 1e6:.1f} | "
                   f"{gbs:.0f} | {gbs / PEAK_GBS:.1%} |")
    out += ["", f"Sum of mean kernel times x launches per pass: {pass_us / 1e3:.3f} ms "
                f"({sum(nbytes[o] * launches[o] for o in launches) / (pass_us * 1e-6) / 1e9:.0f} GB/s "
                f"algorithmic)."]
    # Attention (the benchmark's attention leg): the flash kernel, told apart by
    # grid size: one workgroup of 8 waves (512 work-items) per 256 queries of
    # one (sequence, head), the (sequence, head) count rounded up to the 8 XCDs.
    # When the last query tile is partial and there are at least two such
    # tiles per CU (256 CUs), the call is two launches (the full tiles, then
    # the partial ones); its time is their sum.
    att = defaultdict(list)
    t_tok = GRID[0] * GRID[1] + PREFIX
    for r in csv.DictReader(open(legs)):
        if "flash_f16_kernel" in r["Kernel_Name"]:
            att[int(r["Grid_Size_X"])].append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    shapes = {"frame": (args.frames, t_tok), "global": (1, args.frames * t_tok)}

    def att_grids(s_, tt):
        """(main launch grid, tail launch grid or None) in work-items."""
        sh, qt = s_ * HEADS, -(-tt // 256)
        per_tile = 8 * -(-sh // 8) * 512
        if tt % 256 and qt > 1 and sh >= 2 * 256:
            return per_tile * (qt - 1), per_tile
        return per_tile * qt, None

    att_grid = {name: att_grids(s_, tt) for name, (s_, tt) in shapes.items()}
    if any(att_grid[n][0] in att for n in shapes):
        out += ["", "## Attention (flash_f16_kernel, f16, 16 heads of 64)", "",
                "| call | grid work-items | kernel calls | mean us | TFLOP/s | of 2.5 PFLOP/s |",
                "|---|---|---|---|---|---|"]
        for name, (s_, tt) in shapes.items():
            grid, tail = att_grid[name]
            durs = att.get(grid)
            if not durs:
                continue
            m = st.mean(durs) + (st.mean(att[tail]) if tail and att.get(tail) else 0.0)
            tf = 4.0 * tt * tt * HEAD_DIM * s_ * HEADS / (m * 1e-6) / 1e12
            shown = f"{grid} + {tail}" if tail else str(grid)
            out.append(f"| {name} (S={s_}, T={tt}) | {shown} | {len(durs)} | {m:.1f} | {tf:.0f} | "
                       f"{tf / MFMA_PEAK_TFLOPS:.1%} |")
    cache = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
             for r in csv.DictReader(open(legs))
             if "concat_vec_kernelIDF16_f" in r["Kernel_Name"]
             and int(r["Grid_Size_X"]) >= 256 * 256]
    if cache:
        rows_c = args.frames * t_tok
        cb = rows_c * 2 * DIM * 6
        m = st.mean(cache)
        # hs_cache_build and the reference sequence's cast_to_f32 run this
        # kernel on the same number of 8-element chunks and move the same
        # bytes (2 B in, 4 B out per element), so one row covers both.
        out += ["", "## Cache build (concat_vec_kernel, f16 in, f32 out)", "",
                "| calls | mean us | algorithmic MB per call | GB/s | of 8 TB/s |",
                "|---|---|---|---|---|",
                f"| {len(cache)} | {m:.1f} | {cb / 1e6:.1f} | {cb / (m * 1e-6) / 1e9:.0f} | "
                f"{cb / (m * 1e-6) / 1e9 / PEAK_GBS:.1%} |"]
    gem = defaultdict(list)
    for r in csv.DictReader(open(legs)):
        if "gemm_f16_kernel" in r["Kernel_Name"]:
            epi = r["Kernel_Name"].split("gemm_f16_kernelILi")[1][0]
            gem[(epi, int(r["Grid_Size_X"]))].append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    if gem:
        m = args.frames * t_tok

        def grid_items(n):
            # the fast path's launch: 256 x 256 output tiles, rounded up to a
            # multiple of 8 workgroups (one per XCD), 512 work-items each
            tiles = -(-m // 256) * (n // 256)
            return -(-tiles // 8) * 8 * 512

        # (epilogue, n) -> the layers of that launch shape; proj and fc2
        # share both, and fc2 (k = 4096) runs the longer half of the calls
        layers = {("3", 3 * DIM): [("qkv", DIM)],
                  ("0", DIM): [("q / k / v (reference sequence, comparison)", DIM)],
                  ("0", HIDDEN): [("fc1, no epilogue (reference sequence, comparison)", DIM)],
                  ("1", HIDDEN): [("fc1", DIM)], ("2", DIM): [("proj", DIM), ("fc2", HIDDEN)]}
        epis = ["bias", "bias + GELU", "bias + LayerScale + residual",
                "bias, heads, QK-norm + RoPE"]
        out += ["", "## Linear layers (gemm_f16_kernel, f16, epilogue fused)", "",
                "| layer | epilogue | kernel calls | mean us | TFLOP/s | of 2.5 PFLOP/s |",
                "|---|---|---|---|---|---|"]
        for (epi, n), cands in layers.items():
            durs = sorted(gem.get((epi, grid_items(n)), []))
            if not durs:
                continue
            size = len(durs) // len(cands)
            for i, (name, k) in enumerate(cands):
                part = durs[i * size:(i + 1) * size]
                mu = st.mean(part)
                tf = 2.0 * m * n * k / (mu * 1e-6) / 1e12
                out.append(f"| {name} | {epis[int(epi)]} | {len(part)} | {mu:.1f} | "
                           f"{tf:.0f} | {tf / MFMA_PEAK_TFLOPS:.1%} |")
    if args.pmc_fetch and args.pmc_write:
        def counters(path, name):
            # The calibration copy (torch's device-to-device copy_) runs as
            # the runtime's blit kernel __amd_rocclr_copyBuffer.
            per_op, copy = defaultdict(list), []
            for r in csv.DictReader(open(path)):
                if r.get("Counter_Name") != name:
                    continue
                v = float(r["Counter_Value"])
                op = kernel_op(r["Kernel_Name"])
                if op:
                    per_op[op].append(v)
                elif "rocclr_copyBuffer" in r["Kernel_Name"]:
                    copy.append(v)
            return per_op, (max(copy) if copy else None)

        fetch, f_cal = counters(args.pmc_fetch, "FETCH_SIZE")
        write, w_cal = counters(args.pmc_write, "WRITE_SIZE")
        known_kib = args.calibrate_copy_mib * 1024.0
        f_scale = known_kib / f_cal if f_cal else 1.0
        w_scale = known_kib / w_cal if w_cal else 1.0
        out += ["", "## HBM traffic (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE; KiB per dispatch)",
                "", f"Calibration: a {args.calibrate_copy_mib} MiB device copy read "
                f"{f_cal} KiB (FETCH_SIZE) and wrote {w_cal} KiB (WRITE_SIZE); scale factors "
                f"{f_scale:.4f} (fetch), {w_scale:.4f} (write).", "",
                "| op | dispatches | FETCH KiB | WRITE KiB | HBM MB/launch (scaled) | "
                "algorithmic MB | ratio |", "|---|---|---|---|---|---|---|"]
        traffic = {"frames": args.frames, "dtype": args.dtype, "fetch_scale": f_scale,
                   "write_scale": w_scale, "ops": {}}
        for op in OPS:
            if not fetch[op] or not write[op]:
                continue
            fk, wk = st.mean(fetch[op]), st.mean(write[op])
            hbm = (fk * f_scale + wk * w_scale) * 1024.0
            traffic["ops"][op] = {"fetch_kib": fk, "write_kib": wk,
                                  "hbm_bytes_per_launch": int(hbm),
                                  "algorithmic_bytes": nbytes[op]}
            out.append(f"| {op} | {len(fetch[op])} | {fk:.0f} | {wk:.0f} | {hbm / 1e6:.1f} | "
                       f"{nbytes[op] / 1e6:.1f} | {hbm / nbytes[op]:.3f} |")
        if args.traffic_json:
            with open(args.traffic_json, "w") as f:
                json.dump(traffic, f, indent=1)
    print("\n".join(out))


COUNTER_PAIR = {"bias_gelu_kernel": "bias + GELU", "copy_kernel": "copy probe"}


def counter_pair(frames: int) -> None:
    """bias + GELU on (frames * 1374, 4096) f16 with its fc1 bias, then the
    copy probe (one 16-byte vector per lane, streaming: the fastest shape)
    on the same bytes, each launched 8 times over 3 rotating buffer sets
    (more than the Infinity Cache holds): the workload of the op-against-
    probe counter comparison (rocprofv3 --pmc, one counter set per run)."""
    import torch

    from headshot_amd.context import HipContext

    ctx = HipContext("cuda:0")
    lib = load_ceiling()
    rows = frames * (GRID[0] * GRID[1] + PREFIX)
    g = torch.Generator(device="cpu").manual_seed(13)
    sets = [(torch.randn((rows, HIDDEN), generator=g).half().to(ctx.device),
             torch.empty((rows, HIDDEN), device=ctx.device, dtype=torch.float16))
            for _ in range(3)]
    bias = (torch.randn(HIDDEN, generator=g) * 0.02).to(ctx.device)
    stream = torch.cuda.current_stream().cuda_stream
    n16 = rows * HIDDEN * 2 // 16
    for i in range(8):
        x, o = sets[i % 3]
        ctx.bias_gelu(x, bias, out=o)
    torch.cuda.synchronize()
    for i in range(8):
        x, o = sets[i % 3]
        rc = lib.hsc_run(KINDS["copy"], CEILING_SHAPES["streaming x1"], x.data_ptr(), None,
                         o.data_ptr(), None, n16, 0, 0, stream)
        if rc != 0:
            raise RuntimeError(f"hsc_run(copy) returned {rc}")
    torch.cuda.synchronize()
    print(json.dumps({"counter_pair": "done", "rows": rows, "cols": HIDDEN}), flush=True)


def clock_trace(kind: str, frames: int) -> None:
    """The shader clock while kernels run (bench_ceiling.hip's hsc_clock: a
    one-wave sampler on a second stream records the shader-clock and 100 MHz
    real-time counters every 10 us; one-sample markers on the kernels' own
    stream delimit the phases). ``gelu``: bias + GELU on (frames * 1374,
    4096) f16 launched 16 times, its copy probe (one vector per lane,
    streaming) 16 times, GELU 16 times again, each launch between event
    pairs; ``pass``: 18 replays of the fused-op pass's graph. Prints one JSON
    line: per-phase launch times and clock (mean and minimum over 0.5 ms
    windows) and the clock per window."""
    import torch

    from headshot_amd.context import HipContext

    ctx = HipContext("cuda:0")
    lib = load_ceiling()
    dev = ctx.device
    main = torch.cuda.current_stream()
    step = 1000  # real-time ticks (10 us) between samples

    def clock(buf, n, st, stp):
        rc = lib.hsc_clock(buf.data_ptr(), n, stp, st.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"hsc_clock returned {rc}")

    phases = []  # (label, thunk, launches)
    if kind == "gelu":
        rows = frames * (GRID[0] * GRID[1] + PREFIX)
        nbytes = rows * HIDDEN * 4
        g = torch.Generator(device="cpu").manual_seed(13)
        sets = [(torch.randn((rows, HIDDEN), generator=g).half().to(dev),
                 torch.empty((rows, HIDDEN), device=dev, dtype=torch.float16))
                for _ in range(max(1, -(-ROTATE_BYTES // nbytes)))]
        bias = (torch.randn(HIDDEN, generator=g) * 0.02).to(dev)
        n16 = rows * HIDDEN * 2 // 16
        count = [0]

        def gelu():
            x, o = sets[count[0] % len(sets)]
            count[0] += 1
            ctx.bias_gelu(x, bias, out=o)

        def copy():
            x, o = sets[count[0] % len(sets)]
            count[0] += 1
            rc = lib.hsc_run(KINDS["copy"], CEILING_SHAPES["streaming x1"], x.data_ptr(), None,
                             o.data_ptr(), None, n16, 0, 0, main.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"hsc_run(copy) returned {rc}")

        phases = [("bias_gelu", gelu, 16), ("copy probe", copy, 16), ("bias_gelu", gelu, 16)]
        est_ms = 48 * nbytes / 4e9
        what = {"rows": rows, "cols": HIDDEN, "bytes_per_launch": nbytes}
    elif kind == "matrix":
        t = GRID[0] * GRID[1] + PREFIX
        g = torch.Generator(device="cpu").manual_seed(7)
        att = {}
        for name, (s_, tt) in {"global": (1, frames * t), "frame": (frames, t)}.items():
            q, k, v = (torch.randn((s_, HEADS, tt, HEAD_DIM), generator=g).half().to(dev)
                       for _ in range(3))
            o = torch.empty((s_ * tt, HEADS * HEAD_DIM), dtype=torch.float16, device=dev)
            ctx.attention_merged(q, k, v, out=o)
            att[name] = (ctx.last_launch, 4.0 * tt * tt * HEAD_DIM * s_ * HEADS, (q, k, v, o))
        m = frames * t
        x = torch.randn((m, DIM), generator=g).half().to(dev)
        w = (torch.randn((HIDDEN, DIM), generator=g) / DIM ** 0.5).half().to(dev)
        bias = (torch.randn(HIDDEN, generator=g) * 0.02).to(dev)
        o1 = torch.empty((m, HIDDEN), dtype=torch.float16, device=dev)
        ctx.linear(x, w, bias, out=o1)
        fc1 = ctx.last_launch
        ctx.linear_gelu(x, w, bias, out=o1)
        fc1_gelu = ctx.last_launch
        lin_flops = 2.0 * m * HIDDEN * DIM
        phases = [("global attention", att["global"][0], 6), ("frame attention", att["frame"][0], 40),
                  ("fc1, bias", fc1, 40), ("fc1 + GELU", fc1_gelu, 40)]
        flops = {"global attention": att["global"][1], "frame attention": att["frame"][1],
                 "fc1, bias": lin_flops, "fc1 + GELU": lin_flops}
        est_ms = 6 * 9.0 + 40 * 0.4 + 80 * 0.5
        what = {"tokens": m}
    else:
        b = Pass(ctx, frames, torch.float16, distinct=True)
        b.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            b.run()
        graph.replay()
        torch.cuda.synchronize()
        phases = [("pass", graph.replay, 18)]
        est_ms = 18 * b.pass_bytes / 4e9
        what = {"pass_bytes": b.pass_bytes}
    for _, fn, _ in phases:
        fn()
    torch.cuda.synchronize()
    n = int((est_ms + 20.0) * 100)  # samples, 10 us apart
    samples = torch.zeros(2 * n, dtype=torch.int64, device=dev)
    marks = torch.zeros(2 * (len(phases) + 1), dtype=torch.int64, device=dev)
    side = torch.cuda.Stream(device=dev)
    clock(samples, n, side, step)
    torch.cuda._sleep(5_000_000)
    events = []
    for i, (label, fn, k) in enumerate(phases):
        clock(marks[2 * i:], 1, main, 0)
        evs = []
        for _ in range(k):
            a, e = KernelEvent(), KernelEvent()
            a.record()
            fn()
            e.record()
            evs.append((a, e))
        events.append(evs)
    clock(marks[2 * len(phases):], 1, main, 0)
    torch.cuda.synchronize()
    sm = samples.cpu().view(-1, 2).tolist()
    mk = [r for _, r in marks.cpu().view(-1, 2).tolist()]
    t0 = sm[0][1]
    w = 50  # samples per 0.5 ms window
    windows = []
    for i in range(0, n - w, w):
        (c0, r0), (c1, r1) = sm[i], sm[i + w]
        windows.append(((r0 + r1) / 2, (c1 - c0) / ((r1 - r0) / 100.0)))
    out_phases = []
    for i, (label, _, k) in enumerate(phases):
        inside = [mhz for r, mhz in windows if mk[i] <= r < mk[i + 1]]
        us = [round(a.elapsed_time(e) * 1e3, 1) for a, e in events[i]]
        entry = {"phase": label, "launches": k, "start_ms": round((mk[i] - t0) / 1e5, 2),
                 "end_ms": round((mk[i + 1] - t0) / 1e5, 2), "launch_us": us,
                 "clock_mhz_mean": round(sum(inside) / len(inside)) if inside else None,
                 "clock_mhz_min": round(min(inside)) if inside else None}
        if kind == "matrix" and inside:
            # the phase's rate against the dense f16 peak (quoted at 2.4
            # GHz) and against that peak scaled to the clock it ran at
            tf = flops[label] / (sum(us) / len(us) * 1e-6) / 1e12
            at_clock = MFMA_PEAK_TFLOPS * entry["clock_mhz_mean"] / 2400.0
            entry.update({"TFLOP/s": round(tf, 1), "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                          "peak_at_clock_TFLOP/s": round(at_clock, 1),
                          "frac_at_clock": round(tf / at_clock, 4)})
        out_phases.append(entry)
    print(json.dumps({"clock_trace": kind, "frames": frames, **what, "phases": out_phases,
                      "clock_mhz_per_0.5ms": [[round((r - t0) / 1e5, 2), round(m)]
                                              for r, m in windows]}), flush=True)


def summarize_pair(paths) -> None:
    """Mean per dispatch of every counter in the --counter-pair CSVs for the
    op and the probe, their ratio, and the kernel-trace duration; derived:
    memory instructions in flight per busy cycle (SQ_INST_LEVEL_VMEM /
    SQ_BUSY_CYCLES) and wave cycles per wave."""
    import csv
    import statistics as st
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))
    dur = defaultdict(list)
    for path in paths:
        for r in csv.DictReader(open(path)):
            who = next((v for k, v in COUNTER_PAIR.items() if k in r["Kernel_Name"]), None)
            if who is None:
                continue
            vals[who][r["Counter_Name"]].append(float(r["Counter_Value"]))
            dur[who].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    op, probe = COUNTER_PAIR.values()
    if not vals[op] or not vals[probe]:
        print("no bias_gelu_kernel / copy_kernel dispatches in these CSVs")
        return
    a = {k: st.mean(v) for k, v in vals[op].items()}
    b = {k: st.mean(v) for k, v in vals[probe].items()}
    out = [f"| counter | {op} | {probe} | {op} / {probe} |", "|---|---|---|---|",
           f"| duration under the profiler (us) | {st.mean(dur[op]):.1f} | {st.mean(dur[probe]):.1f} "
           f"| {st.mean(dur[op]) / st.mean(dur[probe]):.3f} |"]
    for k in sorted(set(a) & set(b)):
        ratio = f"{a[k] / b[k]:.3f}" if b[k] else "-"
        out.append(f"| {k} | {a[k]:.4g} | {b[k]:.4g} | {ratio} |")
    derived = [("SQ_INST_LEVEL_VMEM / SQ_BUSY_CYCLES", "SQ_INST_LEVEL_VMEM", "SQ_BUSY_CYCLES"),
               ("SQ_WAVE_CYCLES / SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_WAVES")]
    for name, num, den in derived:
        if all(x in a and x in b for x in (num, den)) and a[den] and b[den]:
            ra, rb = a[num] / a[den], b[num] / b[den]
            out.append(f"| {name} | {ra:.4g} | {rb:.4g} | {ra / rb:.3f} |")
    print("\n".join(out))


def main():
    args = parse()
    if args.summarize:
        summarize(args)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.summarize_pair:
        summarize_pair(args.summarize_pair)
        return
    if args.clock_trace:
        clock_trace(args.clock_trace, args.frames)
        return
    if args.counter_pair:
        counter_pair(args.frames)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU: the fused per-layer ops are "
                                   "row-local and shard by frames with no exchange, so the "
                                   "figure that matters is one GPU's; run with --gpus 1"}))
        sys.exit(2)
    import torch

    from headshot_amd.context import HipContext

    dtype = torch.float16 if args.dtype == "f16" else torch.float32
    ctx = HipContext("cuda:0")
    bench = Pass(ctx, args.frames, dtype, distinct=not args.shared_inputs, fuse=args.fuse_layernorm)
    torch.cuda.synchronize()

    # HBM counter calibration: one plain copy of known size (outside timing).
    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        a = torch.ones(n, device=ctx.device, dtype=torch.float32)
        b_ = torch.empty_like(a)
        b_.copy_(a)
        torch.cuda.synchronize()
        del a, b_

    for _ in range(args.warmup):
        bench.run()
    torch.cuda.synchronize()

    launch = "eager"
    graph = None
    if not args.eager:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                bench.run()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            launch = "hip_graph"
        except Exception as exc:  # capture unsupported: time eager launches
            print(f"graph capture failed ({exc}); timing eager launches", file=sys.stderr)
            graph = None

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            bench.run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps

    per_op, per_op_cold, roofline, ops_ms, ceilings, pass_cold = {}, None, None, None, None, None
    workloads = None
    if args.op_passes > 0:
        per_op = op_rates(bench, per_op_times(bench, args.op_passes))
        flush = cache_flusher(ctx.device)
        per_op_cold = op_rates(bench, per_op_times(bench, args.op_passes, flush=flush))
        if not args.no_ceilings:
            ceilings = ceiling_times(bench, per_op, per_op_cold, flush)
            if "bias_gelu" in ceilings:
                pus = gelu_in_pass_probe_us(bench, args.op_passes)
                if pus:
                    ceilings["bias_gelu"]["in_pass_probe_us"] = round(pus, 2)
                    ceilings["bias_gelu"]["op_frac_of_in_pass_probe"] = round(
                        pus / per_op["bias_gelu"]["us"], 4)
        pass_cold = pass_from_ops(bench, per_op_cold)
        if not args.no_workloads:
            workloads = workload_legs(ctx, args.op_passes, flush)
        del flush
        ops_ms = round(sum(per_op[op]["us"] * bench.launches[op] for op in bench.ops) / 1e3, 3)
        dominant = max(bench.ops, key=lambda op: per_op[op]["us"] * bench.launches[op])
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": per_op[dominant]["GB/s"],
                    "peak": PEAK_GBS, "unit": "GB/s", "frac": per_op[dominant]["frac"],
                    "traffic": None}
        traffic = load_traffic(dominant, args.frames, args.dtype)
        if traffic is not None:
            roofline["traffic"] = traffic["bytes_per_launch"]
            roofline["traffic_source"] = traffic["source"]
    value = bench.pass_bytes / (ms * 1e-3) / 1e9
    sequences = None
    if args.op_passes > 0:
        this = {"fused_layernorm": args.fuse_layernorm, "launches": sum(bench.launches.values()),
                "ms": round(ms, 3), "pass_bytes": bench.pass_bytes,
                "GB/s": round(value, 1), "frac": round(value / PEAK_GBS, 4)}
        other = sequence_pass(ctx, args.frames, dtype, not args.shared_inputs, args.steps,
                              fuse=not args.fuse_layernorm)
        sequences = {"six_op": other if args.fuse_layernorm else this,
                     "fused_layernorm": this if args.fuse_layernorm else other}

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic: torch seeded N(0,1) activations/GEMM outputs, random-init params "
                "(LN gamma N(1,.02), beta/biases/pos N(0,.02), LayerScale 1e-5)",
        "config": {"workload": f"aggregator fused-op pass: assembly + {N_FRAME_BLOCKS} frame + "
                               f"{N_GLOBAL_BLOCKS} global blocks",
                   "block_inputs": "shared" if args.shared_inputs else "per block",
                   "block_sequence": ("4 ops (LayerScale + residual fused with the LayerNorm after it)"
                                      if args.fuse_layernorm else
                                      "6 ops (LN1, QK-norm pair, LS1, LN2, GELU, LS2)"),
                   "frames": args.frames, "tokens_per_frame": bench.t, "dim": DIM,
                   "heads": HEADS, "head_dim": HEAD_DIM, "hidden": HIDDEN, "prefix": PREFIX,
                   "grid": f"{GRID[0]}x{GRID[1]}", "eps": EPS, "launch": launch},
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "pass_bytes": bench.pass_bytes,
        "tokens_per_s": round(bench.rows / (ms * 1e-3), 1),
        "ops_ms_per_step": ops_ms,
        "pass_cold": pass_cold,
        "ms_per_pass_fused_layernorm": (sequences or {}).get("fused_layernorm", {}).get("ms"),
        "sequences": sequences,
        "ops": per_op,
        "ops_cold": per_op_cold,
        "ceilings": ceilings,
        "roofline": roofline,
        "workloads": workloads,
    }
    if args.attention_iters > 0:
        line["attention"] = attention_times(ctx, args.frames, args.attention_iters)
        flush = cache_flusher(ctx.device)
        # the HBM legs run ~0.1 ms a launch: at least 20 timed launches each
        hbm_iters = max(20, args.attention_iters)
        line["cache_build"] = cache_times(ctx, args.frames, hbm_iters, flush)
        line["surface"] = surface_times(ctx, args.frames, hbm_iters, flush)
        del flush
        line["linear"] = gemm_times(ctx, args.frames, args.attention_iters)
        line["block"] = block_times(ctx, args.frames, max(1, args.attention_iters // 2))
        line["f32_s2"] = f32_block_times(ctx, args.attention_iters)
        trunk_iters = args.trunk_iters if args.trunk_iters >= 0 else max(1, args.attention_iters // 5)
        if trunk_iters > 0:
            line["trunk"] = trunk_times(ctx, args.frames, trunk_iters)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(ctx, args.cpu_seconds)
        legs = {"pass_sample": cpu_pass_sample(bench, args.cpu_seconds / 2)}
        if args.attention_iters > 0:
            legs.update(cpu_baseline_legs(args.frames))
        line["cpu_baseline_legs"] = legs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
