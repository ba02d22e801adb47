"""bench.py's contract on the CPU: the one-GPU rule, the algorithmic byte
counts its rates divide by, and the kernel names its rocprofv3 summaries
group by."""
import json
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_algorithmic_bytes_per_token():
    rows, patches = 32 * 1374, 32 * 1369
    b = bench.op_bytes(rows, 2, patches, 1369)
    assert b["layernorm"] == rows * 4096             # 2048 R + 2048 W
    assert b["qknorm_rope"] == rows * 8192           # q and k in one launch
    assert b["bias_gelu"] == rows * 16384            # hidden 4096, 1R + 1W
    assert b["bias_ls_residual"] == rows * 6144      # 2R + 1W
    assert b["assemble"] == patches * 4096 + 1369 * 4096 + rows * 2048
    per_block = (2 * b["layernorm"] + b["qknorm_rope"] + 2 * b["bias_ls_residual"]
                 + b["bias_gelu"])
    assert per_block == rows * 45056
    # f32 storage doubles every activation term (the f32 patches and table stay)
    b32 = bench.op_bytes(rows, 4, patches, 1369)
    assert b32["layernorm"] == 2 * b["layernorm"]
    assert b32["assemble"] == patches * 4096 + 1369 * 4096 + rows * 4096


def test_kernel_names_map_to_ops():
    names = {
        "_ZN2hs12_GLOBAL__N_113ln_vec_kernelIDF16_Li2ELi2EEEvPKT_PKfS6_PS2_lf": "layernorm",
        "_ZN2hs12_GLOBAL__N_114qkn_row_kernelIDF16_Li16ELb1ELb1ELi2EEEvNS0_10QknTensorsIT_EEPKfS6_liif":
            "qknorm_rope",
        "_ZN2hs12_GLOBAL__N_114bias_ls_kernelIDF16_Lb1ELi1EEEvPKT_S4_PKfS6_PS2_li":
            "bias_ls_residual",
        "_ZN2hs12_GLOBAL__N_116bias_gelu_kernelIDF16_Lb1ELi1EEEvPKT_PKfPS2_li": "bias_gelu",
        "_ZN2hs12_GLOBAL__N_115assemble_kernelIDF16_fLi4ELi4EEEvPKT0_PKfS6_PKT_S9_PS7_iiiii":
            "assemble",
        "_ZN2hs12_GLOBAL__N_116flash_f16_kernelEPKDF16_S2_S2_PDF16_iiiifi": None,
        "__amd_rocclr_copyBuffer": None,
    }
    for name, op in names.items():
        assert bench.kernel_op(name) == op, name


def test_host_threads_uses_the_visible_cores_within_the_share(monkeypatch):
    visible = len(os.sched_getaffinity(0))
    monkeypatch.delenv("OMP_NUM_THREADS", raising=False)
    assert bench.host_threads() == (visible, visible)
    monkeypatch.setenv("OMP_NUM_THREADS", "1")
    assert bench.host_threads() == (1, visible)
    monkeypatch.setenv("OMP_NUM_THREADS", str(visible + 100))
    assert bench.host_threads() == (visible, visible)


def test_ceiling_probes_cover_every_op():
    assert set(bench.CEILING_PROBES) == set(bench.OPS)
    # every probe kernel serves an op of the pass, or the cache build (widen)
    # or the in-place rope_apply (inplace) legs
    used = {probe for probe, _ in bench.CEILING_PROBES.values()} | {"widen", "inplace"}
    assert used == set(bench.KINDS)


def test_pass_launches_count_each_op_of_the_sequence():
    fused = bench.pass_launches(24, 24, fuse=True)
    unfused = bench.pass_launches(24, 24)
    assert sum(fused.values()) == 1 + 4 * 48 + 1, fused  # 4 per block, + assembly, + LN1
    assert sum(unfused.values()) == 1 + 6 * 48, unfused
    # each fused LayerScale + LayerNorm pair skips the LayerNorm's re-read of
    # the row the LayerScale wrote: 1024 f16 = 2048 B per token
    b = bench.op_bytes(100, 2, 0, 0)
    per = lambda l: sum(b[k] * v for k, v in l.items() if k != "assemble")  # noqa: E731
    assert per(unfused) - per(fused) == 95 * 100 * 1024 * 2


def test_ceiling_library_exports_its_entry_point():
    import ctypes

    if not os.path.exists(bench.CEILING_LIB):
        bench.build_ceiling()
    lib = ctypes.CDLL(bench.CEILING_LIB)
    assert hasattr(lib, "hsc_run")
    # argument checks run on the host, before any launch
    run = bench.load_ceiling().hsc_run
    assert run(7, 0, None, None, None, None, 0, 0, 0, None) == -1    # unknown kind
    assert run(0, 8, None, None, None, None, 0, 0, 0, None) == -1    # unknown shape
    assert run(0, -1, None, None, None, None, 0, 0, 0, None) == -1   # unknown shape
    assert run(3, 1, None, None, None, None, 6, 0, 0, None) == -1    # cast needs n % 4 == 0
    assert run(0, 0, None, None, None, None, -1, 0, 0, None) == -1   # negative size
    assert run(2, 1, None, None, None, None, 0, 0, 5, None) == 0     # empty: no launch
    assert run(0, 3, None, None, None, None, 0, 0, 0, None) == 0     # empty: no launch


def test_summarize_counters_stall_table(tmp_path, capsys):
    """The counter summary adds the stall table when a pass collected the
    SQ_WAIT counters: shares are quad-cycle counts over SQ_WAVE_CYCLES."""
    head = "Kernel_Name,Grid_Size,Counter_Name,Counter_Value,Start_Timestamp,End_Timestamp\n"
    name = "void hs::(anonymous namespace)::flash_f16_kernel(x)"
    rows = [("SQ_INSTS_MFMA", 100), ("SQ_INSTS_VALU", 800), ("SQ_VALU_MFMA_BUSY_CYCLES", 3200),
            ("GRBM_GUI_ACTIVE", 8000), ("SQ_WAVE_CYCLES", 512000), ("SQ_WAIT_ANY", 128000),
            ("SQ_WAIT_INST_ANY", 204800), ("SQ_WAIT_INST_LDS", 25600)]
    path = tmp_path / "c.csv"
    path.write_text(head + "".join(f'"{name}",4096,{k},{v},0,1000\n' for k, v in rows))
    bench.summarize_counters([str(path)])
    out = capsys.readouterr().out
    # 1000 cycles per XCD, 1024 SIMDs: 4 x 512000 quad-cycles = 2 waves per SIMD
    assert "| flash_f16_kernel | 4096 | 2.00 | 25.0% | 40.0% | 5.0% |" in out


def test_summarize_pair_ratios(tmp_path, capsys):
    """The op-against-probe counter table: per-dispatch means, the ratio,
    durations from the timestamps, and the derived in-flight and per-wave
    figures; other kernels in the CSV are ignored."""
    head = "Kernel_Name,Grid_Size,Counter_Name,Counter_Value,Start_Timestamp,End_Timestamp\n"
    gelu = "void hs::(anonymous namespace)::bias_gelu_kernel<_Float16, true, 1>(x)"
    copy = "void (anonymous namespace)::copy_kernel<true, 1>(x)"
    other = "void hs::(anonymous namespace)::ln_vec_kernel<_Float16, 2, 2>(x)"
    lines = []
    for name, scale, ns in ((gelu, 2.0, 120000), (copy, 1.0, 110000), (other, 9.0, 5000)):
        for k, v in (("SQ_WAVES", 10), ("SQ_WAVE_CYCLES", 100), ("SQ_BUSY_CYCLES", 5),
                     ("SQ_INST_LEVEL_VMEM", 20)):
            lines += [f'"{name}",4096,{k},{v * scale},0,{ns}\n'] * 2
    path = tmp_path / "p.csv"
    path.write_text(head + "".join(lines))
    bench.summarize_pair([str(path)])
    out = capsys.readouterr().out
    assert "| duration under the profiler (us) | 120.0 | 110.0 | 1.091 |" in out
    assert "| SQ_INST_LEVEL_VMEM | 40 | 20 | 2.000 |" in out
    assert "| SQ_INST_LEVEL_VMEM / SQ_BUSY_CYCLES | 4 | 4 | 1.000 |" in out
    assert "| SQ_WAVE_CYCLES / SQ_WAVES | 10 | 10 | 1.000 |" in out
