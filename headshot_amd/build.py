"""Build libheadshot_hip.so (hipcc --offload-arch=gfx950) in-tree.

``python -m headshot_amd.build`` or ``headshot_amd.build.build()``. Objects
go to ``headshot_amd/_build/``; the library lands next to this file so it
travels with the source tree. Always recompiles (the build check is meant
to exercise the compiler).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libheadshot_hip.so")

ARCH = os.environ.get("HS_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

HIP_SOURCES = [
    "hs_runtime.hip",
    "hs_norm.hip",
    "hs_qknorm_rope.hip",
    "hs_elementwise.hip",
    "hs_assemble.hip",
    "hs_attention.hip",
    "hs_cache.hip",
    "hs_gemm.hip",
]
# Host-only C++ (bit-exact RoPE tables): no FMA contraction.
CXX_SOURCES = ["hs_rope_tables.cpp"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed FP32 (v_pk_*_f32) code generation stays off.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
# Per-source additions. Attention: MFMA accumulators in ordinary VGPRs (the
# default AGPR form costs a copy of every score and output accumulator per
# key tile), and no NaN-quieting canonicalisation around fmaxf in the
# softmax max (NaN inputs give NaN-polluted output either way).
SOURCE_FLAGS = {
    "hs_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
}
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall",
             f"-I{INCLUDE}"]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    err = "\n".join(line for line in proc.stderr.splitlines()
                    if "packed-fp32-ops" not in line and line.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{proc.stdout}\n{err}")
    return err


def build(verbose: bool = False, defines=(), lib_path: str = LIB, build_dir: str = BUILD) -> str:
    """Compile every source and link ``lib_path``. ``defines`` (``NAME=VALUE``
    strings) override the kernels' launch-shape constants."""
    os.makedirs(build_dir, exist_ok=True)
    dflags = [f"-D{d}" for d in defines]
    jobs = []
    for src in HIP_SOURCES:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        jobs.append([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), *dflags, "-c",
                     os.path.join(CSRC, src), "-o", obj])
    for src in CXX_SOURCES:
        obj = os.path.join(build_dir, src.replace(".cpp", ".o"))
        jobs.append(["g++", *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as pool:
        for msg in pool.map(_run, jobs):
            if msg and verbose:
                print(msg, file=sys.stderr)
    objs = [j[-1] for j in jobs]
    tmp = lib_path + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, lib_path)
    return lib_path


if __name__ == "__main__":
    print(build(verbose=True))
