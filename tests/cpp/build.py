"""Build tests/cpp/hs_kernel_tests (C++ kernel tests over include/headshot_hip.hpp).

Links headshot_amd/libheadshot_hip.so with an rpath relative to the binary,
so the test runs from any checkout location.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "hs_kernel_tests")


def build() -> str:
    hipcc = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
    cmd = [hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
           f"-I{os.path.join(ROOT, 'include')}", os.path.join(HERE, "kernels.cpp"),
           f"-L{os.path.join(ROOT, 'headshot_amd')}", "-lheadshot_hip",
           "-Wl,-rpath,$ORIGIN/../../headshot_amd", "-o", OUT + ".tmp"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"C++ test build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(), file=sys.stderr)
