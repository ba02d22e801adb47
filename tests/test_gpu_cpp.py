"""Runs the C++ kernel tests (tests/cpp/kernels.cpp, built by
tests/cpp/build.py / __graft_entry__.build()) — the reference's GPU kernel
tests restated over the C++ host surface include/headshot_hip.hpp."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "hs_kernel_tests")


def test_cpp_kernel_tests():
    assert os.path.exists(BIN), "build tests/cpp/hs_kernel_tests first (tests/cpp/build.py)"
    proc = subprocess.run([BIN], capture_output=True, text=True, timeout=100)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "0 failed" in proc.stdout
