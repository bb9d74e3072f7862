"""Runs the C++ smoke test of the libtorch fkc:: API (the counterpart of the
reference's tests/cpp/smoke.cpp) as a child process on the GPU."""

from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(REPO, "flash-kmeans-cuda_amd", "flash_kmeans_cuda", "bin", "fkc_cpp_smoke")


def test_cpp_smoke_binary():
    assert os.path.exists(EXE), "build it with flash-kmeans-cuda_amd/build.py"
    proc = subprocess.run([EXE], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "C++ smoke test passed" in proc.stdout
    assert "update/finalize D=257 passed" in proc.stdout
