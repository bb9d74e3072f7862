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
    assert "0 failed" in proc.stdout and "lloyd: 5 iterations" in proc.stdout


CONSUMER = os.path.join(REPO, "flash-kmeans-cuda_amd", "_cmake", "consumer", "consumer_smoke")


def test_installed_package_consumer():
    """The consumer built against the CMake install tree (find_package
    flash_kmeans_cuda CONFIG, target flash_kmeans_cuda::flash_kmeans_cuda):
    nearest-centroid labels against exact fp64 distances, a 5-iteration
    Lloyd run, one HIP runtime in the process."""
    assert os.path.exists(CONSUMER), "build it with flash-kmeans-cuda_amd/build.py"
    proc = subprocess.run([CONSUMER], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "installed package works" in proc.stdout
    assert "hip_runtimes=1" in proc.stdout
