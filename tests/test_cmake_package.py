"""The CMake install/export package, built from scratch on the CPU: configure
and build flash-kmeans-cuda_amd/CMakeLists.txt, `cmake --install` it into a
temporary prefix, then configure and build the consumer project
(cpp_tests/consumer) against that prefix alone, as the reference's
tests/cpp/consumer does for its package (CMakeLists.txt:99-125).  Running
the consumer needs a GPU (tests/test_gpu_cpp_smoke.py runs the in-tree
build of it)."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "flash-kmeans-cuda_amd")


def _run(cmd, **kw):
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=900, **kw)
    assert proc.returncode == 0, " ".join(cmd) + "\n" + proc.stdout[-3000:] + proc.stderr[-3000:]
    return proc


@pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not installed")
def test_install_tree_and_consumer_build(tmp_path):
    import torch
    gen = ["-G", "Ninja"] if shutil.which("ninja") else []
    prefix = f"{torch.utils.cmake_prefix_path};/opt/rocm"
    bdir, inst, cons = tmp_path / "build", tmp_path / "install", tmp_path / "consumer"
    _run(["cmake", "-S", PKG, "-B", str(bdir), *gen, "-DCMAKE_BUILD_TYPE=Release",
          f"-DCMAKE_PREFIX_PATH={prefix}"])
    _run(["cmake", "--build", str(bdir), "-j", "8"])
    _run(["cmake", "--install", str(bdir), "--prefix", str(inst)])
    cfgdir = inst / "lib" / "cmake" / "flash_kmeans_cuda"
    for f in ["flash_kmeans_cudaConfig.cmake", "flash_kmeans_cudaConfigVersion.cmake",
              "flash_kmeans_cudaTargets.cmake"]:
        assert (cfgdir / f).exists(), f
    assert (inst / "include" / "fkc.h").exists()
    assert (inst / "include" / "flash_kmeans_cuda" / "flash_kmeans_cuda.h").exists()
    assert (inst / "lib" / "libfkc.so").exists() and (inst / "lib" / "libflash_kmeans_cuda.so").exists()
    targets = (cfgdir / "flash_kmeans_cudaTargets.cmake").read_text()
    assert "flash_kmeans_cuda::flash_kmeans_cuda" in targets and "flash_kmeans_cuda::fkc" in targets
    # the consumer sees only the install prefix (plus torch and ROCm)
    _run(["cmake", "-S", os.path.join(PKG, "cpp_tests", "consumer"), "-B", str(cons), *gen,
          "-DCMAKE_BUILD_TYPE=Release", f"-DCMAKE_PREFIX_PATH={inst};{prefix}"])
    _run(["cmake", "--build", str(cons)])
    exe = cons / "consumer_smoke"
    assert exe.exists()
    # installed library resolves libfkc next to itself
    dyn = _run(["readelf", "-d", str(inst / "lib" / "libflash_kmeans_cuda.so")]).stdout
    assert "$ORIGIN" in dyn and "libfkc.so" in dyn
