"""In-tree build of the gfx950 kernel library and its C++ consumers.

Outputs (git-ignored, shipped with the tree to the GPU box):
  flash_kmeans_cuda/libfkc.so                 C-ABI library (include/fkc.h)
  flash_kmeans_cuda/libflash_kmeans_cuda.so   libtorch fkc:: API on top of it
  flash_kmeans_cuda/bin/fkc_cpp_smoke         C++ smoke test of the fkc:: API

  _cmake/install/                             CMake install/export package
                                              (cmake --install of CMakeLists.txt)
  _cmake/consumer/consumer_smoke              C++ consumer built against it

Usage: python flash-kmeans-cuda_amd/build.py [--only capi|torch|cmake|all] [-j N]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
PKG = os.path.join(HERE, "flash_kmeans_cuda")
OBJ = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]

# Extra flags per source.  assign_mfma.hip: its running maxima are fmaxf
# chains over matrix-core results; with NaNs honoured the compiler must quiet
# every operand first (one extra v_max per score), which nearly doubles the
# kernel's vector-ALU work.  Scores are NaN only for NaN inputs, whose labels
# are unspecified anyway.
SOURCE_FLAGS = {"assign_mfma.hip": ["-fno-honor-nans"]}

KERNEL_SOURCES = [
    "assign_mfma.hip",
    "assign_valu.hip",
    "label_sort.hip",
    "update.hip",
    "finalize.hip",
    "quality.hip",
    "capi_noalloc.hip",
]
HOST_SOURCES = ["capi.cpp"]


def _run(cmd: list[str], quiet: bool = False) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n"
                           f"{' '.join(cmd)}\n{proc.stdout}\n{err}")
    if err.strip() and not quiet:
        sys.stderr.write(err + "\n")


def _compile(src: str) -> str:
    os.makedirs(OBJ, exist_ok=True)
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    _run([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), *lang, "-c", path,
          "-o", out])
    return out


def build_capi(jobs: int) -> str:
    srcs = KERNEL_SOURCES + HOST_SOURCES
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    lib = os.path.join(PKG, "libfkc.so")
    tmp = lib + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs,
          "-o", tmp])
    os.replace(tmp, lib)
    return lib


def _torch_paths() -> tuple[list[str], str]:
    import torch
    root = os.path.dirname(torch.__file__)
    incs = [os.path.join(root, "include"),
            os.path.join(root, "include", "torch", "csrc", "api", "include")]
    return incs, os.path.join(root, "lib")


def build_torch_api() -> list[str]:
    """libtorch fkc:: API (flash_kmeans_cuda.h) and its C++ smoke test."""
    incs, tlib = _torch_paths()
    api_dir = os.path.join(HERE, "torch_api")
    cxx = shutil.which("g++") or "g++"
    common = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__",
              "-DUSE_ROCM", "-D_GLIBCXX_USE_CXX11_ABI=1",
              "-I", INCLUDE, "-I", api_dir, "-I", os.path.join(ROCM, "include")]
    for i in incs:
        common += ["-isystem", i]
    # torch's libraries come first in DT_NEEDED so that torch's own HIP
    # runtime (file libamdhip64.so, soname libamdhip64.so.7) is mapped before
    # libfkc.so asks for libamdhip64.so.7: the loader then reuses it instead of
    # mapping a second HIP runtime from /opt/rocm.  Nothing here links the HIP
    # runtime directly.
    torch_libs = ["-L", tlib, "-Wl,-rpath," + tlib, "-Wl,--no-as-needed",
                  "-lc10_hip", "-ltorch_hip", "-lc10", "-ltorch_cpu", "-ltorch"]
    lib = os.path.join(PKG, "libflash_kmeans_cuda.so")
    _run([cxx, *common, "-shared", os.path.join(api_dir, "api.cpp"),
          "-o", lib + ".tmp", *torch_libs, "-L", PKG, "-Wl,-rpath,$ORIGIN",
          "-lfkc"])
    os.replace(lib + ".tmp", lib)
    bindir = os.path.join(PKG, "bin")
    os.makedirs(bindir, exist_ok=True)
    exe = os.path.join(bindir, "fkc_cpp_smoke")
    _run([cxx, *common, os.path.join(HERE, "cpp_tests", "smoke.cpp"),
          "-o", exe + ".tmp", *torch_libs, "-L", PKG,
          "-Wl,-rpath,$ORIGIN/..", "-lflash_kmeans_cuda", "-lfkc"])
    os.replace(exe + ".tmp", exe)
    return [lib, exe]


CMAKE_DIR = os.path.join(HERE, "_cmake")


def build_cmake_package(jobs: int) -> list[str]:
    """The CMake install/export package (CMakeLists.txt) into _cmake/install,
    then the installed-package consumer (cpp_tests/consumer) against it."""
    import torch
    cmake = shutil.which("cmake")
    if cmake is None:
        raise RuntimeError("cmake not found")
    gen = ["-G", "Ninja"] if shutil.which("ninja") else []
    prefix = f"{torch.utils.cmake_prefix_path};{ROCM}"
    bdir = os.path.join(CMAKE_DIR, "build")
    inst = os.path.join(CMAKE_DIR, "install")
    cons = os.path.join(CMAKE_DIR, "consumer")
    # (Torch's CMake config prints warnings on every configure: quiet.)
    _run([cmake, "-S", HERE, "-B", bdir, *gen, "-DCMAKE_BUILD_TYPE=Release",
          f"-DCMAKE_PREFIX_PATH={prefix}"], quiet=True)
    _run([cmake, "--build", bdir, "-j", str(max(1, jobs))], quiet=True)
    _run([cmake, "--install", bdir, "--prefix", inst], quiet=True)
    _run([cmake, "-S", os.path.join(HERE, "cpp_tests", "consumer"), "-B", cons, *gen,
          "-DCMAKE_BUILD_TYPE=Release", f"-DCMAKE_PREFIX_PATH={inst};{prefix}"], quiet=True)
    _run([cmake, "--build", cons, "-j", str(max(1, jobs))], quiet=True)
    return [inst, os.path.join(cons, "consumer_smoke")]


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=["capi", "torch", "cmake", "all"], default="all")
    ap.add_argument("-j", "--jobs", type=int,
                    default=min(8, os.cpu_count() or 1))
    args = ap.parse_args(argv)
    if args.only in ("capi", "all"):
        print(build_capi(args.jobs))
    if args.only in ("torch", "all"):
        for p in build_torch_api():
            print(p)
    if args.only in ("cmake", "all"):
        for p in build_cmake_package(args.jobs):
            print(p)
    return 0


if __name__ == "__main__":
    sys.exit(main())
