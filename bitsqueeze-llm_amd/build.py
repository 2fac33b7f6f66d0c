"""Builds the MI355X (gfx950) bitsqz_llm library in-tree.

    python bitsqueeze-llm_amd/build.py        # -> bitsqueeze-llm_amd/lib/libbitsqz_llm_lib.so
    python bitsqueeze-llm_amd/build.py --package   # + the installed CMake package under _install/

Every HIP source under csrc/ is compiled with hipcc for gfx950 into an object
under _build/, and the objects are linked into one shared library whose
SONAME matches the reference's installed library (libbitsqz_llm_lib.so.0).
The exported symbols are the nine C++-linkage functions of
include/bitsqz_llm.hpp, topk_compute_num_topk_columns and the extern "C"
functions of include/bitsqz_llm_c.h; everything else is hidden.
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
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libbitsqz_llm_lib.so")
ARCH = os.environ.get("BSQ_OFFLOAD_ARCH", "gfx950")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", f"--offload-arch={ARCH}",
    # no packed FP32 math (v_pk_*_f32) anywhere
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wno-unused-command-line-argument",
]
# Sources whose arithmetic must round operation by operation (bit-exact codecs).
NO_CONTRACT = {"quant.hip", "topk.hip", "runtime.hip", "recon.hip", "legacy.hip"}
# Per-file extra flags: the register-resident FP64 factorisations need their
# fully unrolled loops kept unrolled so the per-thread matrix stays in VGPRs.
EXTRA = {"linalg.hip": ["-mllvm", "-pragma-unroll-threshold=200000"],
         "chol.hip": ["-mllvm", "-pragma-unroll-threshold=200000"],
         "sytrd.hip": ["-mllvm", "-pragma-unroll-threshold=200000"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    flags = list(COMMON)
    if os.path.basename(src) in NO_CONTRACT:
        flags.append("-ffp-contract=off")
    flags += EXTRA.get(os.path.basename(src), [])
    cmd = [hipcc(), *flags, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


INSTALL = os.path.join(HERE, "_install")
CMAKE_BUILD = os.path.join(BUILD, "cmake")
CONSUMER_SRC = os.path.join(ROOT, "tests", "cmake_consumer")
CONSUMER_BUILD = os.path.join(CONSUMER_SRC, "_build")
CONSUMER_BIN = os.path.join(CONSUMER_BUILD, "bsq_consumer")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"failed: {' '.join(cmd)}\n{r.stdout[-4000:]}\n{r.stderr[-4000:]}")


def package(verbose: bool = True) -> str:
    """The installed CMake package (CMakeLists.txt beside this file): builds
    the same sources into libbitsqz_llm_lib.so.0.1.0 and installs it, the
    headers and bitsqz_llmConfig.cmake under _install/; then builds the
    downstream test program tests/cmake_consumer against that installed
    package with find_package(bitsqz_llm CONFIG)."""
    cmake = shutil.which("cmake")
    if not cmake:
        raise RuntimeError("cmake not found")
    jobs = str(max(1, min(8, os.cpu_count() or 1)))
    _run([cmake, "-S", HERE, "-B", CMAKE_BUILD, f"-DCMAKE_INSTALL_PREFIX={INSTALL}", "-DCMAKE_BUILD_TYPE=Release",
          f"-DCMAKE_HIP_ARCHITECTURES={ARCH}"])
    _run([cmake, "--build", CMAKE_BUILD, "-j", jobs])
    _run([cmake, "--install", CMAKE_BUILD])
    _run([cmake, "-S", CONSUMER_SRC, "-B", CONSUMER_BUILD, f"-DCMAKE_PREFIX_PATH={INSTALL}",
          "-DCMAKE_BUILD_TYPE=Release"])
    _run([cmake, "--build", CONSUMER_BUILD, "-j", jobs])
    if verbose:
        print(f"installed the CMake package under {INSTALL}; built {CONSUMER_BIN}")
    return INSTALL


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs,
           "-Wl,-soname,libbitsqz_llm_lib.so.0"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    try:
        build()
        if "--package" in sys.argv:
            package()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
