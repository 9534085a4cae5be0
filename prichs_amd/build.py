"""Builds libprichs_hip.so in-tree with hipcc for gfx950.

Every .hip file under csrc/ is compiled to an object in parallel, then linked
into prichs_amd/libprichs_hip.so.  No JIT cache and no site-packages install:
the library sits next to this file so it travels with the source tree.
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
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libprichs_hip.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libprichs_hip.so)")


COMMON_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall",
    # Keep hipcc from forming packed-FP32 instructions (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_host(verbose)
    return LIB


HOST = os.path.join(HERE, "host")
HOST_LIB = os.path.join(HERE, "libprichs_host.so")
HOST_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_gpu_model_engine.cpp")
HOST_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "test_gpu_model_engine")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _gxx(args, what):
    cxx = os.environ.get("CXX", "g++")
    r = subprocess.run([cxx, *args], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stderr}")


def build_host(verbose: bool = False) -> str:
    """The C++ host mirror of GpuModelEngine (libprichs_host.so, over the C ABI
    of libprichs_hip.so) and its C++ test program; plain host C++ with the HIP
    runtime, so g++ builds it.  rpaths are relative ($ORIGIN) so both travel
    with the tree."""
    flags = ["-std=c++17", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__",
             "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"), "-I", HOST]
    rocm_lib = ["-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    _gxx([*flags, "-fPIC", "-shared", os.path.join(HOST, "gpu_model_engine.cpp"), "-L", HERE,
          "-lprichs_hip", *rocm_lib, "-Wl,-rpath,$ORIGIN", "-o", HOST_LIB], "libprichs_host.so")
    _gxx([*flags, HOST_TEST_SRC, "-L", HERE, "-lprichs_host", "-lprichs_hip", *rocm_lib,
          "-Wl,-rpath,$ORIGIN/../../prichs_amd", "-o", HOST_TEST_BIN], "test_gpu_model_engine")
    if verbose:
        print(f"built {HOST_LIB} and {HOST_TEST_BIN}")
    return HOST_LIB


# ---- AddressSanitizer + UBSan build of the host code (CPU tests only) -----
# The library's host code (argument checks, packing, the checkpoint reader,
# the workspace) and the C++ host mirror are compiled with clang's
# -fsanitize=address,undefined into prichs_amd/_build_asan/; device code is
# unchanged.  tests/test_sanitizers.py runs the CPU tests against these
# builds with the clang ASan runtime preloaded.
ASAN_DIR = os.path.join(HERE, "_build_asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libprichs_hip.so")
ASAN_HOST_LIB = os.path.join(ASAN_DIR, "libprichs_host.so")
ASAN_HOST_TEST_BIN = os.path.join(ASAN_DIR, "test_gpu_model_engine")
LLVM = os.path.join(ROCM, "llvm", "bin")
# Each -fsanitize= follows -Xarch_host: host code only.
SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all"]


def asan_runtime() -> str:
    """The clang ASan runtime that the sanitized builds link against."""
    import glob

    hits = sorted(glob.glob(os.path.join(ROCM, "llvm", "lib", "clang", "*", "lib", "linux",
                                         "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise RuntimeError("libclang_rt.asan-x86_64.so not found under ROCm's LLVM")
    return hits[-1]


def _compile_asan(src: str) -> str:
    obj = os.path.join(ASAN_DIR, os.path.basename(src) + ".o")
    flags = [f if f != "-O3" else "-O1" for f in COMMON_FLAGS]
    cmd = [hipcc(), *flags, "-g", *SAN_HOST, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc (sanitized) failed for {src}:\n{r.stderr}")
    return obj


def build_sanitized(verbose: bool = False) -> str:
    os.makedirs(ASAN_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile_asan, srcs))
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *SAN_HOST, *objs, "-o", ASAN_LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{r.stderr}")
    cxx = os.path.join(LLVM, "clang++")
    san = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=all",
           "-g", "-O1"]
    flags = ["-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
             "-I", os.path.join(ROOT, "include"), "-I", HOST]
    rocm_lib = ["-L", os.path.join(ROCM, "lib"), "-lamdhip64",
                f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    for args, what in (
        ([*flags, *san, "-fPIC", "-shared", os.path.join(HOST, "gpu_model_engine.cpp"), "-L",
          ASAN_DIR, "-lprichs_hip", *rocm_lib, "-Wl,-rpath,$ORIGIN", "-o", ASAN_HOST_LIB],
         "sanitized libprichs_host.so"),
        ([*flags, *san, HOST_TEST_SRC, "-L", ASAN_DIR, "-lprichs_host", "-lprichs_hip", *rocm_lib,
          "-Wl,-rpath,$ORIGIN", "-o", ASAN_HOST_TEST_BIN], "sanitized test_gpu_model_engine")):
        r = subprocess.run([cxx, *args], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{what} failed:\n{r.stderr}")
    if verbose:
        print(f"built {ASAN_LIB}, {ASAN_HOST_LIB} and {ASAN_HOST_TEST_BIN}")
    return ASAN_LIB


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--sanitized":
        build_sanitized(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
