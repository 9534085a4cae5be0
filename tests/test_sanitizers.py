"""AddressSanitizer + UndefinedBehaviorSanitizer over the host code, on the CPU.

The library's host code (argument validation, weight packing, the PRICHS02
reader that parses files from outside, the GEMM workspace), the CPU oracle
and the C++ host mirror are rebuilt with clang's -fsanitize=address,undefined
(prichs_amd/build.py build_sanitized, oracle/Makefile asan) and the CPU tests
of those parts run against them in a fresh process with the clang ASan runtime
preloaded: any heap/stack overflow, use-after-free or undefined behaviour
aborts the run.  Device code is not instrumented (GPU sanitizers are not
available on the GPU pool).
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def sanitized():
    from prichs_amd import build

    build.build_sanitized()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    oracle_lib = os.path.join(ROOT, "oracle", "_asan", "liboracle.so")
    env = dict(os.environ)
    env.update({
        "PRICHS_HIP_LIB": build.ASAN_LIB,
        "ORACLE_LIB": oracle_lib,
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    return build, env


def _check(r):
    out = r.stdout + r.stderr
    print(out[-4000:], flush=True)
    assert "ERROR: AddressSanitizer" not in out
    assert "runtime error:" not in out
    assert r.returncode == 0


def test_host_code_under_asan_ubsan(sanitized):
    build, env = sanitized
    env = dict(env, LD_PRELOAD=build.asan_runtime())
    # The sanitized builds are the ones loaded.
    probe = ("import prichs_amd._lib as L, oracle.oracle as O; L.load(); O.lib(); "
             "maps = open('/proc/self/maps').read(); "
             "assert '_build_asan/libprichs_hip.so' in maps and '_asan/liboracle.so' in maps")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    _check(r)
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu",
                        "-p", "no:cacheprovider", "tests/test_abi.py", "tests/test_checkpoint.py",
                        "tests/test_oracle.py", "tests/test_oracle_backward.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    _check(r)


def test_cpp_host_mirror_under_asan_ubsan(sanitized):
    # The executable carries clang's ASan runtime itself (no preload): the
    # checkpoint loader on a file written byte by byte, and the no-device
    # error paths of the engine and the GEMM workspace.
    build, env = sanitized
    r = subprocess.run([build.ASAN_HOST_TEST_BIN, "--no-gpu"], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=300)
    _check(r)
