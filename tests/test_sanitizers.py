"""The CPU-side code under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C oracle asan` builds the oracle and the library's host code (the
argument checks, plans and launch set-up of fmha_decode_api.hip, linked with
the kernel parts of the last library build) with both sanitizers.  These
tests run the oracle's own tests, the CPU ABI tests and the paged-guard
tests against those builds in a child process with the matching runtime
preloaded (g++'s libasan for the oracle, clang's for the library, which
hipcc builds); any report fails the run.  This is the class of bug the
reference's int-sized buffers have (fmha_host.cpp:85-93, :132).
"""
import os
import subprocess
import sys

import pytest

from tests.conftest import ROOT

ORACLE = os.path.join(ROOT, "oracle")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


INST_DIR = os.path.join(ROOT, "fmha_amd", "_build")


@pytest.fixture(scope="module")
def asan_builds():
    """The sanitized oracle, and the sanitized library where the kernel parts
    of a library build (fmha_amd/_build) are there to link with (else None:
    the library test is skipped)."""
    subprocess.run(["make", "-C", ORACLE, "-s", "asan-oracle"], check=True, capture_output=True)
    lib = None
    if os.path.isdir(INST_DIR) and any(n.startswith("fmha_decode_inst_") for n in os.listdir(INST_DIR)):
        subprocess.run(["make", "-C", ORACLE, "-s", "asan"], check=True, capture_output=True)
        lib = os.path.join(ORACLE, "_asan", "libfmha_decode.so")
    return os.path.join(ORACLE, "_asan", "liboracle.so"), lib


def _runtime(cmd):
    return subprocess.run(cmd, check=True, capture_output=True, text=True).stdout.strip()


def _pytest(args, preload, extra_env):
    env = dict(ENV, LD_PRELOAD=preload, **extra_env)
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu"]
                         + args, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    return out


def test_oracle_under_sanitizers(asan_builds):
    lib, _ = asan_builds
    preload = _runtime(["g++", "-print-file-name=libasan.so"])
    out = _pytest(["tests/test_oracle.py"], preload, {"FMHA_ORACLE_LIB": lib})
    assert " passed" in out


def test_library_host_code_under_sanitizers(asan_builds):
    _, lib = asan_builds
    if lib is None:
        pytest.skip("no kernel parts in fmha_amd/_build to link the sanitized library with")
    rt = _runtime(["/opt/rocm/llvm/bin/clang", "-print-file-name=libclang_rt.asan-x86_64.so"])
    if not os.path.isabs(rt) or not os.path.exists(rt):
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    out = _pytest(["tests/test_abi.py", "tests/test_paged_guard.py"], rt, {"FMHA_DECODE_LIB": lib})
    assert " passed" in out


def test_sanitizer_is_live(asan_builds):
    """A read past the end of K through the sanitized oracle (lengths that
    claim more rows than the array holds) is reported, so the runs above
    would have caught one."""
    lib, _ = asan_builds
    code = ("import numpy as np, oracle\n"
            "q = np.zeros((1, 1, 64), np.uint16); k = np.zeros((2, 1, 64), np.uint16)\n"
            "oracle.decode(q, k, k, np.array([0, 9], np.int32), 1, 1, 64, 0.125)\n")
    env = dict(ENV, LD_PRELOAD=_runtime(["g++", "-print-file-name=libasan.so"]), FMHA_ORACLE_LIB=lib)
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert res.returncode != 0 and "AddressSanitizer" in res.stderr, res.stderr[-2000:]
