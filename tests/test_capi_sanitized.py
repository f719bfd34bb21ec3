"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

``make -C dw-tpu_amd/csrc asan`` builds the library with instrumented host
code (device code plain).  The argument-check and launch-plan tests
(test_capi.py, test_dense_tiles.py) then run again in a child process that
loads that build (DWTPU_MOE_LIB) with the ASan runtime preloaded; any report
(out-of-bounds or use-after-free access, signed overflow, bad shift, ...)
stops the child with a failure.  CPU only: no entry point reaches a launch.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "dw-tpu_amd", "csrc")
ASAN_LIB = os.path.join(CSRC, "_build_asan", "libdwtpu_moe.so")
CLANG = "/opt/rocm/llvm/bin/clang++"


def _asan_runtime():
    if not os.path.exists(CLANG):
        return None
    r = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


@pytest.fixture(scope="module")
def asan_build():
    runtime = _asan_runtime()
    if runtime is None or shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("no hipcc / make / clang ASan runtime in this image")
    r = subprocess.run(["make", "-C", CSRC, "asan", "-j8"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return runtime


def test_asan_build_is_instrumented(asan_build):
    """The host code calls into the sanitizer runtimes (so it loads only with
    them preloaded): the build is the instrumented one."""
    r = subprocess.run(["nm", "-D", "--undefined-only", ASAN_LIB], capture_output=True, text=True)
    assert r.returncode == 0
    assert "__asan_report_load8" in r.stdout
    assert "__ubsan_handle_" in r.stdout


def test_argument_checks_under_sanitizers(asan_build):
    env = dict(os.environ)
    env.update(DWTPU_MOE_LIB=ASAN_LIB, LD_PRELOAD=asan_build,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    # The header test links a C program against the library: not meaningful
    # for the instrumented build, whose runtime comes from the preload.
    cmd = [sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
           "-k", "not header_is_plain_c",
           os.path.join(ROOT, "tests", "test_capi.py"), os.path.join(ROOT, "tests", "test_dense_tiles.py")]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out and " failed" not in out, out[-2000:]
