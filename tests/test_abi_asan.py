"""The C-ABI validation tests (tests/test_abi.py) against a build of the
library whose host code runs under AddressSanitizer: every argument check
of every entry point is exercised with ASan watching the host code's memory
accesses (the descriptor reads, the error-text formatting, the geometry
arithmetic).  CPU only: no entry point reaches a kernel launch."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc (ROCm) needed to build the sanitized library")
def test_abi_checks_under_host_address_sanitizer():
    sys.path.insert(0, ROOT)
    from terra_amd import build

    lib = build.build_library(asan_host=True)
    syms = subprocess.run(["nm", "-D", lib], stdout=subprocess.PIPE, text=True).stdout
    assert "__asan_report" in syms, "the sanitized build carries no ASan instrumentation"
    env = dict(os.environ, LD_PRELOAD=build.asan_runtime(), TERRA_SWIN_LIB=lib,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=66")
    check = ("import ctypes, terra_amd._lib as L; "
             f"assert L.LIB_PATH == {lib!r}; L.load(); ctypes.CDLL(None).__asan_init; print('asan-loaded')")
    pre = subprocess.run([sys.executable, "-c", check], cwd=ROOT, env=env, stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True, timeout=300)
    assert pre.returncode == 0 and "asan-loaded" in pre.stdout, pre.stdout[-2000:]
    run = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                          os.path.join(ROOT, "tests", "test_abi.py")], cwd=ROOT, env=env, stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True, timeout=600)
    assert run.returncode == 0, run.stdout[-4000:]
    assert "ERROR: AddressSanitizer" not in run.stdout
    assert " passed" in run.stdout
