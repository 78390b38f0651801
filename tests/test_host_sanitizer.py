"""The library's host side (argument checks, launch plans, workspace sizing,
error reporting) under AddressSanitizer and UndefinedBehaviorSanitizer on
the CPU: the C-ABI tests of test_abi.py run in a child process against a
build with host-side ASan + UBSan (device code as usual), with the ASan
runtime preloaded and every report fatal. No GPU is used: those tests stop
at argument checking or at host-only entry points."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.timeout(600)
def test_abi_checks_under_host_sanitizers():
    from zenith_amd import _build

    lib = _build.build_host_sanitized()
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": _build.host_asan_runtime(),
        "ZENITH_HIP_LIB": lib,
        # the interpreter itself is not instrumented and keeps its arenas
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
         os.path.join(ROOT, "tests", "test_abi.py")],
        cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
        timeout=540)
    out = proc.stdout
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert proc.returncode == 0, out[-4000:]
    assert " passed" in out, out[-4000:]
