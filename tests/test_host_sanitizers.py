"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

The argument validation, size arithmetic and error strings of every entry
point run in a library built with sanitized host code
(`_build.build_host_sanitized`; the device code is the product's and is never
launched here). The ABI's own validation tests (tests/test_abi.py) run against
that library in a child process with the ASan runtime preloaded; any
out-of-bounds access, use after free or undefined behaviour aborts it."""

import os
import shutil
import subprocess
import sys

import pytest

from conftest import ROOT

from cab_attention import _build


@pytest.fixture(scope="module")
def sanitized_lib(tmp_path_factory):
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")
    try:
        rt = _build.asan_runtime()
    except RuntimeError as e:
        pytest.skip(str(e))
    return _build.build_host_sanitized(tmp_path_factory.mktemp("asan")), rt


def test_abi_validation_under_asan_and_ubsan(sanitized_lib):
    lib, rt = sanitized_lib
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": str(rt),
        "CAB_HIP_LIB": str(lib),
        # python and torch are not instrumented: only the library's own
        # accesses and the allocator calls are checked.
        "ASAN_OPTIONS": "detect_leaks=0:alloc_dealloc_mismatch=0:detect_odr_violation=0:abort_on_error=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    cmd = [sys.executable, "-m", "pytest", str(ROOT / "tests" / "test_abi.py"), "-q", "-p", "no:cacheprovider",
           "-k", "validation or exports"]
    res = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = res.stdout + res.stderr
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    assert res.returncode == 0, out[-6000:]
    assert " passed" in res.stdout and "failed" not in res.stdout, out[-3000:]
