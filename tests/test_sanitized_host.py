"""The host-side ABI tests (tests/test_abi.py) against a build of the library
with AddressSanitizer and UndefinedBehaviorSanitizer on its host code
(einjax_amd/csrc/build.py --sanitize).  Any out-of-bounds access, use after
free or undefined behaviour on those paths ends the run with a report."""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def sanitized_lib():
    sys.path.insert(0, str(ROOT))
    from einjax_amd.csrc import build

    try:
        runtime = build.san_runtime()
    except RuntimeError as e:
        pytest.skip(str(e))
    return build.build_sanitized(verbose=False), runtime


def test_sanitized_library_is_instrumented(sanitized_lib):
    lib, _ = sanitized_lib
    syms = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True,
                          text=True, check=True).stdout
    assert "__asan_report_load" in syms and "__ubsan_handle_" in syms


def test_abi_tests_under_asan_and_ubsan(sanitized_lib):
    lib, runtime = sanitized_lib
    env = dict(os.environ)
    pre = env.get("LD_PRELOAD")
    env["LD_PRELOAD"] = f"{runtime}:{pre}" if pre else str(runtime)  # ASan must come first
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["EINJAX_AMD_SANITIZED_LIB"] = str(lib)
    env.pop("EJ_INJECT_FAULT", None)
    res = subprocess.run([sys.executable, "-m", "pytest", str(ROOT / "tests" / "test_abi.py"), "-q",
                          "-p", "no:cacheprovider", "-m", "not gpu"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "passed" in out and "ERROR: AddressSanitizer" not in out and "runtime error" not in out
