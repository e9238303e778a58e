"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer:
the library is rebuilt with the host side instrumented (tests/host_sanitized.py;
device code unchanged) and tests/abi_checks.py -- the exports, every size query
and every argument check that test_abi.py runs -- is run against it in a
separate process that preloads the sanitizer runtime and never loads torch
or launches a kernel.  Any sanitizer report fails the test."""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import importlib.util, sys
def load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod
root, lib_path = sys.argv[1], sys.argv[2]
assert "libclang_rt.asan" in open("/proc/self/maps").read(), "sanitizer runtime not loaded"
abi = load("sophia_abi", root + "/sophia_amd/_abi.py")
checks = load("abi_checks", root + "/tests/abi_checks.py")
lib = abi.bind(lib_path)
class Nat:
    SOPHIA_OK = abi.SOPHIA_OK
    SOPHIA_ERR_INVALID = abi.SOPHIA_ERR_INVALID
    SOPHIA_ERR_WORKSPACE = abi.SOPHIA_ERR_WORKSPACE
    @staticmethod
    def last_error():
        msg = lib.sophia_last_error()
        return msg.decode() if msg else ""
checks.check_exports(lib_path, abi.SIGNATURES)
checks.check_host_side(lib, Nat)
print("SANITIZED_ABI_OK", flush=True)
"""


@pytest.fixture(scope="module")
def sanitized_lib(tmp_path_factory):
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    import host_sanitized
    out = str(tmp_path_factory.mktemp("host_sanitized"))
    return host_sanitized.build_host_sanitized(out), host_sanitized.sanitizer_runtime()


def test_abi_checks_under_asan_and_ubsan(sanitized_lib):
    lib_path, runtime = sanitized_lib
    env = dict(os.environ, LD_PRELOAD=runtime, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([sys.executable, "-c", SCRIPT, ROOT, lib_path], capture_output=True, text=True,
                         env=env, timeout=300)
    report = res.stdout[-3000:] + res.stderr[-3000:]
    assert res.returncode == 0, report
    assert "SANITIZED_ABI_OK" in res.stdout, report
    assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, report
