"""The host-side sanitizer leg (CPU only): the oracle, the C ABI's host code
and the N-API addon rebuilt with AddressSanitizer and
UndefinedBehaviorSanitizer (clang's shared runtime, preloaded), then driven
by the CPU tests that exercise them: the oracle's pins, the C ABI's
descriptor contracts, plans and object lifetimes without a device, and the
Node host's record and descriptor checks. Any sanitizer report aborts the
child process and fails the test. The device code is the regular build's;
nothing here runs on a GPU."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "parakeet.wgsl_amd"))
import build  # noqa: E402  (the package's build script)

SAN_ENV = {
    "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:detect_odr_violation=0",
    "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
}


def sanitized_env():
    env = dict(os.environ)
    env.update(SAN_ENV)
    env["LD_PRELOAD"] = build.sanitizer_runtime()
    env["PYTHONDONTWRITEBYTECODE"] = "1"
    return env


def run_child(args, env, timeout=600):
    proc = subprocess.run(args, cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=timeout)
    tail = "\n".join(proc.stdout.splitlines()[-40:])
    assert proc.returncode == 0, f"exit {proc.returncode}\n{tail}"
    assert "ERROR: AddressSanitizer" not in proc.stdout and "runtime error:" not in proc.stdout, tail
    return proc.stdout


def pytest_child(module_attr, library, test_file, *extra):
    """Runs pytest on `test_file` in a child whose module `module_attr`
    (module:attribute) loads `library` instead of the regular build."""
    module, attr = module_attr.split(":")
    code = (f"import sys; sys.path.insert(0, {ROOT!r}); import {module} as m; m.{attr} = {library!r}; "
            f"import pytest; sys.exit(pytest.main([{test_file!r}, '-q', '-x', '-p', 'no:cacheprovider', "
            f"'-m', 'not gpu', *{list(extra)!r}]))")
    return run_child([sys.executable, "-c", code], sanitized_env())


def test_oracle_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "_san/liboracle.so"], check=True)
    out = pytest_child("oracle.pko:LIB_PATH", os.path.join(ROOT, "oracle", "_san", "liboracle.so"),
                       os.path.join(ROOT, "tests", "test_oracle.py"))
    assert " passed" in out


def test_c_abi_host_code_under_asan_and_ubsan():
    lib = build.build_sanitized()
    # every test of the contract file except the one that checks the regular
    # build's link line (the sanitized build also links the sanitizer runtime)
    out = pytest_child("parakeet_wgsl_amd.palette_abi:LIB_PATH", lib, os.path.join(ROOT, "tests", "test_abi_cpu.py"),
                       "-k", "not links_only_the_hip_runtime")
    assert " passed" in out


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_addon_under_asan_and_ubsan():
    build.build_sanitized()
    addon = os.path.join(build.SAN, "pk_napi.node")
    if not os.path.exists(addon):
        pytest.skip("Node headers are not installed")
    env = sanitized_env()
    env["PK_NAPI_ADDON"] = addon
    out = run_child(["node", os.path.join(ROOT, "tests", "node", "host_cpu.js")], env)
    assert "host_cpu ok" in out
