"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer
(tests/sanitize/Makefile, built by build()): the CPU oracle on random and
adversarial inputs, and the C ABI library whose host code is sanitized
(its device code is built as usual) driven through every entry point.  A
run passes when the driver exits 0, which it does only with no sanitizer
report and every check held."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")
BUILD = os.path.join(HERE, "_build")


def _run(binary, timeout):
    path = os.path.join(BUILD, binary)
    if not os.path.exists(path):
        pytest.skip(f"{binary} is not built (build() builds it)")
    env = dict(os.environ)
    # the HIP runtime keeps allocations until the process ends: leaks are not checked
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    print(f"[sanitize] {binary}", flush=True)
    out = subprocess.run([path], capture_output=True, text=True, timeout=timeout, env=env)
    assert out.returncode == 0, (out.stdout[-2000:], out.stderr[-4000:])
    assert "AddressSanitizer" not in out.stderr and "runtime error" not in out.stderr
    return out.stdout


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is missing")
def test_oracle_under_sanitizers():
    if not os.path.exists(os.path.join(BUILD, "oracle_check")):
        subprocess.run(["make", "-s", "-C", HERE, "_build/oracle_check"], check=True)
    assert "ok" in _run("oracle_check", 300)


def test_c_abi_host_checks_under_sanitizers_without_gpu():
    from hachiue_amd import hip
    if hip.device_count() > 0:
        pytest.skip("a GPU is visible: the GPU test runs the full driver")
    assert "host-side checks only, 0 failed" in _run("capi_check", 300)


@pytest.mark.gpu
def test_c_abi_under_sanitizers_on_the_gpu():
    assert "C ABI sanitizer run: ok" in _run("capi_check", 600)
