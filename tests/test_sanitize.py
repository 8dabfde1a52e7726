"""AddressSanitizer / UndefinedBehaviorSanitizer runs of the host code on the
CPU: the host shim (MLL reader over the shipped package and over truncated,
bit-flipped and resealed corrupt packages; the plan classifiers; BLAKE3;
byte accounting) and the C oracle, each built with -fsanitize=address,undefined
(eos_amd.build.build_sanitized, `make -C oracle sanitize`) and driven by
tests/sanitize_child.py in a child process that preloads the sanitizer
runtimes. No GPU call is made; a sanitizer report fails the test."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _runtime(name: str) -> str:
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip(f"{name} not available")
    return path


def test_host_code_under_asan_and_ubsan():
    from eos_amd import build
    lib = build.build_sanitized()
    subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "sanitize"], check=True)
    olib = os.path.join(REPO, "oracle", "liboracle_asan.so")
    env = dict(os.environ)
    env["LD_PRELOAD"] = ":".join([_runtime("libasan.so"), _runtime("libubsan.so")])
    # Python itself is not instrumented and keeps memory until exit.
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    proc = subprocess.run([sys.executable, os.path.join(REPO, "tests", "sanitize_child.py"), lib, olib],
                          capture_output=True, text=True, env=env, timeout=600)
    report = proc.stderr[-4000:]
    assert "AddressSanitizer" not in proc.stderr, report
    assert "runtime error" not in proc.stderr, report
    assert proc.returncode == 0, report
    assert proc.stdout.strip().endswith("OK"), proc.stdout[-2000:] + report
