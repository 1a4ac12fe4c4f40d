"""Sanitizer runs on the CPU (memory and undefined-behaviour checking of the host side; GPU
sanitizer builds are not used): the oracle built with AddressSanitizer + UBSan and driven
through its entry points (tests/sanitize/oracle_run.py), and the library's host code built
likewise and driven through the C ABI's device-free validation paths
(tests/sanitize/host_driver.cpp).  Each must finish with no sanitizer report."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")


def _make(target):
    subprocess.run(["make", "-s", "-j8", "-C", SAN, target], check=True, capture_output=True, text=True, timeout=900)


def _clean_env(**extra):
    env = dict(os.environ)
    env.update(ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               **extra)
    return env


def test_oracle_under_asan_and_ubsan():
    _make("oracle")
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                             check=True).stdout.strip()
    env = _clean_env(LD_PRELOAD=libasan, IRODORI_ORACLE_LIB=os.path.join(SAN, "_build", "liboracle_asan.so"),
                     OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, os.path.join(SAN, "oracle_run.py")], env=env, capture_output=True,
                       text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    assert r.stdout.strip().endswith("ok")


@pytest.mark.skipif(not shutil.which("/opt/rocm/bin/hipcc"), reason="hipcc not installed")
def test_host_code_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "irodori-tts-burn_amd")], check=True,
                   capture_output=True, text=True, timeout=900)
    _make("host")
    r = subprocess.run([os.path.join(SAN, "_build", "host_driver")], env=_clean_env(), capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    assert r.stdout.strip().endswith("ok (0 failures)")
