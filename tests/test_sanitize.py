"""Host sanitizer run of the library's encoder and the C oracle: tests/sanitize builds encode.cpp and nwc_oracle.c
with AddressSanitizer + UndefinedBehaviorSanitizer (g++/gcc, host code only) into one program that encodes the
encoder tests' matrices (BF16 and fp8, layouts 0/1/2, ragged and multithreaded sizes) with both encoders, compares
every output byte and decode table, and decodes the streams back to the inputs.  Any sanitizer report fails the run.
CPU only."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


@pytest.mark.timeout(600)
def test_encoder_and_oracle_under_asan_ubsan():
    if shutil.which("g++") is None or shutil.which("make") is None:
        pytest.skip("g++ / make not available")
    b = subprocess.run(["make", "-C", HERE, "-s", "-j4"], capture_output=True, text=True)
    if b.returncode and "asan" in (b.stdout + b.stderr).lower() and "cannot find" in (b.stdout + b.stderr):
        pytest.skip("sanitizer runtime libraries not installed")
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([os.path.join(HERE, "_build", "encode_selftest")], capture_output=True, text=True, env=env,
                       timeout=540)
    report = r.stdout + r.stderr
    assert r.returncode == 0, report[-4000:]
    assert "ERROR: AddressSanitizer" not in report and "runtime error" not in report, report[-4000:]
    assert "cases ok" in r.stdout
