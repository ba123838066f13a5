"""The CPU-side code under AddressSanitizer and UBSan: the oracle's C sources (GGUF load, the three
encoders, CTC, TDT and its trace, Whisper steps and window search) and the product's host-only Whisper
search, built by tests/sanitize/Makefile into one program (tests/sanitize/driver.cpp) and run on the
small synthetic models.  The sanitizers abort on their first report (leak checking on); the program
also compares the product's search with the oracle's on 400 seeded cases."""

import os
import shutil
import subprocess

import pytest

from wavo_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(ROOT, "build", "sanitize")


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None, reason="needs gcc and g++")
def test_oracle_and_host_search_under_sanitizers():
    subprocess.run(["make", "-s", "-j8", f"OUT={OUT}"], cwd=os.path.join(ROOT, "tests", "sanitize"), check=True)
    exe = os.path.join(OUT, "driver")
    libs = subprocess.run(["ldd", exe], capture_output=True, text=True, check=True).stdout
    assert "libasan" in libs and "libubsan" in libs
    models = [synth.model_path(n, small=True) for n in ("gigaam", "parakeet", "whisper")]
    env = dict(os.environ, OMP_NUM_THREADS="2", ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, *models, str(synth.SMALL["whisper"]["vocab"])], capture_output=True, text=True,
                       env=env, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "0 mismatches" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
