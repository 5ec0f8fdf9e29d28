"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C oracle asan` builds oracle/asan_check.c with fms_oracle.c (sanitizer
runtimes linked statically) into oracle/_asan/fms_oracle_check, which calls
every oracle entry point on exactly sized heap buffers with the edge cases the
reference's tests use (empty documents, fully masked rows, junk tape entries,
indices outside 1..N).  Any out-of-bounds access, leak or undefined behaviour
ends the run with a non-zero status.
"""
import os
import shutil
import subprocess

import pytest

ORACLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")


@pytest.mark.skipif(shutil.which("make") is None or shutil.which("gcc") is None,
                    reason="needs make and gcc")
def test_oracle_clean_under_asan_and_ubsan():
    b = subprocess.run(["make", "-s", "-C", ORACLE, "asan"], capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="2")
    r = subprocess.run([os.path.join(ORACLE, "_asan", "fms_oracle_check")], capture_output=True,
                       text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "oracle asan check ok" in r.stdout
