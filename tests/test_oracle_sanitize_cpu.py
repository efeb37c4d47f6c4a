"""The oracle under AddressSanitizer and UndefinedBehaviorSanitizer: `make -C
oracle sanitize` builds oracle/sanitize_check.c with tl_oracle.c and runs the
composed path (per-row and layer-major multi-row decode, LM head) on small
seeded models with hidden > intermediate and the reverse.  Any sanitizer
report, or a per-row / multi-row mismatch, fails it."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("make") is None, reason="needs gcc and make")
def test_oracle_clean_under_asan_ubsan():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:]
    assert r.stdout.count(": ok") == 2, r.stdout[-4000:]
